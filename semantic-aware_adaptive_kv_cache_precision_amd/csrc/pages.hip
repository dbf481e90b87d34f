// Byte-moving kernels of the cache: batched page copies (shadows out,
// restores in, tail compaction), the decode row store, and the importance
// scores' fill and fold.
//
// These are HBM- or host-link-bound integer/byte work: each is laid out for
// coalesced 16-byte accesses and enough workgroups to fill 256 CUs, with no
// attempt to route them through matrix cores.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>

namespace mi
{
  namespace
  {

    // The bytes a workgroup of the page copy moves: 256 threads, four
    // 16-byte units each.
    constexpr std::size_t kCopyChunk = 256 * 4 * 16;

    // A batch of page copies (from[p] to to[p], `units` of Unit each):
    // workgroup x copies chunk x % chunks of page first + x / chunks, a Unit
    // a thread a pass over the chunk.
    template <typename Unit>
    __global__ void __launch_bounds__(256)
        copy_pages_kernel(const void *const *__restrict__ from, void *const *__restrict__ to,
                          std::size_t units, std::size_t chunks, int first)
    {
      constexpr std::size_t kChunkUnits = kCopyChunk / sizeof(Unit);
      const std::size_t page = first + blockIdx.x / chunks;
      const std::size_t begin = (blockIdx.x % chunks) * kChunkUnits;
      const std::size_t end = begin + kChunkUnits < units ? begin + kChunkUnits : units;
      const Unit *src = static_cast<const Unit *>(from[page]);
      Unit *dst = static_cast<Unit *>(to[page]);
      for (std::size_t i = begin + threadIdx.x; i < end; i += 256)
      {
        dst[i] = src[i];
      }
    }

    // Rows start .. start + n of one layer into its FP16 pages (pages: the
    // layer's page addresses; a page holds page_tokens key rows, then as many
    // value rows): workgroup y takes row y, its threads the row's channels.
    __global__ void store_pages_kernel(const std::uint16_t *__restrict__ keys,
                                       const std::uint16_t *__restrict__ values,
                                       const unsigned long long *__restrict__ pages,
                                       int page_tokens, int width, int start)
    {
      const int position = start + static_cast<int>(blockIdx.y);
      auto *page = reinterpret_cast<std::uint16_t *>(pages[position / page_tokens]);
      std::uint16_t *k_row = page + static_cast<std::size_t>(position % page_tokens) * width;
      std::uint16_t *v_row = k_row + static_cast<std::size_t>(page_tokens) * width;
      const std::size_t from = static_cast<std::size_t>(blockIdx.y) * width;
      for (int c = blockIdx.x * blockDim.x + threadIdx.x; c < width; c += gridDim.x * blockDim.x)
      {
        k_row[c] = keys[from + c];
        v_row[c] = values[from + c];
      }
    }

    __global__ void fill_kernel(float *out, std::size_t count, float value)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        out[i] = value;
      }
    }

    // The fold of one layer's page masses (heads rows of `pages`) into its
    // scores: a thread a page, the heads' masses added in head order, their
    // mean, then ewma_step. The library is built with -ffp-contract=off, so
    // nothing here fuses.
    __global__ void fold_kernel(float *__restrict__ scores, const float *__restrict__ mass,
                                int heads, int pages, float alpha)
    {
      const int page = blockIdx.x * blockDim.x + threadIdx.x;
      if (page >= pages)
      {
        return;
      }
      float total = 0.0f;
      const float *column = mass + page;
      for (int h = 0; h < heads; ++h, column += pages)
      {
        total = __fadd_rn(total, *column);
      }
      scores[page] = ewma_step(scores[page], __fdiv_rn(total, static_cast<float>(heads)), alpha);
    }

    int grid_for(std::size_t count, int threads, int cap = 65536)
    {
      return static_cast<int>(std::max<std::size_t>(
          1, std::min<std::size_t>((count + threads - 1) / threads, cap)));
    }

    // Pages a launch's y dimension holds.
    constexpr int kMaxGridY = 65535;

  } // namespace

  void launch_copy_pages(const void *const *from, void *const *to, std::size_t bytes, int count,
                         hipStream_t stream)
  {
    if (count <= 0 || bytes == 0)
    {
      return;
    }
    const auto go = [&](auto unit) {
      using Unit = decltype(unit);
      const std::size_t units = bytes / sizeof(Unit);
      const std::size_t chunks = (bytes + kCopyChunk - 1) / kCopyChunk;
      // A launch's x dimension holds 2^31 - 1 workgroups.
      const int per_launch = static_cast<int>(std::min<std::size_t>(
          count, std::max<std::size_t>(1, 0x7fffffffULL / chunks)));
      for (int first = 0; first < count; first += per_launch)
      {
        const int n = std::min(per_launch, count - first);
        hipLaunchKernelGGL(copy_pages_kernel<Unit>, dim3(static_cast<unsigned>(n * chunks)),
                           dim3(256), 0, stream, from, to, units, chunks, first);
        hip_check(hipGetLastError(), "copy pages kernel launch");
      }
    };
    // Pages sit at multiples of their size from granule-aligned bases, and
    // shadows at multiples of theirs in page-aligned host allocations.
    if (bytes % 16 == 0)
    {
      go(uint4{});
    }
    else
    {
      go(std::uint8_t{});
    }
  }

  void launch_store_pages(const void *keys, const void *values, const unsigned long long *pages,
                          int page_tokens, std::size_t row, int start, int n, hipStream_t stream)
  {
    if (n <= 0 || row == 0)
    {
      return;
    }
    const int threads = 256;
    const int blocks_x = static_cast<int>((row + threads - 1) / threads);
    for (int first = 0; first < n; first += kMaxGridY)
    {
      const int rows = std::min(kMaxGridY, n - first);
      hipLaunchKernelGGL(store_pages_kernel, dim3(blocks_x, rows), dim3(threads), 0, stream,
                         static_cast<const std::uint16_t *>(keys) + static_cast<std::size_t>(first) * row,
                         static_cast<const std::uint16_t *>(values) + static_cast<std::size_t>(first) * row,
                         pages, page_tokens, static_cast<int>(row), start + first);
    }
    hip_check(hipGetLastError(), "store pages kernel launch");
  }

  void launch_fill(float *out, std::size_t count, float value, hipStream_t stream)
  {
    if (count == 0)
    {
      return;
    }
    hipLaunchKernelGGL(fill_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream, out, count,
                       value);
    hip_check(hipGetLastError(), "fill kernel launch");
  }

  void launch_fold(float *scores, const float *mass, int heads, int pages, float alpha,
                   hipStream_t stream)
  {
    if (pages <= 0)
    {
      return;
    }
    hipLaunchKernelGGL(fold_kernel, dim3((pages + 255) / 256), dim3(256), 0, stream, scores, mass,
                       heads, pages, alpha);
    hip_check(hipGetLastError(), "fold kernel launch");
  }

} // namespace mi
