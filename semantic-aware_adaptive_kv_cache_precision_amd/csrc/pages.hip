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

    // Copy page blockIdx.y: `units` of Unit from from[y] to to[y], the
    // blocks of x striding over them (reference: page_copy.cu:25-37).
    template <typename Unit>
    __global__ void copy_pages_kernel(const void *const *__restrict__ from,
                                      void *const *__restrict__ to, std::size_t units, int first)
    {
      const auto *src = static_cast<const Unit *>(from[first + blockIdx.y]);
      auto *dst = static_cast<Unit *>(to[first + blockIdx.y]);
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < units; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        dst[i] = src[i];
      }
    }

    // One thread per fp16 element of the n rows: token i / row at position
    // start + i / row (reference: kv_pages.cu:26-43).
    __global__ void store_pages_kernel(const std::uint16_t *__restrict__ keys,
                                       const std::uint16_t *__restrict__ values,
                                       const unsigned long long *__restrict__ pages,
                                       int page_tokens, std::size_t row, int start,
                                       std::size_t count)
    {
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < count; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const int position = start + static_cast<int>(i / row);
        auto *page = reinterpret_cast<std::uint16_t *>(pages[position / page_tokens]);
        std::uint16_t *key = page + static_cast<std::size_t>(position % page_tokens) * row + i % row;
        key[0] = keys[i];
        key[static_cast<std::size_t>(page_tokens) * row] = values[i];
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

    // One thread per page (reference: importance_scores.cu:31-50). The
    // library is built with -ffp-contract=off, so nothing below fuses.
    __global__ void fold_kernel(float *__restrict__ scores, const float *__restrict__ mass,
                                int heads, int pages, float alpha)
    {
      for (int page = blockIdx.x * blockDim.x + threadIdx.x; page < pages;
           page += gridDim.x * blockDim.x)
      {
        float total = 0.0f;
        for (int h = 0; h < heads; ++h)
        {
          total = __fadd_rn(total, mass[static_cast<std::size_t>(h) * pages + page]);
        }
        const float observed = __fdiv_rn(total, static_cast<float>(heads));
        const float old = scores[page];
        scores[page] = isnan(old) ? observed
                                  : __fadd_rn(__fmul_rn(alpha, observed),
                                              __fmul_rn(__fsub_rn(1.0f, alpha), old));
      }
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
    const int threads = 256;
    const auto go = [&](auto unit) {
      using Unit = decltype(unit);
      const std::size_t units = bytes / sizeof(Unit);
      // A few workgroups a page: a page is tens of KiB, and a batch holds
      // thousands, so the grid fills the device either way.
      const int blocks = static_cast<int>(std::min<std::size_t>((units + threads - 1) / threads, 8));
      for (int first = 0; first < count; first += kMaxGridY)
      {
        const int n = std::min(kMaxGridY, count - first);
        hipLaunchKernelGGL(copy_pages_kernel<Unit>, dim3(blocks, n), dim3(threads), 0, stream,
                           from, to, units, first);
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
    const std::size_t count = static_cast<std::size_t>(n) * row;
    if (count == 0)
    {
      return;
    }
    hipLaunchKernelGGL(store_pages_kernel, dim3(grid_for(count, 256)), dim3(256), 0, stream,
                       static_cast<const std::uint16_t *>(keys),
                       static_cast<const std::uint16_t *>(values), pages, page_tokens, row, start,
                       count);
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
    hipLaunchKernelGGL(fold_kernel, dim3(grid_for(pages, 256)), dim3(256), 0, stream, scores, mass,
                       heads, pages, alpha);
    hip_check(hipGetLastError(), "fold kernel launch");
  }

} // namespace mi
