// Page requantisation kernels for gfx950: a batch of FP16 pages quantised to
// INT8/INT4/INT2 in one launch, and the dequantiser.
//
// Arithmetic follows the reference exactly (src/core_kernels/quant.cu):
//   - keys per (head, channel) over the page's P positions, values per
//     (token, head) over head_dim (quant.cu:76-187);
//   - zero-point = the group's minimum, stored exactly in fp16;
//   - scale = scale_bits_of (fp64 range / levels, nearest fp16, one ulp up
//     if short: quant.cu:44-56);
//   - code = rintf((x - zero) / scale) in fp32 IEEE arithmetic, clamped,
//     0 for a zero scale (quant.cu:60-70);
//   - dequantised value = fp16_rn(fmaf(code, scale, zero)) (quant.cu:243-266).
//
// Layout of the work (MI355X-first, not the reference's two launches per
// batch): one workgroup quantises one whole page. It streams the FP16 page
// (possibly pinned host memory mapped for the device) into LDS once with
// 16-byte loads, computes every group there, assembles the quantised page in
// LDS, and writes it out with 16-byte stores. Every input byte crosses HBM or
// the host link once and every output byte once.

#include "common.hpp"
#include "kernels.hpp"
#include "quant_core.hpp"

namespace mi
{
  namespace
  {

    constexpr int kQuantThreads = 256;
    using quant_core::block_copy;
    using quant_core::quantise_in_lds;

    // One workgroup per page: page blockIdx.x + first of the batch.
    template <int Bits>
    __global__ void __launch_bounds__(kQuantThreads)
        quantise_pages_kernel(const void *const *__restrict__ rows,
                              void *const *__restrict__ pages, const void *row0, void *page0,
                              std::ptrdiff_t values_offset, PageLayout L, int page_tokens,
                              int kv_heads, int head_dim)
    {
      extern __shared__ uint4 lds_raw[];
      const std::size_t half_bytes =
          static_cast<std::size_t>(page_tokens) * kv_heads * head_dim * 2;
      const std::size_t in_bytes = 2 * half_bytes;
      std::uint16_t *in = reinterpret_cast<std::uint16_t *>(lds_raw);
      std::uint8_t *out = reinterpret_cast<std::uint8_t *>(lds_raw) + ((in_bytes + 15) / 16) * 16;
      // A batch names its pages in tables; a single page comes by value.
      const auto *src = static_cast<const std::uint8_t *>(rows ? rows[blockIdx.x] : row0);
      auto *dst = static_cast<std::uint8_t *>(pages ? pages[blockIdx.x] : page0);
      block_copy(reinterpret_cast<std::uint8_t *>(in), src, half_bytes);
      block_copy(reinterpret_cast<std::uint8_t *>(in) + half_bytes, src + values_offset,
                 half_bytes);
      __syncthreads();
      quantise_in_lds<Bits>(in, out, L, page_tokens, kv_heads, head_dim);
      __syncthreads();
      block_copy(dst, out, L.page_bytes);
    }

    // One half of a quantised page back to fp16, a thread per code byte.
    // Element e of the half is row e / width; its group is its channel,
    // e % width, for keys, and its (token, head), e / head_dim, for values.
    template <int Bits, bool PerChannel>
    __global__ void dequantise_kernel(const std::uint8_t *__restrict__ codes,
                                      const std::uint16_t *__restrict__ scales,
                                      const std::uint16_t *__restrict__ zeros,
                                      std::uint16_t *__restrict__ out, std::size_t bytes,
                                      int width, int head_dim)
    {
      constexpr int kPerByte = 8 / Bits;
      constexpr unsigned kMask = (1u << Bits) - 1;
      for (std::size_t i = static_cast<std::size_t>(blockIdx.x) * blockDim.x + threadIdx.x;
           i < bytes; i += static_cast<std::size_t>(gridDim.x) * blockDim.x)
      {
        const unsigned byte = codes[i];
#pragma unroll
        for (int c = 0; c < kPerByte; ++c)
        {
          const std::size_t e = i * kPerByte + c;
          const std::size_t group = PerChannel ? e % width : e / head_dim;
          const float q = static_cast<float>((byte >> (c * Bits)) & kMask);
          const float v = fmaf(q, half_bits_to_float(scales[group]),
                               half_bits_to_float(zeros[group]));
          out[e] = __half_as_ushort(__float2half_rn(v));
        }
      }
    }

    template <typename F>
    void with_bits(int tier, F &&f)
    {
      switch (tier)
      {
      case kINT8: f(std::integral_constant<int, 8>{}); return;
      case kINT4: f(std::integral_constant<int, 4>{}); return;
      case kINT2: f(std::integral_constant<int, 2>{}); return;
      }
      throw InvalidArgument("FP16 is not a quantised tier: its page has no codes and no metadata");
    }

    std::size_t quant_lds_bytes(const PageLayout &L, int page_tokens, int kv_heads, int head_dim)
    {
      const std::size_t in = fp16_page_bytes(page_tokens, static_cast<std::size_t>(kv_heads) * head_dim);
      return ((in + 15) / 16) * 16 + ((L.page_bytes + 15) / 16) * 16;
    }

    // LDS a workgroup may take on gfx950.
    constexpr std::size_t kMaxLds = 160 * 1024;

  } // namespace

  void launch_quantise_pages(const void *const *rows, void *const *pages, const void *row0,
                             void *page0, std::ptrdiff_t values_offset, int count, int tier,
                             int page_tokens, int kv_heads, int head_dim, hipStream_t stream)
  {
    const PageLayout L = page_layout(tier, page_tokens, kv_heads, head_dim);
    if (count <= 0)
    {
      return;
    }
    // 32-token pages at head_dim 64 or 128 (16-byte aligned rows): the
    // register quantiser, a lane a task, every page of the batch at once.
    if (launch_quantise_registers(rows, pages, row0, page0, values_offset, count, tier,
                                  page_tokens, kv_heads, head_dim, stream))
    {
      return;
    }
    const std::size_t lds = quant_lds_bytes(L, page_tokens, kv_heads, head_dim);
    if (lds > kMaxLds)
    {
      throw InvalidArgument("a page of " + std::to_string(page_tokens) + " positions at " +
                            std::to_string(kv_heads * head_dim) +
                            " elements does not fit one workgroup's LDS to quantise");
    }
    with_bits(tier, [&](auto bits) {
      constexpr int B = decltype(bits)::value;
      auto kernel = quantise_pages_kernel<B>;
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute quantise LDS");
      }
      // A grid's x dimension holds far more than any batch of pages.
      hipLaunchKernelGGL(kernel, dim3(count), dim3(kQuantThreads), lds, stream, rows, pages, row0,
                         page0, values_offset, L, page_tokens, kv_heads, head_dim);
      hip_check(hipGetLastError(), "quantise pages kernel launch");
    });
  }

  void launch_dequantise_page(const void *page, void *keys, void *values, int tier,
                              int page_tokens, int kv_heads, int head_dim, hipStream_t stream)
  {
    const PageLayout L = page_layout(tier, page_tokens, kv_heads, head_dim);
    const std::size_t bytes = L.value_codes - L.key_codes;
    const int width = kv_heads * head_dim;
    const auto *p = static_cast<const std::uint8_t *>(page);
    const auto meta = [p](std::size_t off) { return reinterpret_cast<const std::uint16_t *>(p + off); };
    const int threads = 256;
    const int blocks = static_cast<int>(std::min<std::size_t>((bytes + threads - 1) / threads, 4096));
    with_bits(tier, [&](auto bits) {
      constexpr int B = decltype(bits)::value;
      hipLaunchKernelGGL((dequantise_kernel<B, true>), dim3(blocks), dim3(threads), 0, stream,
                         p + L.key_codes, meta(L.key_scales), meta(L.key_zeros),
                         static_cast<std::uint16_t *>(keys), bytes, width, head_dim);
      hip_check(hipGetLastError(), "dequantise keys kernel launch");
      hipLaunchKernelGGL((dequantise_kernel<B, false>), dim3(blocks), dim3(threads), 0, stream,
                         p + L.value_codes, meta(L.value_scales), meta(L.value_zeros),
                         static_cast<std::uint16_t *>(values), bytes, width, head_dim);
      hip_check(hipGetLastError(), "dequantise values kernel launch");
    });
  }

} // namespace mi
