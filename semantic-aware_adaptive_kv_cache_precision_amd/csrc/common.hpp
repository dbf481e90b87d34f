// Shared definitions of the MI355X KV-cache library: tiers, the quantised
// page layout, error types, and the fp16 helpers the kernels share.
//
// Everything here is written for gfx950 (wave64, CDNA4) and the HIP runtime;
// host and device code both include it.
#pragma once

#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>

#include <cstddef>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace mi
{

  // The four precision tiers, highest first (reference: paged_kv_cache.h:16-25).
  enum Tier : int
  {
    kFP16 = 0,
    kINT8 = 1,
    kINT4 = 2,
    kINT2 = 3,
  };
  constexpr int kTierCount = 4;
  // A page-table tier entry no query reads: evicted or masked
  // (reference: device_ops.h:91-96).
  constexpr std::uint8_t kUnreadPage = 0xFF;

  inline const char *tier_name(int tier)
  {
    switch (tier)
    {
    case kFP16: return "FP16";
    case kINT8: return "INT8";
    case kINT4: return "INT4";
    case kINT2: return "INT2";
    }
    return "an unknown tier";
  }
  // A lower tier has fewer bits a value: a larger number.
  inline bool is_lower(int a, int b) { return a > b; }

  // ---- errors ---------------------------------------------------------------
  // Each maps to one status code of the C ABI and one Python exception class
  // of the shim (reference: bindings.cpp:546-554, check.h:18-57).
  struct InvalidArgument : std::runtime_error { using std::runtime_error::runtime_error; };
  struct OutOfRange : std::runtime_error { using std::runtime_error::runtime_error; };
  struct PageNotFound : std::runtime_error { using std::runtime_error::runtime_error; };
  struct OpenPageError : std::runtime_error { using std::runtime_error::runtime_error; };
  struct OutOfMemory : std::runtime_error { using std::runtime_error::runtime_error; };
  struct LogicError : std::runtime_error { using std::runtime_error::runtime_error; };
  struct Full : std::runtime_error { using std::runtime_error::runtime_error; };
  struct DeviceError : std::runtime_error { using std::runtime_error::runtime_error; };

  inline void hip_check(hipError_t e, const char *what)
  {
    if (e == hipSuccess)
    {
      return;
    }
    const std::string msg = std::string(what) + ": " + hipGetErrorString(e);
    if (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation)
    {
      (void)hipGetLastError(); // an allocation failure is not sticky
      throw OutOfMemory(msg);
    }
    throw DeviceError(msg);
  }

  // ---- the quantised page layout ----------------------------------------------
  // Regions back to back, W = kv_heads * head_dim (reference: quant.h:28-44):
  // key codes (P rows of W codes), value codes (the same), key scales (W fp16),
  // key zeros (W), value scales (P * kv_heads), value zeros (P * kv_heads).
  // Below 8 bits, 8/bits consecutive codes share a byte, the first lowest.
  struct PageLayout
  {
    int bits;
    std::size_t key_codes;
    std::size_t value_codes;
    std::size_t key_scales;
    std::size_t key_zeros;
    std::size_t value_scales;
    std::size_t value_zeros;
    std::size_t metadata_bytes;
    std::size_t page_bytes;
    double effective_bits;
  };

  inline int bits_of(int tier)
  {
    switch (tier)
    {
    case kINT8: return 8;
    case kINT4: return 4;
    case kINT2: return 2;
    }
    throw InvalidArgument("FP16 is not a quantised tier: its page has no codes and no metadata");
  }

  // The one place the layout's arithmetic is written (reference: quant.cu:358-392).
  inline PageLayout page_layout(int tier, int page_tokens, int kv_heads, int head_dim)
  {
    const int bits = bits_of(tier);
    if (page_tokens <= 0 || kv_heads <= 0 || head_dim <= 0)
    {
      throw InvalidArgument("page_tokens, kv_heads and head_dim must be positive, got " +
                            std::to_string(page_tokens) + ", " + std::to_string(kv_heads) +
                            ", " + std::to_string(head_dim));
    }
    if (head_dim * bits % 8 != 0)
    {
      throw InvalidArgument("head_dim " + std::to_string(head_dim) + " at " +
                            std::to_string(bits) +
                            " bits leaves a value group sharing a byte with the next");
    }
    const std::size_t width = static_cast<std::size_t>(kv_heads) * head_dim;
    const std::size_t codes = static_cast<std::size_t>(page_tokens) * width * bits / 8;
    const std::size_t key_meta = width * 2;
    const std::size_t value_meta = static_cast<std::size_t>(page_tokens) * kv_heads * 2;
    PageLayout l{};
    l.bits = bits;
    l.key_codes = 0;
    l.value_codes = codes;
    l.key_scales = 2 * codes;
    l.key_zeros = l.key_scales + key_meta;
    l.value_scales = l.key_zeros + key_meta;
    l.value_zeros = l.value_scales + value_meta;
    l.page_bytes = l.value_zeros + value_meta;
    l.metadata_bytes = l.page_bytes - 2 * codes;
    l.effective_bits = 8.0 * static_cast<double>(l.page_bytes) /
                       static_cast<double>(2 * static_cast<std::size_t>(page_tokens) * width);
    return l;
  }

  // An FP16 page: P rows of keys, then P rows of values (reference: kv_pages.cu:62-66).
  inline std::size_t fp16_page_bytes(int page_tokens, std::size_t kv_width)
  {
    return 2 * static_cast<std::size_t>(page_tokens) * kv_width * 2;
  }

  inline std::size_t page_bytes_at(int tier, int page_tokens, int kv_heads, int head_dim)
  {
    return tier == kFP16
               ? fp16_page_bytes(page_tokens, static_cast<std::size_t>(kv_heads) * head_dim)
               : page_layout(tier, page_tokens, kv_heads, head_dim).page_bytes;
  }

  // ---- fp16 helpers -----------------------------------------------------------
  // Round a double to the nearest fp16, ties to even, in one rounding (no
  // detour through fp32, which could round twice). The bits of the result.
  __host__ __device__ inline std::uint16_t half_bits_from_double(double x)
  {
    std::uint64_t b;
    std::memcpy(&b, &x, sizeof(b));
    const std::uint16_t sign = static_cast<std::uint16_t>((b >> 48) & 0x8000u);
    const int exp = static_cast<int>((b >> 52) & 0x7ff);
    const std::uint64_t mant = b & 0xFFFFFFFFFFFFFull;
    if (exp == 0x7ff)
    {
      return static_cast<std::uint16_t>(sign | 0x7c00u | (mant != 0 ? 0x200u : 0u));
    }
    if (exp == 0)
    {
      return sign; // below 2^-1022: far under half of fp16's least subnormal
    }
    const int e = exp - 1023;
    const std::uint64_t sig = mant | (1ull << 52); // value = sig * 2^(e - 52)
    // Normal fp16 keeps 11 significant bits; a subnormal counts units of 2^-24.
    const int shift = e >= -14 ? 42 : 28 - e;
    if (shift > 62)
    {
      return sign;
    }
    std::uint64_t q = sig >> shift;
    const std::uint64_t rem = sig & ((1ull << shift) - 1);
    const std::uint64_t halfway = 1ull << (shift - 1);
    if (rem > halfway || (rem == halfway && (q & 1u)))
    {
      ++q;
    }
    if (e >= -14)
    {
      int he = e + 15;
      if (q == 2048)
      {
        q = 1024;
        ++he;
      }
      if (he >= 31)
      {
        return static_cast<std::uint16_t>(sign | 0x7c00u);
      }
      return static_cast<std::uint16_t>(sign | (he << 10) | (q & 0x3ffu));
    }
    // q <= 1024; 1024 is the least normal's bit pattern, as wanted.
    return static_cast<std::uint16_t>(sign | q);
  }

  __host__ __device__ inline float half_bits_to_float(std::uint16_t h)
  {
#if defined(__HIP_DEVICE_COMPILE__)
    // On the device, the hardware conversion: exact, subnormals included.
    return __half2float(__ushort_as_half(h));
#else
    const std::uint32_t sign = static_cast<std::uint32_t>(h & 0x8000u) << 16;
    const int exp = (h >> 10) & 0x1f;
    std::uint32_t mant = h & 0x3ffu;
    std::uint32_t bits;
    if (exp == 0x1f)
    {
      bits = sign | 0x7f800000u | (mant << 13);
    }
    else if (exp != 0)
    {
      bits = sign | (static_cast<std::uint32_t>(exp - 15 + 127) << 23) | (mant << 13);
    }
    else if (mant == 0)
    {
      bits = sign;
    }
    else
    {
      int e = -14;
      while ((mant & 0x400u) == 0)
      {
        mant <<= 1;
        --e;
      }
      bits = sign | (static_cast<std::uint32_t>(e + 127) << 23) | ((mant & 0x3ffu) << 13);
    }
    float f;
    std::memcpy(&f, &bits, sizeof(f));
    return f;
#endif
  }

  // fp16 bits to fp32 on the device: the hardware conversion, exact
  // (subnormals included, fp16 denormals being on in HIP's default mode).
  __device__ inline float h2f(std::uint16_t h) { return __half2float(__ushort_as_half(h)); }

  // A block's max or sum of one float per thread, returned to every thread.
  // `scratch` holds a float per wave. Every thread of the block must call it.
  template <bool kMax>
  __device__ inline float block_reduce(float v, float *scratch)
  {
    for (int offset = warpSize / 2; offset > 0; offset /= 2)
    {
      const float o = __shfl_xor(v, offset);
      v = kMax ? fmaxf(v, o) : v + o;
    }
    const int wave = threadIdx.x / warpSize;
    const int waves = (blockDim.x + warpSize - 1) / warpSize;
    __syncthreads();
    if (threadIdx.x % warpSize == 0)
    {
      scratch[wave] = v;
    }
    __syncthreads();
    v = scratch[0];
    for (int w = 1; w < waves; ++w)
    {
      v = kMax ? fmaxf(v, scratch[w]) : v + scratch[w];
    }
    return v;
  }

  __device__ inline float widen_value(const float *x, std::size_t i) { return x[i]; }
  __device__ inline float widen_value(const std::uint16_t *x, std::size_t i) { return h2f(x[i]); }

  // 1 / RMS of one row, in the summation order every RMSNorm here shares
  // (the standalone kernel, the decode step's fused norms, the row launch),
  // so that their normed rows agree to the bit: lanes 0..255 each sum the
  // squares of the elements i = lane (mod 256) in order, a wave adds its
  // lanes by an xor butterfly, and the four wave sums are added in wave
  // order (reference arithmetic: rmsnorm.cu:33-84, fp32 throughout).
  // `partial` is four floats of LDS; every thread of the block calls it.
  template <typename In>
  __device__ inline float inv_rms(const In *x, int hidden, float eps, float *partial)
  {
    float acc = 0.0f;
    if (threadIdx.x < 256)
    {
      for (int i = threadIdx.x; i < hidden; i += 256)
      {
        const float v = widen_value(x, i);
        acc += v * v;
      }
    }
    for (int offset = 32; offset > 0; offset >>= 1)
    {
      acc += __shfl_xor(acc, offset);
    }
    if (threadIdx.x < 256 && threadIdx.x % 64 == 0)
    {
      partial[threadIdx.x / 64] = acc;
    }
    __syncthreads();
    const float total = ((partial[0] + partial[1]) + partial[2]) + partial[3];
    return rsqrtf(total / static_cast<float>(hidden) + eps);
  }

  // x * scale * w for the row's elements, one fp16 rounding each, eight a
  // thread through 16-byte stores where the row allows, else one.
  template <typename In>
  __device__ inline void normed_row(const In *x, const std::uint16_t *w, std::uint16_t *out,
                                    int hidden, float scale)
  {
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    const bool wide = hidden % 8 == 0 && (reinterpret_cast<std::uintptr_t>(out) |
                                          reinterpret_cast<std::uintptr_t>(w)) % 16 == 0;
    if (wide)
    {
      for (int r = threadIdx.x; r < hidden / 8; r += blockDim.x)
      {
        const u32x4 wv = *reinterpret_cast<const u32x4 *>(w + 8 * r);
        u32x4 o;
#pragma unroll
        for (int k = 0; k < 4; ++k)
        {
          const float a = widen_value(x, 8 * r + 2 * k) * scale * h2f(static_cast<std::uint16_t>(wv[k]));
          const float b =
              widen_value(x, 8 * r + 2 * k + 1) * scale * h2f(static_cast<std::uint16_t>(wv[k] >> 16));
          o[k] = static_cast<unsigned>(__half_as_ushort(__float2half(a))) |
                 (static_cast<unsigned>(__half_as_ushort(__float2half(b))) << 16);
        }
        *reinterpret_cast<u32x4 *>(out + 8 * r) = o;
      }
      return;
    }
    for (int i = threadIdx.x; i < hidden; i += blockDim.x)
    {
      out[i] = __half_as_ushort(__float2half(widen_value(x, i) * scale * h2f(w[i])));
    }
  }

  // RoPE of one pair (reference: rope.cu:32-54): channel j's value x1 and
  // channel j + hd/2's x2 turned by the angle's cos c and sin s, each result
  // rounded once to fp16. Every rotation here goes through this, so that
  // they agree to the bit.
  __device__ inline void rope_pair(float x1, float x2, float c, float s, std::uint16_t &lo,
                                   std::uint16_t &hi)
  {
    lo = __half_as_ushort(__float2half(x1 * c - x2 * s));
    hi = __half_as_ushort(__float2half(x2 * c + x1 * s));
  }

  // One EWMA step of a page's importance score (reference:
  // importance_scores.cu:31-50): `observed` is the heads' mean mass (summed
  // in head order, then divided); the new score is alpha * observed +
  // (1 - alpha) * old, each operation rounded once, and a page never
  // observed (NaN) takes the observation.
  __device__ inline float ewma_step(float old, float observed, float alpha)
  {
    return isnan(old) ? observed
                      : __fadd_rn(__fmul_rn(alpha, observed), __fmul_rn(__fsub_rn(1.0f, alpha), old));
  }

  // The group's scale (reference: quant.cu:44-56): its range over the
  // 2^bits - 1 steps, formed in fp64 and rounded to the nearest fp16, then
  // one fp16 ulp up if that fell short of the exact value, so that the last
  // level always reaches the maximum and no code is clamped.
  __host__ __device__ inline std::uint16_t scale_bits_of(float lo, float hi, int bits)
  {
    const double levels = static_cast<double>((1 << bits) - 1);
    const double exact = (static_cast<double>(hi) - static_cast<double>(lo)) / levels;
    const std::uint16_t nearest = half_bits_from_double(exact);
    if (static_cast<double>(half_bits_to_float(nearest)) >= exact)
    {
      return nearest;
    }
    return static_cast<std::uint16_t>(nearest + 1); // non-negative: next bit pattern is next up
  }

  // Largest page_tokens / head_dim / kv_heads any kernel here is built for.
  constexpr int kMaxHeadDim = 256;

} // namespace mi
