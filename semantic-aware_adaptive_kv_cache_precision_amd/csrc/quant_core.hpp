// The quantiser's device arithmetic, shared by the batch quantiser
// (quant.hip) and the page jobs (page_jobs.hip).
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
#pragma once

#include "common.hpp"

namespace mi
{
  namespace quant_core
  {
    // Copies `bytes` from src to dst by the workgroup, 16 bytes a lane where
    // both are 16-byte aligned and the size a multiple of 16, else bytewise.
    __device__ inline void block_copy(std::uint8_t *__restrict__ dst,
                                      const std::uint8_t *__restrict__ src,
                                      std::size_t bytes)
    {
      const bool wide = ((reinterpret_cast<std::uintptr_t>(dst) |
                          reinterpret_cast<std::uintptr_t>(src) | bytes) &
                         15u) == 0;
      if (wide)
      {
        const std::size_t n = bytes / 16;
        const uint4 *s = reinterpret_cast<const uint4 *>(src);
        uint4 *d = reinterpret_cast<uint4 *>(dst);
        for (std::size_t i = threadIdx.x; i < n; i += blockDim.x)
        {
          d[i] = s[i];
        }
      }
      else
      {
        for (std::size_t i = threadIdx.x; i < bytes; i += blockDim.x)
        {
          dst[i] = src[i];
        }
      }
    }

    template <int Bits>
    __device__ inline unsigned code_of(float x, float zero, float scale)
    {
      constexpr float kLevels = static_cast<float>((1 << Bits) - 1);
      if (scale == 0.0f)
      {
        return 0u;
      }
      const float q = rintf((x - zero) / scale);
      return static_cast<unsigned>(fminf(fmaxf(q, 0.0f), kLevels));
    }

    // The IEEE quotients of the elements whose product quotient lies near a
    // half-integer (quotients_of's rare path).
    __device__ inline void ieee_quotients(const float (&d)[8], const float (&scale)[8],
                                                const float (&inv)[8], float (&q)[8])
    {
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        const float p = d[c] * inv[c];
        if (fabsf(p - rintf(p)) > 0.5f - 0x1p-13f && scale[c] != 0.0f)
        {
          q[c] = rintf(d[c] / scale[c]);
        }
      }
    }

    // scale_bits_of for the ranges scale_bits_fast leaves to it (negative,
    // huge or NaN), out of line.
    __device__ __noinline__ std::uint16_t scale_bits_general(float lo, float hi, int bits)
    {
      return scale_bits_of(lo, hi, bits);
    }

    // Eight codes as code_of gives them, as integer-valued floats: the
    // quotients formed as (x - zero) * inv, inv = 1 / scale (IEEE, 0 for a
    // zero scale), where that settles the rounding. With x in
    // [zero, zero + levels * scale] a quotient q is at most ~256 and the
    // product is within 1.5 * 2^-23 * q <= 4.6e-5 of the IEEE quotient, so
    // the two round to the same integer unless q lies within that of a
    // half-integer. Where some lane of the wave has a q within 2^-13 of one,
    // the IEEE quotients are formed for those elements (a branch the wave
    // takes in ~1 row of 8; the empty volatile asm keeps the compiler from
    // computing the divisions on every path). For such x the rounded
    // quotient already lies in [0, levels] (scale >= (hi - lo) / levels, and
    // the product's excess over levels is under 1e-4), so the reference's
    // clamp leaves it unchanged and is not applied. Same codes as code_of,
    // bit for bit, for finite inputs.
    template <int Bits>
    __device__ inline void quotients_of(const float (&x)[8], const float (&zero)[8],
                                        const float (&scale)[8], const float (&inv)[8],
                                        float (&q)[8])
    {
      float d[8];
      bool near = false;
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        d[c] = x[c] - zero[c];
        const float p = d[c] * inv[c];
        q[c] = rintf(p);
        near |= fabsf(p - q[c]) > 0.5f - 0x1p-13f;
      }
      if (__builtin_amdgcn_ballot_w64(near) != 0)
      {
        // The empty volatile asm keeps the compiler from forming the
        // divisions on the common path.
        asm volatile("" ::: "memory");
        ieee_quotients(d, scale, inv, q);
      }
    }

    // scale_bits_of without a double division: the smallest fp16 s with
    // s * levels >= hi - lo (what scale_bits_of's nearest-then-up gives:
    // hi - lo is a multiple of 2^-24 and levels <= 255, so the double
    // rounding of (hi - lo) / levels cannot move it across an fp16 value).
    // The fp32 estimate rounded to fp16 is within half an fp16 ulp (plus
    // 2^-22 relative) of the quotient, so the answer is it or the next up;
    // products and differences in double are exact.
    __device__ inline std::uint16_t scale_bits_fast(float lo, float hi, int bits)
    {
      const double range = static_cast<double>(hi) - static_cast<double>(lo);
      const double levels = static_cast<double>((1 << bits) - 1);
      if (range == 0.0)
      {
        return 0; // a constant group
      }
      if (!(range > 0.0) || !(range < 65504.0))
      {
        return scale_bits_general(lo, hi, bits); // negative, huge or NaN ranges
      }
      const float estimate = static_cast<float>(range) * (1.0f / static_cast<float>(levels));
      const std::uint16_t c = __half_as_ushort(__float2half_rn(estimate));
      if (static_cast<double>(half_bits_to_float(c)) * levels < range)
      {
        return static_cast<std::uint16_t>(c + 1);
      }
      if (c > 0 && static_cast<double>(half_bits_to_float(static_cast<std::uint16_t>(c - 1))) *
                           levels >= range)
      {
        return static_cast<std::uint16_t>(c - 1);
      }
      return c;
    }

    // 1 / scale for codes_of: IEEE, and 0 for a zero scale (every element
    // of such a group equals its zero, so q = 0).
    __device__ inline float inverse_of(float scale) { return scale != 0.0f ? 1.0f / scale : 0.0f; }

    __device__ inline float lds_half(const std::uint16_t *p, std::size_t i)
    {
      return __half2float(__ushort_as_half(p[i]));
    }

    // Quantises one FP16 page already in LDS (`in`: P rows of keys then P of
    // values, W halves each) into `out` (LDS, the layout's page_bytes).
    template <int Bits>
    __device__ void quantise_in_lds(const std::uint16_t *__restrict__ in,
                                    std::uint8_t *__restrict__ out,
                                    const PageLayout &L, int page_tokens,
                                    int kv_heads, int head_dim)
    {
      constexpr int kPerByte = 8 / Bits;
      const int width = kv_heads * head_dim;
      const int columns = width / kPerByte;
      const std::uint16_t *keys = in;
      const std::uint16_t *values = in + static_cast<std::size_t>(page_tokens) * width;
      std::uint16_t *k_scales = reinterpret_cast<std::uint16_t *>(out + L.key_scales);
      std::uint16_t *k_zeros = reinterpret_cast<std::uint16_t *>(out + L.key_zeros);
      std::uint16_t *v_scales = reinterpret_cast<std::uint16_t *>(out + L.value_scales);
      std::uint16_t *v_zeros = reinterpret_cast<std::uint16_t *>(out + L.value_zeros);

      // Keys: a lane owns the kPerByte channels that share a byte of every row.
      for (int column = threadIdx.x; column < columns; column += blockDim.x)
      {
        const int first = column * kPerByte;
        float lo[kPerByte], hi[kPerByte], scale[kPerByte];
#pragma unroll
        for (int c = 0; c < kPerByte; ++c)
        {
          lo[c] = INFINITY;
          hi[c] = -INFINITY;
        }
        for (int t = 0; t < page_tokens; ++t)
        {
#pragma unroll
          for (int c = 0; c < kPerByte; ++c)
          {
            const float x = lds_half(keys, static_cast<std::size_t>(t) * width + first + c);
            lo[c] = fminf(lo[c], x);
            hi[c] = fmaxf(hi[c], x);
          }
        }
#pragma unroll
        for (int c = 0; c < kPerByte; ++c)
        {
          const std::uint16_t s = scale_bits_of(lo[c], hi[c], Bits);
          k_scales[first + c] = s;
          k_zeros[first + c] = __half_as_ushort(__float2half(lo[c]));
          scale[c] = half_bits_to_float(s);
        }
        for (int t = 0; t < page_tokens; ++t)
        {
          unsigned byte = 0;
#pragma unroll
          for (int c = 0; c < kPerByte; ++c)
          {
            const float x = lds_half(keys, static_cast<std::size_t>(t) * width + first + c);
            byte |= code_of<Bits>(x, lo[c], scale[c]) << (c * Bits);
          }
          out[L.key_codes + static_cast<std::size_t>(t) * columns + column] =
              static_cast<std::uint8_t>(byte);
        }
      }

      // Values: a wave per (token, head) group, lanes reducing its range.
      const int lane = threadIdx.x % warpSize;
      const int wave = threadIdx.x / warpSize;
      const int waves = blockDim.x / warpSize;
      const int groups = page_tokens * kv_heads;
      const int bytes = head_dim / kPerByte;
      for (int group = wave; group < groups; group += waves)
      {
        const std::uint16_t *x = values + static_cast<std::size_t>(group) * head_dim;
        float lo = INFINITY, hi = -INFINITY;
        for (int i = lane; i < head_dim; i += warpSize)
        {
          const float v = lds_half(x, i);
          lo = fminf(lo, v);
          hi = fmaxf(hi, v);
        }
        for (int offset = warpSize / 2; offset > 0; offset /= 2)
        {
          lo = fminf(lo, __shfl_xor(lo, offset));
          hi = fmaxf(hi, __shfl_xor(hi, offset));
        }
        const std::uint16_t s = scale_bits_of(lo, hi, Bits);
        if (lane == 0)
        {
          v_scales[group] = s;
          v_zeros[group] = __half_as_ushort(__float2half(lo));
        }
        const float scale = half_bits_to_float(s);
        std::uint8_t *codes = out + L.value_codes + static_cast<std::size_t>(group) * bytes;
        for (int b = lane; b < bytes; b += warpSize)
        {
          unsigned byte = 0;
#pragma unroll
          for (int c = 0; c < kPerByte; ++c)
          {
            byte |= code_of<Bits>(lds_half(x, b * kPerByte + c), lo, scale) << (c * Bits);
          }
          codes[b] = static_cast<std::uint8_t>(byte);
        }
      }
    }

  } // namespace quant_core
} // namespace mi
