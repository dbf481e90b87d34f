// The register quantiser's tasks and a store's row jobs, shared by the page
// job kernels (page_jobs.hip) and the decode's combine, which seals a
// step's page (decode.hip).
//
// A 32-token page of W = kv_heads * head_dim channels (head_dim 64 or 128)
// is W tasks of 64 elements, a lane each, none staged through LDS:
//   - key task (j, g), W/2 of them: channels [8j, 8j + 8) of rows
//     [8g, 8g + 8), eight 16-byte loads. A key channel's range is over all
//     32 rows, so the four tasks of a chunk (adjacent lanes) fold their
//     minima and maxima with two lane exchanges; each then codes its own
//     8 rows, one 2/4/8-byte store a row;
//   - value task (r, h, part), W/2 of them: channels [64 part, 64 part + 64)
//     of head h in row r, eight 16-byte loads; at head_dim 128 the two
//     parts of a (row, head) group fold their range with one exchange; the
//     codes leave in 16-byte stores.
// Codes, scales and zeros follow quant_core.hpp (the reference's rules,
// quant.cu:44-199) to the bit.

#pragma once

#include "common.hpp"
#include "kernels.hpp"
#include "quant_core.hpp"

namespace mi
{
  namespace page_tasks
  {
    constexpr int kP = 32; // the register quantiser's page

    // Rows [0, split) at lo, rows [split, P) at hi; `width` halves a row.
    struct Rows
    {
      const std::uint16_t *lo;
      const std::uint16_t *hi;
      int split;
      int width;
      __device__ const std::uint16_t *row(int t) const
      {
        return t < split ? lo + static_cast<std::size_t>(t) * width
                         : hi + static_cast<std::size_t>(t - split) * width;
      }
    };

    // Rows and pages are device (or host-mapped) memory, never LDS: reached
    // through global-address-space pointers, so that the compiler issues
    // global rather than flat instructions (a flat access also counts
    // against the LDS and scalar-load wait counter).
    // (Native vectors: HIP's uint4 and uint2 are classes, whose copy
    // constructor would take the value back through a generic reference.)
    typedef unsigned words4 __attribute__((ext_vector_type(4)));
    typedef unsigned words2 __attribute__((ext_vector_type(2)));
    typedef const __attribute__((address_space(1))) words4 *global_cw4;
    typedef __attribute__((address_space(1))) words4 *global_w4;
    typedef __attribute__((address_space(1))) words2 *global_w2;
    typedef __attribute__((address_space(1))) unsigned *global_u32;
    typedef __attribute__((address_space(1))) std::uint16_t *global_u16;

    __device__ inline uint4 load16(const std::uint16_t *p)
    {
      const words4 w = *((global_cw4)(p));
      return uint4{w.x, w.y, w.z, w.w};
    }
    __device__ inline void store16(void *p, uint4 v)
    {
      *((global_w4)(p)) = words4{v.x, v.y, v.z, v.w};
    }

    // fp16 bits to fp32 by the hardware conversion (exact, denormals kept).
    __device__ inline float f16_bits(unsigned bits)
    {
      return __half2float(__ushort_as_half(static_cast<unsigned short>(bits)));
    }

    __device__ inline float half_at(const uint4 &v, int c)
    {
      const unsigned w = c < 2 ? v.x : c < 4 ? v.y : c < 6 ? v.z : v.w;
      return f16_bits((c & 1) ? (w >> 16) : (w & 0xFFFFu));
    }

    __device__ inline unsigned half_of(float x) { return __half_as_ushort(__float2half_rn(x)); }

    // What a task does with the page it reads.
    enum class Emit : int
    {
      kCodes,  // the quantised page at dst
      kRound,  // this half through the tier and back, as FP16 rows at dst
      kRaw,    // this half's rows as they are, at dst
    };

    // Eight codes of one 16-byte run (eight fp16 values), packed the first
    // lowest: 8 (INT8), 4 (INT4) or 2 (INT2) bytes. The codes are exact
    // integers in floats: two INT4 (or four INT2) codes are combined into
    // one byte's value exactly (q0 + 16 q1, ...) and each byte is placed by
    // v_cvt_pk_u8_f32 (of an integer: no rounding).
    template <int Bits>
    __device__ __forceinline__ unsigned long long codes8(const uint4 &v, const float (&lo)[8],
                                                         const float (&scale)[8],
                                                         const float (&inv)[8])
    {
      float x[8], q[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        x[c] = half_at(v, c);
      }
      quant_core::quotients_of<Bits>(x, lo, scale, inv, q);
      if constexpr (Bits == 8)
      {
        unsigned w0 = 0, w1 = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
          w0 = __builtin_amdgcn_cvt_pk_u8_f32(q[c], c, w0);
          w1 = __builtin_amdgcn_cvt_pk_u8_f32(q[4 + c], c, w1);
        }
        return static_cast<unsigned long long>(w0) | (static_cast<unsigned long long>(w1) << 32);
      }
      else if constexpr (Bits == 4)
      {
        unsigned w = 0;
#pragma unroll
        for (int c = 0; c < 4; ++c)
        {
          w = __builtin_amdgcn_cvt_pk_u8_f32(fmaf(q[2 * c + 1], 16.0f, q[2 * c]), c, w);
        }
        return w;
      }
      else
      {
        unsigned w = 0;
#pragma unroll
        for (int c = 0; c < 2; ++c)
        {
          const float b = fmaf(q[4 * c + 3], 64.0f,
                               fmaf(q[4 * c + 2], 16.0f, fmaf(q[4 * c + 1], 4.0f, q[4 * c])));
          w = __builtin_amdgcn_cvt_pk_u8_f32(b, c, w);
        }
        return w;
      }
    }

    template <int Bits>
    __device__ __forceinline__ void store_codes8(std::uint8_t *at, unsigned long long packed)
    {
      if constexpr (Bits == 8)
      {
        *((global_w2)(at)) =
            words2{static_cast<unsigned>(packed), static_cast<unsigned>(packed >> 32)};
      }
      else if constexpr (Bits == 4)
      {
        *((global_u32)(at)) = static_cast<unsigned>(packed);
      }
      else
      {
        *((global_u16)(at)) = static_cast<std::uint16_t>(packed);
      }
    }

    // fmaf(code, scale, zero) to fp16 for eight codes, as dequantise_page.
    template <int Bits>
    __device__ __forceinline__ uint4 round8(const uint4 &v, const float (&lo)[8],
                                            const float (&scale)[8], const float (&inv)[8])
    {
      float x[8], q[8];
      unsigned h[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        x[c] = half_at(v, c);
      }
      quant_core::quotients_of<Bits>(x, lo, scale, inv, q);
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        h[c] = half_of(fmaf(q[c], scale[c], lo[c]));
      }
      return uint4{h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16),
                   h[6] | (h[7] << 16)};
    }

    // A key task: channels [8j, 8j + 8) of rows [8g, 8g + 8). The four tasks
    // of chunk j sit in lanes 4j .. 4j + 3 of one wave. The eight rows are
    // loaded at once and held in registers: the ranges (folded across the
    // chunk's four lanes), then the codes a row at a time.
    template <int Bits>
    __device__ __forceinline__ void key_task(const Rows &keys, int j, int g, int W,
                                             std::uint8_t *dst, const PageLayout &L, Emit emit,
                                             int rows_limit, int dst_row)
    {
      if (emit == Emit::kRaw)
      {
        auto *out = reinterpret_cast<std::uint16_t *>(dst);
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
          // A fill brings fewer rows than a page: rows past them are not read.
          const int t = 8 * g + i;
          if (t < rows_limit)
          {
            store16(out + static_cast<std::size_t>(dst_row + t) * W + 8 * j,
                    load16(keys.row(t) + 8 * j));
          }
        }
        return;
      }
      float lo[8], hi[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        lo[c] = INFINITY;
        hi[c] = -INFINITY;
      }
      // The eight rows stay in registers from the range to the codes.
      uint4 raw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
        raw[i] = load16(keys.row(8 * g + i) + 8 * j);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
#pragma unroll
        for (int c = 0; c < 8; ++c)
        {
          const float x = half_at(raw[i], c);
          lo[c] = fminf(lo[c], x);
          hi[c] = fmaxf(hi[c], x);
        }
      }
      // The chunk's four row groups: lanes that differ in the low two bits.
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        lo[c] = fminf(lo[c], __shfl_xor(lo[c], 1));
        hi[c] = fmaxf(hi[c], __shfl_xor(hi[c], 1));
        lo[c] = fminf(lo[c], __shfl_xor(lo[c], 2));
        hi[c] = fmaxf(hi[c], __shfl_xor(hi[c], 2));
      }
      float scale[8], inv[8];
      unsigned sword[4] = {0, 0, 0, 0}, zword[4] = {0, 0, 0, 0};
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        const std::uint16_t s = quant_core::scale_bits_fast(lo[c], hi[c], Bits);
        scale[c] = f16_bits(s);
        inv[c] = quant_core::inverse_of(scale[c]);
        sword[c / 2] |= static_cast<unsigned>(s) << (16 * (c % 2));
        zword[c / 2] |= half_of(lo[c]) << (16 * (c % 2));
      }
      if (emit == Emit::kCodes)
      {
        if (g == 0)
        {
          store16(reinterpret_cast<std::uint16_t *>(dst + L.key_scales) + 8 * j,
                  uint4{sword[0], sword[1], sword[2], sword[3]});
          store16(reinterpret_cast<std::uint16_t *>(dst + L.key_zeros) + 8 * j,
                  uint4{zword[0], zword[1], zword[2], zword[3]});
        }
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
          const int t = 8 * g + i;
          const std::size_t e = static_cast<std::size_t>(t) * W + 8 * j; // first element
          store_codes8<Bits>(dst + L.key_codes + e * Bits / 8,
                             codes8<Bits>(raw[i], lo, scale, inv));
        }
        return;
      }
      // Round trip: each code back to fp16, as dequantise_page gives it.
      auto *out = reinterpret_cast<std::uint16_t *>(dst);
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
        const int t = 8 * g + i;
        store16(out + static_cast<std::size_t>(t) * W + 8 * j,
                round8<Bits>(raw[i], lo, scale, inv));
      }
    }

    // A value task: channels [64 part, 64 part + 64) of head h in row r.
    // At head_dim 128 the group's two parts sit in adjacent lanes. The row's
    // eight 16-byte runs held in registers, as a key task's rows.
    template <int Bits, int HD>
    __device__ __forceinline__ void value_task(const Rows &values, int r, int h, int part,
                                               int kv_heads, int W, std::uint8_t *dst,
                                               const PageLayout &L, Emit emit, int rows_limit,
                                               int dst_row)
    {
      const int ch0 = h * HD + 64 * part;
      if (r >= rows_limit)
      {
        return; // a fill's row past those it brings: nothing to read or write
      }
      const std::uint16_t *src = values.row(r) + ch0;
      // FP16 output rows (raw and round trip) sit in the page's second half.
      auto *out = reinterpret_cast<std::uint16_t *>(dst) + static_cast<std::size_t>(kP) * W;
      if (emit == Emit::kRaw)
      {
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
          store16(out + static_cast<std::size_t>(dst_row + r) * W + ch0 + 8 * i,
                  load16(src + 8 * i));
        }
        return;
      }
      float lo = INFINITY, hi = -INFINITY;
      uint4 raw[8];
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
        raw[i] = load16(src + 8 * i);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
#pragma unroll
        for (int c = 0; c < 8; ++c)
        {
          const float x = half_at(raw[i], c);
          lo = fminf(lo, x);
          hi = fmaxf(hi, x);
        }
      }
      if constexpr (HD == 128)
      {
        lo = fminf(lo, __shfl_xor(lo, 1));
        hi = fmaxf(hi, __shfl_xor(hi, 1));
      }
      const std::uint16_t sbits = quant_core::scale_bits_fast(lo, hi, Bits);
      const float scale = f16_bits(sbits);
      const float inverse = quant_core::inverse_of(scale);
      float los[8], scales[8], invs[8];
#pragma unroll
      for (int c = 0; c < 8; ++c)
      {
        los[c] = lo;
        scales[c] = scale;
        invs[c] = inverse;
      }
      if (emit == Emit::kCodes)
      {
        if (part == 0)
        {
          const int group = r * kv_heads + h;
          ((global_u16)(dst + L.value_scales))[group] = sbits;
          ((global_u16)(dst + L.value_zeros))[group] = static_cast<std::uint16_t>(half_of(lo));
        }
        // The run's 64 codes (8 Bits bytes), 16-byte aligned: whole
        // 16-byte stores.
        std::uint8_t *at =
            dst + L.value_codes + (static_cast<std::size_t>(r) * W + ch0) * Bits / 8;
        unsigned words[2 * Bits];
#pragma unroll
        for (int i = 0; i < 8; ++i)
        {
          const unsigned long long packed = codes8<Bits>(raw[i], los, scales, invs);
          if constexpr (Bits == 8)
          {
            words[2 * i] = static_cast<unsigned>(packed);
            words[2 * i + 1] = static_cast<unsigned>(packed >> 32);
          }
          else if constexpr (Bits == 4)
          {
            words[i] = static_cast<unsigned>(packed);
          }
          else if (i % 2 == 0)
          {
            words[i / 2] = static_cast<unsigned>(packed);
          }
          else
          {
            words[i / 2] |= static_cast<unsigned>(packed) << 16;
          }
        }
#pragma unroll
        for (int w = 0; w < 2 * Bits; w += 4)
        {
          store16(at + 4 * w, uint4{words[w], words[w + 1], words[w + 2], words[w + 3]});
        }
        return;
      }
#pragma unroll
      for (int i = 0; i < 8; ++i)
      {
        store16(out + static_cast<std::size_t>(r) * W + ch0 + 8 * i,
                round8<Bits>(raw[i], los, scales, invs));
      }
    }

    // Task `task` (of W) of one 32-token page: keys first, then values.
    template <int Bits, int HD>
    __device__ __forceinline__ void page_task(int task, const Rows &keys, const Rows &values, int kv_heads,
                              std::uint8_t *dst, const PageLayout &L, Emit key_emit,
                              Emit value_emit, int rows_limit = kP, int dst_row = 0)
    {
      const int W = kv_heads * HD;
      if (task < W / 2)
      {
        key_task<Bits>(keys, task >> 2, task & 3, W, dst, L, key_emit, rows_limit, dst_row);
      }
      else
      {
        constexpr int kParts = HD / 64;
        const int v = task - W / 2;
        const int group = v / kParts;
        value_task<Bits, HD>(values, group / kv_heads, group % kv_heads, v % kParts, kv_heads, W,
                             dst, L, value_emit, rows_limit, dst_row);
      }
    }

    // One task of a store's row job (RowJob): a fill of open-page rows, a
    // seal (copy or quantise) of a full page from its rows, or the Halves
    // diagnostic's round trip.
    template <int HD>
    __device__ __forceinline__ void run_row_task(const RowJob &j, const PageLayout *lay, int task, int kv_heads)
    {
      const int W = kv_heads * HD;
      const RowJobKind kind = static_cast<RowJobKind>(j.kind);
      const Rows keys{j.k_lo, j.k_hi, j.split, W};
      const Rows values{j.v_lo, j.v_hi, j.split, W};
      const Emit ke = kind == RowJobKind::kQuantise   ? Emit::kCodes
                      : kind == RowJobKind::kRoundKeys ? Emit::kRound
                                                       : Emit::kRaw;
      const Emit ve = kind == RowJobKind::kQuantise     ? Emit::kCodes
                      : kind == RowJobKind::kRoundValues ? Emit::kRound
                                                         : Emit::kRaw;
      const int rows = kind == RowJobKind::kFill ? j.rows : kP;
      const int dst_row = kind == RowJobKind::kFill ? j.dst_row : 0;
      const bool coded = ke != Emit::kRaw || ve != Emit::kRaw;
      const PageLayout &L = lay[coded ? j.tier : kINT8];
      const int bits = coded ? L.bits : 0;
      switch (bits)
      {
      case 8: page_task<8, HD>(task, keys, values, kv_heads, j.dst, L, ke, ve, rows, dst_row); break;
      case 4: page_task<4, HD>(task, keys, values, kv_heads, j.dst, L, ke, ve, rows, dst_row); break;
      case 2: page_task<2, HD>(task, keys, values, kv_heads, j.dst, L, ke, ve, rows, dst_row); break;
      default: page_task<8, HD>(task, keys, values, kv_heads, j.dst, L, Emit::kRaw, Emit::kRaw, rows,
                                dst_row);
      }
    }

  } // namespace page_tasks
} // namespace mi
