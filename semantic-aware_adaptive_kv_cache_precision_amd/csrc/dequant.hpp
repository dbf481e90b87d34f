// Codes to fp16 values in registers with packed fp16 arithmetic, shared by
// the decode and chunk-attention kernels.
//
// Eight codes of a quantised page (reference layout: quant.cu:358-392, the
// first code in the lowest bits) become eight fp16 values code * scale +
// zero: each code's byte is spliced under the high byte of fp16 1024 by
// v_perm (the fp16 1024 + code, exact), 1024 is subtracted (exact), and one
// packed fp16 fma forms code * scale + zero rounded once. The reference forms
// code * scale + zero in fp32 and rounds that to fp16 (quant.cu:403-450);
// rounding the exact value once differs from it only where the fp32 value
// lands on an fp16 tie, by one fp16 ulp.

#pragma once

namespace mi
{
  namespace dq
  {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

    constexpr unsigned kMagic = 0x64646464u; // the high byte of fp16 1024, four times

    // Two codes spliced as fp16 (1024 + code) -> code * s + z, packed pairs.
    __device__ inline unsigned dq2(unsigned spliced, unsigned s, unsigned z)
    {
      const _Float16 k1024 = static_cast<_Float16>(1024.0f);
      half2v h = __builtin_bit_cast(half2v, spliced);
      h = h - half2v{k1024, k1024};
      h = __builtin_elementwise_fma(h, __builtin_bit_cast(half2v, s),
                                    __builtin_bit_cast(half2v, z));
      return __builtin_bit_cast(unsigned, h);
    }

    // Eight codes, natural order (the first in the lowest bits), to eight fp16
    // values: INT8 codes in w0 (first four) and w1, INT4 in w0, INT2 in w0's
    // low 16 bits. s2/z2: four packed (scale, scale') and (zero, zero') pairs.
    template <int Bits>
    __device__ inline half8 dequant_step(unsigned w0, unsigned w1, u32x4 s2, u32x4 z2)
    {
      u32x4 out;
      if constexpr (Bits == 8)
      {
        out[0] = dq2(__builtin_amdgcn_perm(kMagic, w0, 0x04010400u), s2[0], z2[0]);
        out[1] = dq2(__builtin_amdgcn_perm(kMagic, w0, 0x04030402u), s2[1], z2[1]);
        out[2] = dq2(__builtin_amdgcn_perm(kMagic, w1, 0x04010400u), s2[2], z2[2]);
        out[3] = dq2(__builtin_amdgcn_perm(kMagic, w1, 0x04030402u), s2[3], z2[3]);
      }
      else if constexpr (Bits == 4)
      {
        const unsigned lo = w0 & 0x0F0F0F0Fu;        // bytes n0 n2 n4 n6
        const unsigned hi = (w0 >> 4) & 0x0F0F0F0Fu; // bytes n1 n3 n5 n7
        const unsigned n0123 = __builtin_amdgcn_perm(hi, lo, 0x05010400u);
        const unsigned n4567 = __builtin_amdgcn_perm(hi, lo, 0x07030602u);
        out[0] = dq2(__builtin_amdgcn_perm(kMagic, n0123, 0x04010400u), s2[0], z2[0]);
        out[1] = dq2(__builtin_amdgcn_perm(kMagic, n0123, 0x04030402u), s2[1], z2[1]);
        out[2] = dq2(__builtin_amdgcn_perm(kMagic, n4567, 0x04010400u), s2[2], z2[2]);
        out[3] = dq2(__builtin_amdgcn_perm(kMagic, n4567, 0x04030402u), s2[3], z2[3]);
      }
      else
      {
        const unsigned c04 = w0 & 0x0303u;        // bytes c0 c4
        const unsigned c15 = (w0 >> 2) & 0x0303u; // bytes c1 c5
        const unsigned c26 = (w0 >> 4) & 0x0303u; // bytes c2 c6
        const unsigned c37 = (w0 >> 6) & 0x0303u; // bytes c3 c7
        const unsigned ab = c04 | (c15 << 16);    // bytes c0 c4 c1 c5
        const unsigned cd = c26 | (c37 << 16);    // bytes c2 c6 c3 c7
        out[0] = dq2(__builtin_amdgcn_perm(kMagic, ab, 0x04020400u), s2[0], z2[0]);
        out[1] = dq2(__builtin_amdgcn_perm(kMagic, cd, 0x04020400u), s2[1], z2[1]);
        out[2] = dq2(__builtin_amdgcn_perm(kMagic, ab, 0x04030401u), s2[2], z2[2]);
        out[3] = dq2(__builtin_amdgcn_perm(kMagic, cd, 0x04030401u), s2[3], z2[3]);
      }
      return __builtin_bit_cast(half8, out);
    }
  } // namespace dq
} // namespace mi
