// Cross-lane folds of a wave64 over the lane pairs (l, l ^ 16) and
// (l, l ^ 32), as the gfx950 VALU lane swaps v_permlane16_swap and
// v_permlane32_swap: no LDS round trip, unlike a shuffle through
// ds_bpermute. Given two copies of a value, the swap leaves each lane the
// pair's two values, lower lane first, so every lane of a pair computes the
// same result. Written as asm: the compiler's builtins for these swaps take
// two equal inputs to give two equal results, which the hardware does not.
#pragma once

#include <hip/hip_runtime.h>

namespace mi
{
  // x as the sum of two fp16 values: hi = fp16(x), lo = fp16(x - hi). The
  // difference is exact in fp32 (hi is x rounded to fp16), formed here by
  // one fma whose -1 comes through an empty asm the compiler cannot see
  // into, so that it stays an fma of an fp16 operand and is issued as
  // v_fma_mix_f32 (the conversion inside the instruction) instead of a
  // conversion back to fp32 and a subtraction. The bits are those of
  // fp16(x - float(hi)).
  __device__ inline void split_half(float x, _Float16 &hi, _Float16 &lo)
  {
    float neg_one = -1.0f;
    asm("" : "+s"(neg_one));
    hi = static_cast<_Float16>(x);
    lo = static_cast<_Float16>(__builtin_fmaf(static_cast<float>(hi), neg_one, x));
  }

  // The pair's (lower, upper) values of v over lanes l and l ^ 16.
  __device__ inline void lane_pair16(float v, float &lo, float &hi)
  {
    lo = v;
    hi = v;
    asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
  }
  // The same over lanes l and l ^ 32.
  __device__ inline void lane_pair32(float v, float &lo, float &hi)
  {
    lo = v;
    hi = v;
    asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(lo), "+v"(hi));
  }
  __device__ inline float lane_max16(float v)
  {
    float lo, hi;
    lane_pair16(v, lo, hi);
    return fmaxf(lo, hi);
  }
  __device__ inline float lane_max32(float v)
  {
    float lo, hi;
    lane_pair32(v, lo, hi);
    return fmaxf(lo, hi);
  }
  __device__ inline float lane_sum16(float v)
  {
    float lo, hi;
    lane_pair16(v, lo, hi);
    return lo + hi;
  }
  __device__ inline float lane_sum32(float v)
  {
    float lo, hi;
    lane_pair32(v, lo, hi);
    return lo + hi;
  }
} // namespace mi
