// The decode attention fast path for gfx950: one query per head over a page
// table of 32-token pages at FP16/INT8/INT4/INT2, split across pages, with
// each page's attention mass and the importance-score EWMA fused in, for one
// layer or for several layers in one launch.
//
// Semantics are the reference's decode step (src/core_kernels/attention.cu:
// CausalPagedKV :302-364, PageMass :375-411, combine :754-815;
// importance_scores.cu:31-50): the scale applied to q.k in fp32, fp32
// softmax and accumulation, fp16 output, a page's mass its share of each
// head's softmax, the EWMA folded with every operation rounded once.
//
// Work layout (MI355X-first):
//   - a wave64 owns one 32-token page of one KV head, for every query head of
//     that KV head's group (up to 16): the page is read from HBM once. Lane
//     group g (lane / 16) holds the contiguous channels [g hd/4, (g+1) hd/4)
//     of rows r and 16 + r (r = lane % 16), so each row's codes are one
//     16-byte global load at INT4 (two at INT8, one 8-byte load at INT2);
//   - codes are dequantised in registers with packed fp16 arithmetic: bytes
//     spliced into the fp16 1024 + code by v_perm, 1024 subtracted, then one
//     fp16 fma with the page's scale and zero. The reference forms
//     code * scale + zero in fp32 and rounds that to fp16; rounding the exact
//     value once to fp16 differs from it only where the fp32 value lands on
//     an fp16 tie, by one fp16 ulp;
//   - a page's key scales and zeros are read once per wave into LDS and from
//     there 32 channels at a time, not held by all 16 lanes that share them;
//   - q.K^T is a 16x16x32 f16 MFMA a 32-channel step, the page's keys as M
//     and the group's heads as N (q and the keys are exact in fp16, the
//     products in fp32); scores are kept in base-2 units (scale * log2 e
//     folded in), so the softmax weights are single exp2 instructions;
//   - V is transposed in registers by an MFMA against a 0/1 selection
//     matrix (exact), which puts each lane's keys on the K axis of P.V; P is
//     split into an fp16 high and low part, two MFMAs, keeping ~22 bits of P;
//   - each tier has its own straight-line path (keys dequantised and
//     multiplied a step at a time, FP16 values loaded after q.K^T), so that
//     no path holds a whole page twice;
//   - lane % 16 is a head throughout: its scores, softmax state and output
//     live in the same lanes, so only the max/sum over the 4 lane groups
//     crosses lanes;
//   - a workgroup of 8 waves covers 8 consecutive pages of one KV head of one
//     layer and writes one partial (m, l, o); the combine kernel folds the
//     partials, and turns each page's (max, sum) into its mass and the
//     layer's scores.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <vector>

namespace mi
{
  namespace
  {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef _Float16 half2v __attribute__((ext_vector_type(2)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));
    // Global-address-space views: loads through them are global_load_*
    // with the base in scalar registers where uniform, not flat loads.
    typedef const __attribute__((address_space(1))) u32x4 *g_u32x4;
    typedef const __attribute__((address_space(1))) u32x2 *g_u32x2;
    typedef const __attribute__((address_space(1))) unsigned *g_u32;
    typedef const __attribute__((address_space(1))) unsigned short *g_u16;

    constexpr int kWaves = 8;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kPageTokens = 32;
    constexpr int kMaxGroup = 16;
    constexpr int kMaxHeads = 64;
    constexpr int kOwnPage = 0xFE; // the query's own page: open page + chunk rows
    constexpr unsigned kMagic = 0x64646464u; // the high byte of fp16 1024, four times

    struct DecodeArgs
    {
      // Layer l = first_layer + blockIdx.z: its page addresses and tiers at
      // table/tiers + l * table_stride, its open page open_table[l] (or
      // `open` when open_table is null), its q, chunk rows, output, mass and
      // scores at blockIdx.z times the strides from the bases.
      const unsigned long long *table;
      const std::uint8_t *tiers; // null: every page FP16 (a cache that does not seal)
      const unsigned long long *open_table;
      const std::uint16_t *open;
      long long table_stride;
      int first_layer;
      const std::uint16_t *q;
      long long q_stride;
      const std::uint16_t *chunk_k;
      const std::uint16_t *chunk_v;
      long long chunk_stride;
      std::uint16_t *out;
      long long out_stride;
      float *mass;
      long long mass_stride;
      float *scores;
      long long scores_stride;
      float alpha;
      int start;
      bool causal;
      PageLayout lay[kTierCount];
      int seq_k;
      int heads;
      int kv_heads;
      int group;
      int pages;
      int pages_per_wave;
      int splits;
      float scale; // 1/sqrt(hd) * log2 e: scores in base-2 units
      float *partials;   // [launch layer][kv_heads][splits][group][2 + hd]
      float *page_stats; // [launch layer][heads][pages][2]: each page's max and sum
    };

    __device__ inline half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

    __device__ inline f32x4 mfma(half8 a, half8 b, f32x4 c)
    {
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }

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
    // values. s2/z2: four packed (scale, scale') and (zero, zero') pairs.
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
        // w0's low 16 bits: c0..c7, two bits each.
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

    // Loads `Bytes` bytes (4, 8 or a multiple of 16, aligned to that) from
    // global memory into words.
    template <int Bytes>
    __device__ inline void load_words(unsigned *w, const void *p)
    {
      const auto *b = static_cast<const std::uint8_t *>(p);
      if constexpr (Bytes >= 16)
      {
#pragma unroll
        for (int i = 0; i < Bytes / 16; ++i)
        {
          const u32x4 v = *((g_u32x4)(b + 16 * i));
          w[4 * i + 0] = v.x;
          w[4 * i + 1] = v.y;
          w[4 * i + 2] = v.z;
          w[4 * i + 3] = v.w;
        }
      }
      else if constexpr (Bytes == 8)
      {
        const u32x2 v = *((g_u32x2)(b));
        w[0] = v.x;
        w[1] = v.y;
      }
      else
      {
        w[0] = *((g_u32)(b));
      }
    }

    // One FP16 row's run of the lane's channels: HD/32 steps of 8.
    template <int HD>
    __device__ inline void load_fp16_run(half8 *dst, const std::uint16_t *run)
    {
#pragma unroll
      for (int s = 0; s < HD / 32; ++s)
      {
        dst[s] = as_half8(*((g_u32x4)(run + 8 * s)));
      }
    }

    // The channel of o[2 s + h][i] in lane group g: P.V's M index m = 4 g + i
    // reads channel 8 s + m % 8 of the run of lane group 2 h + m / 8.
    template <int HD>
    __device__ inline int out_channel(int s, int h, int g, int i)
    {
      const int m = 4 * g + i;
      return (2 * h + m / 8) * (HD / 4) + 8 * s + m % 8;
    }

    // The running softmax of one wave over its pages, for the lane's head.
    template <int HD>
    struct Running
    {
      float m;
      float l;
      f32x4 o[HD / 16];
    };

    // Everything one page needs beside its bytes.
    struct PageCtx
    {
      int r;
      int g;
      int group;
      int last;     // the page's last valid row
      bool partial; // rows past `last` exist on this page
      bool first;   // the wave's first page: it starts the running softmax
      float scale;
      float *stat;  // this page's (max, sum) slot for head r
    };

    // Scores (base-2 units) from the two 16-key accumulators, masked past
    // the last key; the page's max and sum over the lane group, its stats,
    // and the running softmax merged; returns P (hi, lo) for P.V.
    template <int HD>
    __device__ inline void softmax_page(const f32x4 (&acc)[2], const PageCtx &c, Running<HD> &run,
                                        half8 &p_hi, half8 &p_lo)
    {
      float sc[8];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
          sc[kb * 4 + i] = acc[kb][i] * c.scale;
        }
      }
      if (c.partial)
      {
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          if ((e / 4) * 16 + 4 * c.g + e % 4 > c.last)
          {
            sc[e] = -INFINITY;
          }
        }
      }
      float m_page = sc[0];
#pragma unroll
      for (int e = 1; e < 8; ++e)
      {
        m_page = fmaxf(m_page, sc[e]);
      }
      m_page = fmaxf(m_page, __shfl_xor(m_page, 16));
      m_page = fmaxf(m_page, __shfl_xor(m_page, 32));
      const float m_from = m_page == -INFINITY ? 0.0f : m_page;
      float pv[8];
      float l_page = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        pv[e] = exp2f(sc[e] - m_from);
        l_page += pv[e];
      }
      l_page += __shfl_xor(l_page, 16);
      l_page += __shfl_xor(l_page, 32);
      if (c.g == 0 && c.r < c.group)
      {
        c.stat[0] = m_page;
        c.stat[1] = l_page;
      }
      float f_page = 1.0f;
      if (c.first)
      {
        run.m = m_page;
        run.l = l_page;
      }
      else
      {
        const float m_new = fmaxf(run.m, m_page);
        const float m_new_from = m_new == -INFINITY ? 0.0f : m_new;
        const float f_old = exp2f(run.m - m_new_from);
        f_page = exp2f(m_page - m_new_from);
        run.l = run.l * f_old + l_page * f_page;
        run.m = m_new;
#pragma unroll
        for (int db = 0; db < HD / 16; ++db)
        {
          run.o[db] *= f_old;
        }
      }
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        const float pe = pv[e] * f_page;
        const _Float16 hi = static_cast<_Float16>(pe);
        p_hi[e] = hi;
        p_lo[e] = static_cast<_Float16>(pe - static_cast<float>(hi));
      }
    }

    // P.V for one 32-channel step s: V^T by selection (two MFMAs a 16-channel
    // half), then the high and low parts of P.
    template <int HD>
    __device__ inline void pv_step(Running<HD> &run, int s, half8 v0, half8 v1, int r, int g,
                                   half8 p_hi, half8 p_lo)
    {
#pragma unroll
      for (int h = 0; h < 2; ++h)
      {
        half8 sel;
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          sel[e] = (8 * g + e == r + 16 * h) ? static_cast<_Float16>(1.0f)
                                             : static_cast<_Float16>(0.0f);
        }
        const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
        const f32x4 t0 = mfma(v0, sel, zero);
        const f32x4 t1 = mfma(v1, sel, zero);
        half8 vt;
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
          vt[i] = static_cast<_Float16>(t0[i]);
          vt[4 + i] = static_cast<_Float16>(t1[i]);
        }
        run.o[2 * s + h] = mfma(vt, p_hi, run.o[2 * s + h]);
        run.o[2 * s + h] = mfma(vt, p_lo, run.o[2 * s + h]);
      }
    }

    // A page at INT8/INT4/INT2. `meta` is this wave's 4 * HD bytes of LDS.
    template <int HD, int Bits>
    __device__ inline void quantised_page(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                          const std::uint8_t *page, const PageLayout &L,
                                          std::size_t W, int kvh, int kv_heads, int lane,
                                          unsigned *meta)
    {
      constexpr int S = HD / 32;
      constexpr int kRun = HD / 4;
      constexpr int kRowBytes = kRun * Bits / 8;
      constexpr int kRowWords = kRowBytes / 4;
      constexpr int kMetaLanes = HD / 4; // 8 bytes (4 channels) a lane, a region
      const int r = c.r, g = c.g;
      const std::size_t ch0 = static_cast<std::size_t>(kvh) * HD + g * kRun;
      // Every load first: codes of both rows, the key scales and zeros (two
      // regions, a lane's 8 bytes each), the rows' value scales and zeros.
      unsigned kc[2][kRowWords], vc[2][kRowWords];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const std::size_t at = (static_cast<std::size_t>(kb * 16 + r) * W + ch0) * Bits / 8;
        load_words<kRowBytes>(kc[kb], page + L.key_codes + at);
        load_words<kRowBytes>(vc[kb], page + L.value_codes + at);
      }
      u32x2 km = {0u, 0u};
      const bool meta_lane = lane < 2 * kMetaLanes;
      if (meta_lane)
      {
        const std::size_t region = lane < kMetaLanes ? L.key_scales : L.key_zeros;
        km = *((g_u32x2)(page + region + 2 * static_cast<std::size_t>(kvh) * HD +
                         8 * (lane % kMetaLanes)));
      }
      unsigned vs[2], vz[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const std::size_t grp = static_cast<std::size_t>(kb * 16 + r) * kv_heads + kvh;
        vs[kb] = *((g_u16)(page + L.value_scales + 2 * grp));
        vz[kb] = *((g_u16)(page + L.value_zeros + 2 * grp));
      }
      // The key scales and zeros through LDS: [scales HD halves][zeros HD].
      // LDS operations of one wave complete in order; the fences keep the
      // compiler from moving the reads above the write.
      if (meta_lane)
      {
        *reinterpret_cast<u32x2 *>(meta + 2 * lane) = km;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      // q.K^T a step at a time.
      f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        const u32x4 ks = *reinterpret_cast<const u32x4 *>(meta + (g * kRun + 8 * s) / 2);
        const u32x4 kz = *reinterpret_cast<const u32x4 *>(meta + (HD + g * kRun + 8 * s) / 2);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          unsigned w0, w1 = 0;
          if constexpr (Bits == 8)
          {
            w0 = kc[kb][2 * s];
            w1 = kc[kb][2 * s + 1];
          }
          else if constexpr (Bits == 4)
          {
            w0 = kc[kb][s];
          }
          else
          {
            w0 = kc[kb][s / 2] >> (16 * (s & 1));
          }
          acc[kb] = mfma(dequant_step<Bits>(w0, w1, ks, kz), qb[s], acc[kb]);
        }
      }
      half8 p_hi, p_lo;
      softmax_page<HD>(acc, c, run, p_hi, p_lo);
      // Values: one scale and zero a row (token) of this KV head.
      u32x4 sv[2], zv[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const unsigned sp = vs[kb] | (vs[kb] << 16), zp = vz[kb] | (vz[kb] << 16);
        sv[kb] = u32x4{sp, sp, sp, sp};
        zv[kb] = u32x4{zp, zp, zp, zp};
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        half8 v[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          unsigned w0, w1 = 0;
          if constexpr (Bits == 8)
          {
            w0 = vc[kb][2 * s];
            w1 = vc[kb][2 * s + 1];
          }
          else if constexpr (Bits == 4)
          {
            w0 = vc[kb][s];
          }
          else
          {
            w0 = vc[kb][s / 2] >> (16 * (s & 1));
          }
          v[kb] = dequant_step<Bits>(w0, w1, sv[kb], zv[kb]);
        }
        pv_step<HD>(run, s, v[0], v[1], r, g, p_hi, p_lo);
      }
    }

    // A page of FP16 rows: keys at k0/k1 (rows r and 16 + r, the lane's run),
    // values at v0/v1, loaded after the scores so no page is held twice.
    // Rows past the last key may hold anything: their scores are masked, and
    // their values zeroed so that a non-finite one cannot reach P.V.
    template <int HD>
    __device__ inline void fp16_page(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                     const std::uint16_t *k0, const std::uint16_t *k1,
                                     const std::uint16_t *v0, const std::uint16_t *v1)
    {
      constexpr int S = HD / 32;
      half8 k[2][S];
      load_fp16_run<HD>(k[0], k0);
      load_fp16_run<HD>(k[1], k1);
      f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        acc[0] = mfma(k[0][s], qb[s], acc[0]);
        acc[1] = mfma(k[1][s], qb[s], acc[1]);
      }
      half8 p_hi, p_lo;
      softmax_page<HD>(acc, c, run, p_hi, p_lo);
      half8 v[2][S];
      load_fp16_run<HD>(v[0], v0);
      load_fp16_run<HD>(v[1], v1);
      if (c.partial)
      {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          if (kb * 16 + c.r > c.last)
          {
#pragma unroll
            for (int s = 0; s < S; ++s)
            {
              v[kb][s] = as_half8(u32x4{0u, 0u, 0u, 0u});
            }
          }
        }
      }
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        pv_step<HD>(run, s, v[0][s], v[1][s], c.r, c.g, p_hi, p_lo);
      }
    }

    template <int HD>
    __global__ void __launch_bounds__(kThreads) decode_pages_kernel(DecodeArgs a)
    {
      constexpr int S = HD / 32;  // K steps of q.K^T
      constexpr int DB = HD / 16; // 16-channel blocks of the output
      constexpr int kRun = HD / 4;
      constexpr int kRow = HD + 4;
      extern __shared__ float lds[];

      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int r = lane & 15;
      const int g = lane >> 4;
      const int split = blockIdx.x;
      const int kvh = blockIdx.y;
      const int li = blockIdx.z;
      const int layer = a.first_layer + li;
      const int G = a.group;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t run0 = static_cast<std::size_t>(kvh) * HD + g * kRun;
      // LDS: each wave's key metadata, then the epilogue's per-wave state.
      unsigned *meta = reinterpret_cast<unsigned *>(lds) + wave * HD;
      float *s_m = lds + kWaves * HD;
      float *s_l = s_m + kWaves * G;
      float *s_w = s_l + kWaves * G; // kWaves * G weights, then G maxima
      float *s_o = s_w + kWaves * G + G;

      const unsigned long long *table = a.table + layer * a.table_stride;
      const std::uint8_t *tiers = a.tiers != nullptr ? a.tiers + layer * a.table_stride : nullptr;
      const int own = a.causal ? (a.seq_k - 1) / kPageTokens : -1;
      const int p0 = (split * kWaves + wave) * a.pages_per_wave;
      const std::uint16_t *q_row = a.q + li * a.q_stride +
                                   static_cast<std::size_t>(kvh * G + (r < G ? r : 0)) * HD +
                                   g * kRun;
      float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;

      Running<HD> run;
      run.m = -INFINITY;
      run.l = 0.0f;
#pragma unroll
      for (int db = 0; db < DB; ++db)
      {
        run.o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }

      bool first = true;
      for (int i = 0; i < a.pages_per_wave; ++i)
      {
        const int p = p0 + i;
        if (p >= a.pages)
        {
          break;
        }
        const int tier = !a.causal ? static_cast<int>(kFP16)
                                   : (p < own ? static_cast<int>(tiers[p]) : kOwnPage);
        PageCtx c;
        c.r = r;
        c.g = g;
        c.group = G;
        c.last = a.seq_k - 1 - p * kPageTokens;
        c.partial = c.last < kPageTokens - 1;
        c.first = first;
        c.scale = a.scale;
        c.stat = stats + (static_cast<std::size_t>(kvh * G + r) * a.pages + p) * 2;
        if (tier == kUnreadPage)
        {
          if (g == 0 && r < G)
          {
            c.stat[0] = -INFINITY;
            c.stat[1] = 0.0f;
          }
          continue;
        }
        // q of head r, the lane's run of channels; zero past the group.
        half8 qb[S];
        load_fp16_run<HD>(qb, q_row);
        if (r >= G)
        {
#pragma unroll
          for (int s = 0; s < S; ++s)
          {
            qb[s] = as_half8(u32x4{0u, 0u, 0u, 0u});
          }
        }
        const auto *page = reinterpret_cast<const std::uint8_t *>(table[p]);
        switch (tier)
        {
        case kINT8:
          quantised_page<HD, 8>(run, c, qb, page, a.lay[kINT8], W, kvh, a.kv_heads, lane, meta);
          break;
        case kINT4:
          quantised_page<HD, 4>(run, c, qb, page, a.lay[kINT4], W, kvh, a.kv_heads, lane, meta);
          break;
        case kINT2:
          quantised_page<HD, 2>(run, c, qb, page, a.lay[kINT2], W, kvh, a.kv_heads, lane, meta);
          break;
        case kOwnPage:
        {
          // Rows before `start` from the open page, the rest from the chunk;
          // rows past the last key read row 0 (masked).
          const auto *open = a.open_table != nullptr
                                 ? reinterpret_cast<const std::uint16_t *>(a.open_table[layer])
                                 : a.open;
          const int t_start = a.start - p * kPageTokens;
          const std::uint16_t *ck = a.chunk_k + li * a.chunk_stride;
          const std::uint16_t *cv = a.chunk_v + li * a.chunk_stride;
          const std::uint16_t *rk[2], *rv[2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
          {
            const int t = kb * 16 + r;
            const int tt = t <= c.last ? t : 0;
            if (tt < t_start)
            {
              rk[kb] = open + static_cast<std::size_t>(tt) * W + run0;
              rv[kb] = open + static_cast<std::size_t>(kPageTokens + tt) * W + run0;
            }
            else
            {
              rk[kb] = ck + static_cast<std::size_t>(tt - t_start) * W + run0;
              rv[kb] = cv + static_cast<std::size_t>(tt - t_start) * W + run0;
            }
          }
          fp16_page<HD>(run, c, qb, rk[0], rk[1], rv[0], rv[1]);
          break;
        }
        default:
        {
          const auto *h = reinterpret_cast<const std::uint16_t *>(page);
          fp16_page<HD>(run, c, qb, h + static_cast<std::size_t>(r) * W + run0,
                        h + static_cast<std::size_t>(16 + r) * W + run0,
                        h + static_cast<std::size_t>(kPageTokens + r) * W + run0,
                        h + static_cast<std::size_t>(kPageTokens + 16 + r) * W + run0);
          break;
        }
        }
        first = false;
      }

      // The workgroup's waves into one partial: each wave's state to LDS,
      // then each (wave, head)'s weight at the heads' common max, once.
      if (r < G)
      {
        if (g == 0)
        {
          s_m[wave * G + r] = run.m;
          s_l[wave * G + r] = run.l;
        }
#pragma unroll
        for (int s = 0; s < S; ++s)
        {
#pragma unroll
          for (int h = 0; h < 2; ++h)
          {
#pragma unroll
            for (int i2 = 0; i2 < 4; ++i2)
            {
              s_o[(wave * G + r) * kRow + out_channel<HD>(s, h, g, i2)] = run.o[2 * s + h][i2];
            }
          }
        }
      }
      __syncthreads();
      if (threadIdx.x < kWaves * G)
      {
        const int h = threadIdx.x % G;
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
          top = fmaxf(top, s_m[w * G + h]);
        }
        const float from = top == -INFINITY ? 0.0f : top;
        s_w[threadIdx.x] = exp2f(s_m[threadIdx.x] - from);
        if (threadIdx.x < G)
        {
          s_w[kWaves * G + h] = top;
        }
      }
      __syncthreads();
      float *part = a.partials +
                    ((static_cast<std::size_t>(li) * a.kv_heads + kvh) * a.splits + split) * G *
                        (HD + 2);
      for (int idx = threadIdx.x; idx < G * (HD + 2); idx += kThreads)
      {
        const int h = idx / (HD + 2);
        const int col = idx % (HD + 2);
        float acc = s_w[kWaves * G + h];
        if (col != 0)
        {
          acc = 0.0f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w)
          {
            const float v = col == 1 ? s_l[w * G + h] : s_o[(w * G + h) * kRow + col - 2];
            acc += v * s_w[w * G + h];
          }
        }
        part[idx] = acc;
      }
    }

    // LDS of decode_pages_kernel, bytes.
    std::size_t pages_kernel_lds(int group, int hd)
    {
      return (static_cast<std::size_t>(kWaves) * hd + 3 * kWaves * group + group +
              static_cast<std::size_t>(kWaves) * group * (hd + 4)) *
             sizeof(float);
    }

    constexpr int kCombineThreads = 256;
    constexpr int kCombineDims = 32;
    constexpr int kSplitLanes = kCombineThreads / kCombineDims; // 8
    constexpr int kLoadsAhead = 16; // split rows a thread loads before using any
    constexpr int kHeadsAPass = 16;

    // Folds (m, l) into a running (max, sum), both softmax partials in base 2.
    __device__ inline void fold_partial(float &top, float &sum, float m, float l)
    {
      const float next = fmaxf(top, m);
      const float from = next == -INFINITY ? 0.0f : next;
      sum = sum * exp2f(top - from) + l * exp2f(m - from);
      top = next;
    }

    // Max and sum over a row of 16 lanes, every lane getting the result:
    // quad exchanges (xor 1, xor 2), then half-row and row mirrors, all DPP
    // moves that stay in registers.
    template <int Ctrl>
    __device__ inline float dpp_move(float v)
    {
      return __builtin_bit_cast(
          float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), Ctrl, 0xF, 0xF, true));
    }
    constexpr int kQuadXor1 = 0xB1; // quad_perm [1, 0, 3, 2]
    constexpr int kQuadXor2 = 0x4E; // quad_perm [2, 3, 0, 1]
    constexpr int kRowHalfMirror = 0x141;
    constexpr int kRowMirror = 0x140;

    __device__ inline float row16_max(float v)
    {
      v = fmaxf(v, dpp_move<kQuadXor1>(v));
      v = fmaxf(v, dpp_move<kQuadXor2>(v));
      v = fmaxf(v, dpp_move<kRowHalfMirror>(v));
      v = fmaxf(v, dpp_move<kRowMirror>(v));
      return v;
    }

    __device__ inline float row16_sum(float v)
    {
      v += dpp_move<kQuadXor1>(v);
      v += dpp_move<kQuadXor2>(v);
      v += dpp_move<kRowHalfMirror>(v);
      v += dpp_move<kRowMirror>(v);
      return v;
    }

    // Blocks x < heads * HD/32: one head's 32 output channels; 32 threads
    // read a split's 32 channels (coalesced), 8 splits at a time, each thread
    // issuing the loads of its next 16 splits before it uses any, since the
    // partials come from other XCDs' writes, a far round trip away. Blocks
    // past that: 256 pages' masses and the layer's scores
    // (importance_scores.cu:31-50: heads summed in order, every operation
    // rounded once). blockIdx.y is the launch's layer.
    template <int HD>
    __global__ void __launch_bounds__(kCombineThreads) decode_combine_kernel(DecodeArgs a)
    {
      __shared__ float s_red[kCombineThreads / 64];
      __shared__ float s_acc[kSplitLanes][kCombineDims + 1];
      __shared__ float s_l[kSplitLanes];
      __shared__ float s_top[kMaxHeads];
      __shared__ float s_sum[kMaxHeads];
      const int G = a.group;
      const int li = blockIdx.y;
      const int t = threadIdx.x;
      const auto slot = [&](int h, int s) {
        return a.partials +
               (((static_cast<std::size_t>(li) * a.kv_heads + h / G) * a.splits + s) * G + h % G) *
                   (HD + 2);
      };
      constexpr int kChunks = HD / kCombineDims;
      if (static_cast<int>(blockIdx.x) < a.heads * kChunks)
      {
        const int h = blockIdx.x / kChunks;
        const int d0 = (blockIdx.x % kChunks) * kCombineDims;
        const int c = t % kCombineDims;
        const int j = t / kCombineDims;
        // This thread's running max, output channel and sum over its splits.
        float top = -INFINITY, acc = 0.0f, l = 0.0f;
        for (int s0 = j; s0 < a.splits; s0 += kSplitLanes * kLoadsAhead)
        {
          float mv[kLoadsAhead], lv[kLoadsAhead], ov[kLoadsAhead];
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            const int s = s0 + i * kSplitLanes;
            mv[i] = -INFINITY;
            lv[i] = 0.0f;
            ov[i] = 0.0f;
            if (s < a.splits)
            {
              const float *p = slot(h, s);
              mv[i] = p[0];
              lv[i] = p[1];
              ov[i] = p[2 + d0 + c];
            }
          }
          float next = top;
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            next = fmaxf(next, mv[i]);
          }
          const float from = next == -INFINITY ? 0.0f : next;
          const float keep = exp2f(top - from);
          acc *= keep;
          l *= keep;
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            const float w = exp2f(mv[i] - from);
            acc += ov[i] * w;
            l += lv[i] * w;
          }
          top = next;
        }
        // Across the block: the common max, then every thread's share at it.
        const float all = block_reduce<true>(top, s_red);
        const float from = all == -INFINITY ? 0.0f : all;
        const float keep = exp2f(top - from);
        s_acc[j][c] = acc * keep;
        if (c == 0)
        {
          s_l[j] = l * keep;
        }
        __syncthreads();
        if (t < kCombineDims)
        {
          float sum = 0.0f, total = 0.0f;
#pragma unroll
          for (int u = 0; u < kSplitLanes; ++u)
          {
            sum += s_acc[u][t];
            total += s_l[u];
          }
          a.out[li * a.out_stride + static_cast<std::size_t>(h) * HD + d0 + t] =
              __half_as_ushort(__float2half(sum / total));
        }
        return;
      }
      // Every head's whole max and sum: a 16-lane row a head, each lane
      // folding every 16th split (its loads issued ahead), then the row
      // reduced with DPP moves.
      const int q = t & 15;
      for (int h0 = 0; h0 < a.heads; h0 += kCombineThreads / 16)
      {
        const int h = h0 + t / 16;
        float top = -INFINITY, sum = 0.0f;
        if (h < a.heads)
        {
          for (int s0 = q; s0 < a.splits; s0 += 16 * kLoadsAhead)
          {
            float mv[kLoadsAhead], lv[kLoadsAhead];
#pragma unroll
            for (int i = 0; i < kLoadsAhead; ++i)
            {
              const int s = s0 + 16 * i;
              mv[i] = -INFINITY;
              lv[i] = 0.0f;
              if (s < a.splits)
              {
                const float2 ml = *reinterpret_cast<const float2 *>(slot(h, s));
                mv[i] = ml.x;
                lv[i] = ml.y;
              }
            }
#pragma unroll
            for (int i = 0; i < kLoadsAhead; ++i)
            {
              fold_partial(top, sum, mv[i], lv[i]);
            }
          }
        }
        const float all = row16_max(top);
        const float from = all == -INFINITY ? 0.0f : all;
        const float total = row16_sum(sum * exp2f(top - from));
        if (q == 0 && h < a.heads)
        {
          s_top[h] = from;
          s_sum[h] = total;
        }
      }
      __syncthreads();
      const int page = (blockIdx.x - a.heads * kChunks) * kCombineThreads + t;
      if (page >= a.pages)
      {
        return;
      }
      const float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;
      float *mass = a.mass != nullptr ? a.mass + li * a.mass_stride : nullptr;
      float *scores = a.scores != nullptr ? a.scores + li * a.scores_stride : nullptr;
      const float old = scores != nullptr ? scores[page] : 0.0f; // loaded ahead of the masses
      float total = 0.0f;
      for (int h0 = 0; h0 < a.heads; h0 += kHeadsAPass)
      {
        // The page's (max, sum) of kHeadsAPass heads, loaded together.
        float2 st[kHeadsAPass];
#pragma unroll
        for (int i = 0; i < kHeadsAPass; ++i)
        {
          if (h0 + i < a.heads)
          {
            st[i] = *reinterpret_cast<const float2 *>(
                stats + (static_cast<std::size_t>(h0 + i) * a.pages + page) * 2);
          }
        }
#pragma unroll
        for (int i = 0; i < kHeadsAPass; ++i)
        {
          const int h = h0 + i;
          if (h < a.heads)
          {
            const float share = st[i].y * exp2f(st[i].x - s_top[h]) / s_sum[h];
            if (mass != nullptr)
            {
              mass[static_cast<std::size_t>(h) * a.pages + page] = share;
            }
            total = __fadd_rn(total, share);
          }
        }
      }
      if (scores != nullptr)
      {
        const float observed = __fdiv_rn(total, static_cast<float>(a.heads));
        scores[page] = isnan(old) ? observed
                                  : __fadd_rn(__fmul_rn(a.alpha, observed),
                                              __fmul_rn(__fsub_rn(1.0f, a.alpha), old));
      }
    }

    // The decode workspace: partials and page statistics. Grown on demand and
    // never freed before the process ends, so an address a captured graph
    // holds stays valid.
    float *decode_workspace(std::size_t floats)
    {
      static float *buffer = nullptr;
      static std::size_t held = 0;
      static std::vector<float *> retired;
      if (floats > held)
      {
        if (buffer != nullptr)
        {
          retired.push_back(buffer);
        }
        const std::size_t grown = std::max<std::size_t>(floats, 1 << 20);
        hip_check(hipMalloc(reinterpret_cast<void **>(&buffer), grown * sizeof(float)),
                  "hipMalloc decode workspace");
        held = grown;
      }
      return buffer;
    }

    bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

  } // namespace

  bool decode_fast_applies(const KVSource &kv, const AttentionArgs &a)
  {
    if (a.seq_q != 1 || a.k_bias != nullptr || kv.layout == Layout::kContiguous ||
        kv.page_tokens != kPageTokens || (a.head_dim != 64 && a.head_dim != 128) ||
        a.kv_heads <= 0 || a.heads % a.kv_heads != 0 || a.heads / a.kv_heads > kMaxGroup ||
        a.heads > kMaxHeads || a.seq_k <= 0)
    {
      return false;
    }
    if (!aligned16(a.q) ||
        (kv.layout == Layout::kCausal &&
         (!aligned16(kv.open) || !aligned16(kv.chunk_k) || !aligned16(kv.chunk_v))))
    {
      return false;
    }
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        const PageLayout L = page_layout(t, kPageTokens, a.kv_heads, a.head_dim);
        if ((L.key_scales | L.key_zeros | L.value_codes | L.page_bytes) % 16 != 0)
        {
          return false;
        }
      }
    }
    const int pages = (a.seq_k + kPageTokens - 1) / kPageTokens;
    return (pages + kWaves - 1) / kWaves <= 65535;
  }

  void launch_decode_layers(const KVSource &kv, const AttentionArgs &a, const DecodeLayers &ls,
                            hipStream_t stream)
  {
    if (ls.layers <= 0)
    {
      return;
    }
    DecodeArgs d{};
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        d.lay[t] = page_layout(t, kPageTokens, a.kv_heads, a.head_dim);
      }
    }
    const int group = a.heads / a.kv_heads;
    const int pages = (a.seq_k + kPageTokens - 1) / kPageTokens;
    d.table = kv.pages;
    d.tiers = kv.layout == Layout::kCausal ? kv.tiers : nullptr;
    d.open_table = ls.open_table;
    d.open = kv.open;
    d.table_stride = ls.table_stride;
    d.first_layer = ls.first_layer;
    d.q = a.q;
    d.q_stride = ls.q_stride;
    d.chunk_k = kv.chunk_k;
    d.chunk_v = kv.chunk_v;
    d.chunk_stride = ls.chunk_stride;
    d.out = a.out;
    d.out_stride = ls.out_stride;
    d.mass = a.mass;
    d.mass_stride = ls.mass_stride;
    d.scores = a.scores;
    d.scores_stride = ls.scores_stride;
    d.alpha = a.alpha;
    d.start = kv.start;
    d.causal = kv.layout == Layout::kCausal;
    d.seq_k = a.seq_k;
    d.heads = a.heads;
    d.kv_heads = a.kv_heads;
    d.group = group;
    d.pages = pages;
    // Scores in base-2 units: the softmax weights are exp2 of them.
    d.scale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(a.head_dim)));
    // A page a wave, so a launch has a wave for every page of every KV head,
    // or, unsplit, one workgroup a KV head.
    if (ls.split)
    {
      d.pages_per_wave = 1;
      d.splits = (pages + kWaves - 1) / kWaves;
    }
    else
    {
      d.pages_per_wave = (pages + kWaves - 1) / kWaves;
      d.splits = 1;
    }
    const std::size_t part = static_cast<std::size_t>(ls.layers) * a.kv_heads * d.splits * group *
                             (a.head_dim + 2);
    const std::size_t stats = static_cast<std::size_t>(ls.layers) * a.heads * pages * 2;
    float *ws = decode_workspace(part + stats);
    d.partials = ws;
    d.page_stats = ws + part;
    const int mass_blocks = (a.mass != nullptr || a.scores != nullptr)
                                ? (pages + kCombineThreads - 1) / kCombineThreads
                                : 0;
    const auto run = [&](auto pages_kernel, auto combine_kernel, int hd) {
      const std::size_t lds = pages_kernel_lds(group, hd);
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(pages_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute decode LDS");
      }
      hipLaunchKernelGGL(pages_kernel, dim3(d.splits, a.kv_heads, ls.layers), dim3(kThreads), lds,
                         stream, d);
      hip_check(hipGetLastError(), "decode pages kernel launch");
      hipLaunchKernelGGL(combine_kernel,
                         dim3(a.heads * (hd / kCombineDims) + mass_blocks, ls.layers),
                         dim3(kCombineThreads), 0, stream, d);
      hip_check(hipGetLastError(), "decode combine kernel launch");
    };
    if (a.head_dim == 128)
    {
      run(decode_pages_kernel<128>, decode_combine_kernel<128>, 128);
    }
    else
    {
      run(decode_pages_kernel<64>, decode_combine_kernel<64>, 64);
    }
  }

  bool launch_decode_fast(const KVSource &kv, const AttentionArgs &a, hipStream_t stream)
  {
    if (!decode_fast_applies(kv, a))
    {
      return false;
    }
    // Split only when the caller gave partials, as the reference splits
    // nothing without them.
    DecodeLayers one{};
    one.split = a.partials != nullptr;
    one.layers = 1;
    launch_decode_layers(kv, a, one, stream);
    return true;
  }

} // namespace mi
