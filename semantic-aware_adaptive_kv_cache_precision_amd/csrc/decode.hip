// The decode attention fast path for gfx950: one query per head over a page
// table of 32-token pages at FP16/INT8/INT4/INT2, split across pages, with
// each page's attention mass and the importance-score EWMA fused in.
//
// Semantics are the reference's decode step (src/core_kernels/attention.cu:
// CausalPagedKV :302-364, PageMass :375-411, combine :754-815;
// importance_scores.cu:31-50): codes dequantised exactly as dequantise_page
// does (fmaf, then fp16 round-to-nearest), the scale applied to q.k in fp32,
// fp32 softmax and accumulation, fp16 output.
//
// Work layout (MI355X-first):
//   - a wave64 owns one 32-token page of one KV head at a time, for every
//     query head of that KV head's group (up to 16): the page is read once;
//   - q.K^T is a 16x16x32 f16 MFMA with the page's keys as the M rows and the
//     group's heads as N (q and the dequantised keys are exact in fp16, the
//     products exact in fp32);
//   - V is transposed in registers by an MFMA against a 0/1 selection matrix
//     (exact), which puts each lane's keys on the K axis for P.V; P is split
//     into an fp16 high and low part, two MFMAs, so P.V keeps ~22 bits of P;
//   - every lane keeps the softmax state of one head (lane % 16), in the
//     same lanes that hold that head's scores and output, so no value crosses
//     lanes but the max/sum reductions over the 4 lane groups;
//   - a workgroup of 4 waves covers 4 x pages_per_wave consecutive pages of
//     one KV head and writes one partial (m, l, o); a second, small kernel
//     folds the partials and turns each page's (max, sum) into its mass and
//     the layer's scores.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <vector>

namespace mi
{
  namespace
  {
    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

    constexpr int kWaves = 8;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kPageTokens = 32;
    constexpr int kMaxGroup = 16;
    constexpr int kOwnPage = 0xFE; // the query's own page: open page + chunk rows

    struct DecodeArgs
    {
      const unsigned long long *table; // each page's address
      const std::uint8_t *tiers; // null: every page FP16 (a cache that does not seal)
      const std::uint16_t *open;
      const std::uint16_t *chunk_k;
      const std::uint16_t *chunk_v;
      int start;
      int own; // the query's own page, or -1 for a cache that does not seal
      PageLayout lay[kTierCount];
      const std::uint16_t *q;
      std::uint16_t *out;
      int seq_k;
      int heads;
      int kv_heads;
      int group;
      int pages;
      int pages_per_wave;
      int splits;
      float scale;
      float *partials;   // [kv_heads][splits][group][2 + hd]
      float *page_stats; // [heads][pages][2]: each page's max and sum
      float *mass;       // [heads][pages] or null
      float *scores;     // this layer's scores or null
      float alpha;
    };

    __device__ inline half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

    __device__ inline _Float16 dq(unsigned code, float scale, float zero)
    {
      // dequantise_page's arithmetic: one fp32 fma, one fp16 rounding.
      return static_cast<_Float16>(__float2half_rn(fmaf(static_cast<float>(code), scale, zero)));
    }

    // Eight codes (natural order, the first in the lowest bits) to halves.
    template <int Bits>
    __device__ inline half8 dequant8(u32x2 codes, const float *s, const float *z)
    {
      constexpr unsigned kMask = (1u << Bits) - 1;
      half8 out;
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        const int bit = e * Bits;
        const unsigned word = bit < 32 ? codes.x : codes.y;
        out[e] = dq((word >> (bit & 31)) & kMask, s[e], z[e]);
      }
      return out;
    }

    template <int Bits>
    __device__ inline half8 dequant8_one(u32x2 codes, float s, float z)
    {
      constexpr unsigned kMask = (1u << Bits) - 1;
      half8 out;
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        const int bit = e * Bits;
        const unsigned word = bit < 32 ? codes.x : codes.y;
        out[e] = dq((word >> (bit & 31)) & kMask, s, z);
      }
      return out;
    }

    // Loads the 8 codes of elements [e0, e0 + 8) of a code region.
    template <int Bits>
    __device__ inline u32x2 load_codes(const std::uint8_t *region, std::size_t e0)
    {
      const std::uint8_t *p = region + e0 * Bits / 8;
      u32x2 v;
      if constexpr (Bits == 8)
      {
        v = *reinterpret_cast<const u32x2 *>(p);
      }
      else if constexpr (Bits == 4)
      {
        v.x = *reinterpret_cast<const unsigned *>(p);
        v.y = 0;
      }
      else
      {
        v.x = *reinterpret_cast<const unsigned short *>(p);
        v.y = 0;
      }
      return v;
    }

    __device__ inline f32x4 mfma(half8 a, half8 b, f32x4 c)
    {
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }

    template <int HD>
    struct PageOperands
    {
      static constexpr int kSteps = HD / 32;
      half8 k[2][kSteps];
      half8 v[2][kSteps];
    };

    // Loads and dequantises one page's keys and values for this lane: rows
    // kb * 16 + r (kb = 0, 1), dims s * 32 + 8 g .. + 8 of the KV head.
    template <int HD, int Bits>
    __device__ inline void load_quantised(PageOperands<HD> &op, const std::uint8_t *page,
                                          const PageLayout &L, std::size_t W, int kvh, int kv_heads,
                                          int r, int g)
    {
      constexpr int S = HD / 32;
      const std::size_t kv_off = static_cast<std::size_t>(kvh) * HD;
      const auto *ks = reinterpret_cast<const std::uint16_t *>(page + L.key_scales) + kv_off;
      const auto *kz = reinterpret_cast<const std::uint16_t *>(page + L.key_zeros) + kv_off;
      const auto *vs = reinterpret_cast<const std::uint16_t *>(page + L.value_scales);
      const auto *vz = reinterpret_cast<const std::uint16_t *>(page + L.value_zeros);
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        const int d0 = s * 32 + 8 * g;
        const u32x4 sr = *reinterpret_cast<const u32x4 *>(ks + d0);
        const u32x4 zr = *reinterpret_cast<const u32x4 *>(kz + d0);
        float sc[8], ze[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          sc[e] = h2f(static_cast<std::uint16_t>(sr[e / 2] >> (16 * (e & 1))));
          ze[e] = h2f(static_cast<std::uint16_t>(zr[e / 2] >> (16 * (e & 1))));
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          const int t = kb * 16 + r;
          const std::size_t e0 = static_cast<std::size_t>(t) * W + kv_off + d0;
          op.k[kb][s] = dequant8<Bits>(load_codes<Bits>(page + L.key_codes, e0), sc, ze);
        }
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const int t = kb * 16 + r;
        const std::size_t group = static_cast<std::size_t>(t) * kv_heads + kvh;
        const float s = h2f(vs[group]);
        const float z = h2f(vz[group]);
#pragma unroll
        for (int st = 0; st < S; ++st)
        {
          const std::size_t e0 = static_cast<std::size_t>(t) * W + kv_off + st * 32 + 8 * g;
          op.v[kb][st] = dequant8_one<Bits>(load_codes<Bits>(page + L.value_codes, e0), s, z);
        }
      }
    }

    template <int HD>
    __device__ inline void load_fp16_rows(PageOperands<HD> &op, const std::uint16_t *krow0,
                                          const std::uint16_t *krow1, const std::uint16_t *vrow0,
                                          const std::uint16_t *vrow1, int g)
    {
      constexpr int S = HD / 32;
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        const int d0 = s * 32 + 8 * g;
        op.k[0][s] = as_half8(*reinterpret_cast<const u32x4 *>(krow0 + d0));
        op.k[1][s] = as_half8(*reinterpret_cast<const u32x4 *>(krow1 + d0));
        op.v[0][s] = as_half8(*reinterpret_cast<const u32x4 *>(vrow0 + d0));
        op.v[1][s] = as_half8(*reinterpret_cast<const u32x4 *>(vrow1 + d0));
      }
    }

    template <int HD>
    __global__ void __launch_bounds__(kThreads) decode_pages_kernel(DecodeArgs a)
    {
      constexpr int S = HD / 32;   // 32-dim chunks: K steps of q.K^T
      constexpr int DB = HD / 16;  // 16-dim blocks of the output
      // Each wave's running max, sum and output, for the group's heads.
      extern __shared__ float lds[];
      constexpr int kRow = HD + 4;

      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int r = lane & 15;
      const int g = lane >> 4;
      const int kvh = blockIdx.y;
      const int split = blockIdx.x;
      const int G = a.group;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t kv_off = static_cast<std::size_t>(kvh) * HD;
      float *s_m = lds;
      float *s_l = s_m + kWaves * G;
      float *s_o = s_l + kWaves * G;

      // q of head r of the group, dims s * 32 + 8 g .. + 8; zero past the group.
      half8 qb[S];
      {
        const bool valid = r < G;
        const std::uint16_t *row = a.q + static_cast<std::size_t>(kvh * G + (valid ? r : 0)) * HD;
#pragma unroll
        for (int s = 0; s < S; ++s)
        {
          u32x4 raw = *reinterpret_cast<const u32x4 *>(row + s * 32 + 8 * g);
          if (!valid)
          {
            raw = u32x4{0u, 0u, 0u, 0u};
          }
          qb[s] = as_half8(raw);
        }
      }
      // The 0/1 matrices that transpose V: B[k][n] = (k == n + 16 h).
      half8 sel[2];
#pragma unroll
      for (int h = 0; h < 2; ++h)
      {
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          sel[h][e] = (8 * g + e == r + 16 * h) ? static_cast<_Float16>(1.0f)
                                                : static_cast<_Float16>(0.0f);
        }
      }

      float m_run = -INFINITY;
      float l_run = 0.0f;
      f32x4 o[DB];
#pragma unroll
      for (int db = 0; db < DB; ++db)
      {
        o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }

      const int first = (split * kWaves + wave) * a.pages_per_wave;
      for (int i = 0; i < a.pages_per_wave; ++i)
      {
        const int p = first + i;
        if (p >= a.pages)
        {
          break;
        }
        int tier = kFP16;
        if (a.own >= 0)
        {
          tier = p < a.own ? a.tiers[p] : kOwnPage;
        }
        float *stat = a.page_stats + (static_cast<std::size_t>(kvh * G + r) * a.pages + p) * 2;
        if (tier == kUnreadPage)
        {
          if (g == 0 && r < G)
          {
            stat[0] = -INFINITY;
            stat[1] = 0.0f;
          }
          continue;
        }
        // Rows past the last key hold nothing: masked, and zero in V.
        const int last = a.seq_k - 1 - p * kPageTokens; // last valid row of this page
        PageOperands<HD> op;
        const auto *page = reinterpret_cast<const std::uint8_t *>(a.table[p]);
        switch (tier)
        {
        case kINT8:
          load_quantised<HD, 8>(op, page, a.lay[kINT8], W, kvh, a.kv_heads, r, g);
          break;
        case kINT4:
          load_quantised<HD, 4>(op, page, a.lay[kINT4], W, kvh, a.kv_heads, r, g);
          break;
        case kINT2:
          load_quantised<HD, 2>(op, page, a.lay[kINT2], W, kvh, a.kv_heads, r, g);
          break;
        case kOwnPage:
        {
          // Rows before `start` from the open page, the rest from the chunk.
          const int t_start = a.start - p * kPageTokens;
          const std::uint16_t *rows[2][2];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
          {
            const int t = kb * 16 + r;
            const int tt = t <= last ? t : 0;
            if (tt < t_start)
            {
              rows[kb][0] = a.open + static_cast<std::size_t>(tt) * W + kv_off;
              rows[kb][1] = a.open + static_cast<std::size_t>(kPageTokens + tt) * W + kv_off;
            }
            else
            {
              rows[kb][0] = a.chunk_k + static_cast<std::size_t>(tt - t_start) * W + kv_off;
              rows[kb][1] = a.chunk_v + static_cast<std::size_t>(tt - t_start) * W + kv_off;
            }
          }
          load_fp16_rows<HD>(op, rows[0][0], rows[1][0], rows[0][1], rows[1][1], g);
          break;
        }
        default:
        {
          const auto *h = reinterpret_cast<const std::uint16_t *>(page);
          load_fp16_rows<HD>(op, h + static_cast<std::size_t>(r) * W + kv_off,
                             h + static_cast<std::size_t>(16 + r) * W + kv_off,
                             h + static_cast<std::size_t>(kPageTokens + r) * W + kv_off,
                             h + static_cast<std::size_t>(kPageTokens + 16 + r) * W + kv_off, g);
          break;
        }
        }
        // Zero the rows past the last key, so nothing unwritten reaches P.V.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          if (kb * 16 + r > last)
          {
#pragma unroll
            for (int s = 0; s < S; ++s)
            {
              op.k[kb][s] = as_half8(u32x4{0u, 0u, 0u, 0u});
              op.v[kb][s] = as_half8(u32x4{0u, 0u, 0u, 0u});
            }
          }
        }

        // Scores: lane (head r, group g) gets keys kb * 16 + 4 g + i.
        float sc[8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
          for (int s = 0; s < S; ++s)
          {
            acc = mfma(op.k[kb][s], qb[s], acc);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i)
          {
            const int t = kb * 16 + 4 * g + i;
            sc[kb * 4 + i] = t <= last ? acc[i] * a.scale : -INFINITY;
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
          pv[e] = expf(sc[e] - m_from);
          l_page += pv[e];
        }
        l_page += __shfl_xor(l_page, 16);
        l_page += __shfl_xor(l_page, 32);
        if (g == 0 && r < G)
        {
          stat[0] = m_page;
          stat[1] = l_page;
        }
        // Online merge into this wave's running softmax.
        const float m_new = fmaxf(m_run, m_page);
        const float m_new_from = m_new == -INFINITY ? 0.0f : m_new;
        const float f_old = expf(m_run - m_new_from);
        const float f_page = expf(m_page - m_new_from);
        l_run = l_run * f_old + l_page * f_page;
        m_run = m_new;
#pragma unroll
        for (int db = 0; db < DB; ++db)
        {
          o[db] *= f_old;
        }
        half8 p_hi, p_lo;
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          const float pe = pv[e] * f_page;
          const _Float16 hi = static_cast<_Float16>(pe);
          p_hi[e] = hi;
          p_lo[e] = static_cast<_Float16>(pe - static_cast<float>(hi));
        }
        // V^T by selection, then P.V: o[db][i] = O[head r][db * 16 + 4 g + i].
#pragma unroll
        for (int s = 0; s < S; ++s)
        {
#pragma unroll
          for (int h = 0; h < 2; ++h)
          {
            const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
            const f32x4 t0 = mfma(op.v[0][s], sel[h], zero);
            const f32x4 t1 = mfma(op.v[1][s], sel[h], zero);
            half8 vt;
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
              vt[i] = static_cast<_Float16>(t0[i]);
              vt[4 + i] = static_cast<_Float16>(t1[i]);
            }
            const int db = 2 * s + h;
            o[db] = mfma(vt, p_hi, o[db]);
            o[db] = mfma(vt, p_lo, o[db]);
          }
        }
      }

      // The workgroup's waves into one partial.
      if (r < G)
      {
        if (g == 0)
        {
          s_m[wave * G + r] = m_run;
          s_l[wave * G + r] = l_run;
        }
#pragma unroll
        for (int db = 0; db < DB; ++db)
        {
#pragma unroll
          for (int i = 0; i < 4; ++i)
          {
            s_o[(wave * G + r) * kRow + db * 16 + 4 * g + i] = o[db][i];
          }
        }
      }
      __syncthreads();
      float *part = a.partials + (static_cast<std::size_t>(kvh) * a.splits + split) * G * (HD + 2);
      for (int idx = threadIdx.x; idx < G * (HD + 2); idx += kThreads)
      {
        const int h = idx / (HD + 2);
        const int c = idx % (HD + 2);
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
          top = fmaxf(top, s_m[w * G + h]);
        }
        const float from = top == -INFINITY ? 0.0f : top;
        float acc = 0.0f;
        if (c == 0)
        {
          acc = top;
        }
        else
        {
#pragma unroll
          for (int w = 0; w < kWaves; ++w)
          {
            const float v = c == 1 ? s_l[w * G + h] : s_o[(w * G + h) * kRow + c - 2];
            acc += v * expf(s_m[w * G + h] - from);
          }
        }
        part[idx] = acc;
      }
    }

    constexpr int kCombineThreads = 256;
    constexpr int kCombineDims = 32;

    // Blocks [0, heads * HD / 32): one head's 32 output dims from the
    // partials, a thread a split. Blocks past that: a run of pages' masses,
    // and the layer's scores folded from them (importance_scores.cu:31-50:
    // heads summed in order, every operation rounded once).
    template <int HD>
    __global__ void __launch_bounds__(kCombineThreads) decode_combine_kernel(DecodeArgs a)
    {
      __shared__ float s_red[kCombineThreads / 64];
      __shared__ float s_acc[kCombineThreads][kCombineDims + 1];
      __shared__ float s_top[64];
      __shared__ float s_sum[64];
      const int G = a.group;
      const auto slot = [&](int h, int s) {
        const int kvh = h / G;
        return a.partials + ((static_cast<std::size_t>(kvh) * a.splits + s) * G + h % G) * (HD + 2);
      };
      constexpr int kChunks = HD / kCombineDims;
      const int t = threadIdx.x;
      if (static_cast<int>(blockIdx.x) < a.heads * kChunks)
      {
        const int h = blockIdx.x / kChunks;
        const int d0 = (blockIdx.x % kChunks) * kCombineDims;
        float top = -INFINITY;
        for (int s = t; s < a.splits; s += kCombineThreads)
        {
          top = fmaxf(top, slot(h, s)[0]);
        }
        top = block_reduce<true>(top, s_red);
        const float from = top == -INFINITY ? 0.0f : top;
        float l = 0.0f;
        float acc[kCombineDims];
#pragma unroll
        for (int d = 0; d < kCombineDims; ++d)
        {
          acc[d] = 0.0f;
        }
        for (int s = t; s < a.splits; s += kCombineThreads)
        {
          const float *p = slot(h, s);
          const float w = expf(p[0] - from);
          l += p[1] * w;
#pragma unroll
          for (int d = 0; d < kCombineDims; ++d)
          {
            acc[d] += p[2 + d0 + d] * w;
          }
        }
        l = block_reduce<false>(l, s_red);
#pragma unroll
        for (int d = 0; d < kCombineDims; ++d)
        {
          s_acc[t][d] = acc[d];
        }
        __syncthreads();
        if (t < kCombineDims)
        {
          float sum = 0.0f;
          for (int u = 0; u < kCombineThreads; ++u)
          {
            sum += s_acc[u][t];
          }
          a.out[static_cast<std::size_t>(h) * HD + d0 + t] = __half_as_ushort(__float2half(sum / l));
        }
        return;
      }
      // Every head's whole max and sum, then this block's pages.
      for (int h = 0; h < a.heads; ++h)
      {
        float top = -INFINITY;
        for (int s = t; s < a.splits; s += kCombineThreads)
        {
          top = fmaxf(top, slot(h, s)[0]);
        }
        top = block_reduce<true>(top, s_red);
        const float from = top == -INFINITY ? 0.0f : top;
        float l = 0.0f;
        for (int s = t; s < a.splits; s += kCombineThreads)
        {
          l += slot(h, s)[1] * expf(slot(h, s)[0] - from);
        }
        l = block_reduce<false>(l, s_red);
        if (t == 0)
        {
          s_top[h] = from;
          s_sum[h] = l;
        }
      }
      __syncthreads();
      const int first = (blockIdx.x - a.heads * kChunks) * kCombineThreads;
      const int page = first + t;
      if (page >= a.pages)
      {
        return;
      }
      float total = 0.0f;
      for (int h = 0; h < a.heads; ++h)
      {
        const float *st = a.page_stats + (static_cast<std::size_t>(h) * a.pages + page) * 2;
        const float mass = st[1] * expf(st[0] - s_top[h]) / s_sum[h];
        if (a.mass != nullptr)
        {
          a.mass[static_cast<std::size_t>(h) * a.pages + page] = mass;
        }
        total = __fadd_rn(total, mass);
      }
      if (a.scores != nullptr)
      {
        const float observed = __fdiv_rn(total, static_cast<float>(a.heads));
        const float old = a.scores[page];
        a.scores[page] = isnan(old) ? observed
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

  bool launch_decode_fast(const KVSource &kv, const AttentionArgs &a, hipStream_t stream)
  {
    if (a.seq_q != 1 || a.k_bias != nullptr || kv.layout == Layout::kContiguous ||
        kv.page_tokens != kPageTokens || (a.head_dim != 64 && a.head_dim != 128) ||
        a.heads / a.kv_heads > kMaxGroup || a.seq_k <= 0)
    {
      return false;
    }
    if (!aligned16(a.q) || (kv.layout == Layout::kCausal &&
                            (!aligned16(kv.open) || !aligned16(kv.chunk_k) ||
                             !aligned16(kv.chunk_v))))
    {
      return false;
    }
    DecodeArgs d{};
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        d.lay[t] = page_layout(t, kPageTokens, a.kv_heads, a.head_dim);
        const PageLayout &L = d.lay[t];
        if ((L.key_scales | L.key_zeros | L.value_codes | L.page_bytes) % 16 != 0)
        {
          return false;
        }
      }
    }
    const int group = a.heads / a.kv_heads;
    const int pages = (a.seq_k + kPageTokens - 1) / kPageTokens;
    d.table = kv.pages;
    d.tiers = kv.layout == Layout::kCausal ? kv.tiers : nullptr;
    d.open = kv.open;
    d.chunk_k = kv.chunk_k;
    d.chunk_v = kv.chunk_v;
    d.start = kv.start;
    d.own = kv.layout == Layout::kCausal ? (a.seq_k - 1) / kPageTokens : -1;
    d.q = a.q;
    d.out = a.out;
    d.seq_k = a.seq_k;
    d.heads = a.heads;
    d.kv_heads = a.kv_heads;
    d.group = group;
    d.pages = pages;
    d.scale = 1.0f / sqrtf(static_cast<float>(a.head_dim));
    d.mass = a.mass;
    d.scores = a.scores;
    d.alpha = a.alpha;
    // Pages a wave: one, so a launch has a wave a page of every KV head,
    // unless the caller gave no partials (then one workgroup a KV head, as
    // the reference splits nothing without them).
    if (a.partials != nullptr)
    {
      d.pages_per_wave = 1;
      d.splits = (pages + kWaves - 1) / kWaves;
    }
    else
    {
      d.pages_per_wave = (pages + kWaves - 1) / kWaves;
      d.splits = 1;
    }
    const std::size_t part = static_cast<std::size_t>(a.kv_heads) * d.splits * group *
                             (a.head_dim + 2);
    const std::size_t stats = static_cast<std::size_t>(a.heads) * pages * 2;
    float *ws = decode_workspace(part + stats);
    d.partials = ws;
    d.page_stats = ws + part;
    const dim3 grid(d.splits, a.kv_heads);
    const int mass_blocks = (a.mass != nullptr || a.scores != nullptr)
                                ? (pages + kCombineThreads - 1) / kCombineThreads
                                : 0;
    if (d.splits > 1024 || a.heads > 64)
    {
      return false;
    }
    const auto run = [&](auto pages_kernel, auto combine_kernel, int hd) {
      const std::size_t lds = (2 * kWaves * group + static_cast<std::size_t>(kWaves) * group *
                                                        (hd + 4)) * sizeof(float);
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(pages_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute decode LDS");
      }
      hipLaunchKernelGGL(pages_kernel, grid, dim3(kThreads), lds, stream, d);
      hip_check(hipGetLastError(), "decode pages kernel launch");
      hipLaunchKernelGGL(combine_kernel, dim3(a.heads * (hd / kCombineDims) + mass_blocks),
                         dim3(kCombineThreads), 0, stream, d);
    };
    if (a.head_dim == 128)
    {
      run(decode_pages_kernel<128>, decode_combine_kernel<128>, 128);
    }
    else
    {
      run(decode_pages_kernel<64>, decode_combine_kernel<64>, 64);
    }
    hip_check(hipGetLastError(), "decode combine kernel launch");
    return true;
  }

} // namespace mi
