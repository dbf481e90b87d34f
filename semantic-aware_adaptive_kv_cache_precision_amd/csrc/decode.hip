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
#include "dequant.hpp"
#include "kernels.hpp"
#include "page_tasks.hpp"
#include "lane_ops.hpp"

#include <algorithm>
#include <cmath>
#include <map>
#include <mutex>
#include <numeric>
#include <tuple>
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
      // Streaming launches: the (layer, KV-head block, page) units split into
      // stream_ranges equal contiguous ranges. A range is walked by
      // stream_ways waves of one workgroup together, one KV head of the block
      // each, so that the bytes of a page's KV heads, which share its rows'
      // lines, are asked for at the same time on one CU. A group's splits
      // are the ranges that meet it. 0: fixed splits of pages_per_wave * 8.
      long long stream_units;
      int stream_ranges;
      int stream_ways;
      // The key bias (one layer's, kv_heads x hd fp16), the RoPE table
      // ({cos, sin} per position and angle, fp32) and its first page's
      // angles as fp16 high and low parts ([row][hi | lo][hd]); null: no bias.
      const std::uint16_t *k_bias;
      const float *rope;
      const std::uint16_t *rope_angles;
      // The next layer's page table, read ahead by the combine's last
      // kWarmBlocks blocks (one an XCD): a byte of tier and 8 of address a
      // page.
      const unsigned long long *warm_table;
      const std::uint8_t *warm_tiers;
      int warm_count;
      int mass_blocks;
      // Added to the combine's block index: a launch of mass blocks alone
      // (the deferred fold) starts past the output blocks.
      int block_base;
      // A launch whose position lives on the device (a graphed decode step):
      // seq_k is read from *live_seq_k when the kernels run, and the launch
      // is sized by `pages` and `splits` for the most positions it may see,
      // which stay the strides of every per-page and per-split array. Null:
      // seq_k as given. live_pages and live_splits bound the work either way.
      const int *live_seq_k;
      int live_pages;
      int live_splits;
      int score_every; // a mass block folds only at a seq_k that is a multiple of this
      float *partials;   // [launch layer][kv_heads][splits][group][hd]: each split's output
      float *split_ml;   // [launch layer][kv_heads][group][splits][2]: each split's max and
                         // sum, a head's splits side by side so that they read coalesced
      float *page_stats; // [launch layer][kv_heads][pages][group][2]: each page's max and
                         // sum, a page's heads side by side so that one store writes them
      // Two KV heads of head_dim 64 read as one 128-channel unit (pack = 2;
      // 0 otherwise): kv_heads and group then count packs and a pack's
      // heads, q enters block-diagonal (a head's query in its own KV head's
      // channels, zeros in the other's), a value row's scale and zero come
      // from the lane's own KV head (value_kv_heads of them a row), and each
      // head's partial keeps its own 64 channels. Page statistics stay in
      // the layout of stat_group heads a KV head in every case.
      int pack;
      int value_kv_heads;
      int stat_group;
      // A step's page seal (DecodeLayers::seal) by the combine's block
      // seal_block - 1; 0: none.
      StepStore seal;
      int seal_block;
      // The workgroups a KV head's split launch holds at once (0: no bound).
      // When the live splits exceed it, busy_splits workgroups take the
      // pages: each its own kWaves, and the pages past busy_splits * kWaves
      // a wave each as a second page (kWaves * busy_splits on from its
      // first); the splits past them are written as empty partials, so that
      // readers of live_splits partials see the same layout.
      int busy_splits;
      // The row launch's work in the pages launch (decode_pages_kernel with
      // kRow; a cache that does not seal, no key bias): q and the current
      // row's k are row_qk's raw rows (q_heads then kv_heads), turned by RoPE
      // at position seq_k - 1 from row_table as each wave needs them; the
      // current row's values are row_v; the wave reading the current page
      // takes that row from registers and stores it into the page. One more
      // workgroup forms RMSNorm(row_x) into row_normed when row_x is given.
      // The turned q and k rows go to row_qk_out when it is given.
      const std::uint16_t *row_qk;
      std::uint16_t *row_qk_out;
      const std::uint16_t *row_v;
      const float *row_table;
      int row_q_heads;
      const float *row_x;
      const std::uint16_t *row_norm_weight;
      std::uint16_t *row_normed;
      int row_hidden;
      float row_eps;
    };

    __device__ inline half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }
    __device__ inline u32x4 as_u32x4(half8 v) { return __builtin_bit_cast(u32x4, v); }

    // The launch's position, when it lives on the device: seq_k, the first
    // chunk row (a decode step brings one) and the live bounds.
    __device__ inline void go_live(DecodeArgs &a)
    {
      if (a.live_seq_k != nullptr)
      {
        const int seq_k = *a.live_seq_k;
        a.seq_k = seq_k;
        a.start = seq_k - 1;
        a.live_pages = (seq_k + kPageTokens - 1) / kPageTokens;
        const int per_split = kWaves * a.pages_per_wave;
        a.live_splits = (a.live_pages + per_split - 1) / per_split;
      }
    }

    // 2^x as the one hardware instruction (v_exp_f32): softmax weights and
    // rescale factors, where a result below 2^-126 weighs nothing.
    __device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

    // P enters P.V scaled by 2^14 (exact), so that its fp16 high and low
    // parts stay normal numbers for every weight above 2^-17 of the running
    // maximum, however far a page's own maximum sits below it; o carries the
    // same factor until it leaves the wave.
    constexpr float kPScale = 16384.0f;
    constexpr float kPUnscale = 1.0f / 16384.0f;

    // A partial slot: m, l, then padding to 128 bytes, then the HD outputs,
    // so that each 32-channel chunk of o is one aligned 128-byte line.

    __device__ inline f32x4 mfma(half8 a, half8 b, f32x4 c)
    {
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }

    using dq::dequant_step;

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

    // The key bias as a term of the scores. With k + RoPE(b, t) for the keys
    // (attention.cu:104-116: channel j < hd/2 pairs with j' = j + hd/2),
    // q.RoPE(b, t) = sum over angles j of A_j cos(w_j t) + B_j sin(w_j t),
    // A_j = q_j b_j + q_j' b_j', B_j = q_j' b_j - q_j b_j'. For the rows
    // t = t0 + u of a page, RoPE(b, t) = RoPE(RoPE(b, t0), u): with the bias
    // turned to the page's first row, b(t0) = RoPE(b, t0), the term is
    // [cos | sin](w u) against [A | B] of b(t0), the same for every page but
    // for A and B. That product runs on the matrix cores in the q.K layout,
    // both operands split into fp16 high and low parts (hi.hi + hi.lo + lo.hi)
    // for fp32 accuracy, its left operand the 32 rows of [cos | sin](w u):
    // 16 KB that a workgroup copies to its LDS once, where [cos | sin](w t) of
    // every position would be as many bytes as the keys.
    template <int HD>
    struct KeyBias
    {
      float b, b2;               // lane i's bias b_i, b_i' (i = lane % (HD/2))
      float2 turn;               // cos, sin of angle i at the page's first row
      const std::uint16_t *rows; // the angle rows in LDS, kAngleRowPitch<HD> apart
      float *lds;                // the wave's 2 HD floats of LDS
      int lane;
    };

    // Halves between angle rows in LDS ([hi | lo], padded by 16 bytes so that
    // the 16 rows one read asks for fall in different banks).
    template <int HD>
    constexpr int kAngleRowPitch = 2 * HD + 8;

    // The workgroup's copy of the angle rows [u][hi | lo][HD] (u < 32).
    template <int HD>
    __device__ inline void copy_angle_rows(std::uint16_t *rows, const std::uint16_t *angles)
    {
      constexpr int kChunks = 32 * 2 * HD / 8; // 16 bytes each
      constexpr int kRowChunks = 2 * HD / 8;
      for (int k = threadIdx.x; k < kChunks; k += kThreads)
      {
        const u32x4 v = *((g_u32x4)(angles + 8 * k));
        *reinterpret_cast<u32x4 *>(rows + (k / kRowChunks) * kAngleRowPitch<HD> +
                                   8 * (k % kRowChunks)) = v;
      }
    }

    // Scores (base-2 units) from the two 16-key accumulators, masked past
    // the last key; the page's max and sum over the lane group, its stats,
    // and the running softmax merged; returns P (hi, lo) for P.V. With
    // kEveryPage every page, the first too, takes the merge with no branch
    // (the stream kernel's walk, whose state starts each group at max -inf,
    // sum 0, outputs 0): the rescale factor is exactly 1 wherever a head's
    // maximum did not rise and 0 on a group's first page (exp2(-inf)), and
    // the page's own factor exactly 1 there, so the bits are those of the
    // branches, and the compiler keeps the accumulators in place instead of
    // copying them around them.
    template <int HD, bool kEveryPage = false>
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
      m_page = lane_max32(lane_max16(m_page));
      const float m_from = m_page == -INFINITY ? 0.0f : m_page;
      float pv[8];
      float l_page = 0.0f;
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        pv[e] = exp2_fast(sc[e] - m_from);
        l_page += pv[e];
      }
      l_page = lane_sum32(lane_sum16(l_page));
      if (c.g == 0 && c.r < c.group)
      {
        *reinterpret_cast<float2 *>(c.stat) = make_float2(m_page, l_page);
      }
      float f_page = 1.0f;
      if (!kEveryPage && c.first)
      {
        run.m = m_page;
        run.l = l_page;
      }
      else
      {
        const float m_new = fmaxf(run.m, m_page);
        const float m_new_from = m_new == -INFINITY ? 0.0f : m_new;
        const float f_old = exp2_fast(run.m - m_new_from);
        f_page = exp2_fast(m_page - m_new_from);
        run.l = run.l * f_old + l_page * f_page;
        // o needs rescaling only where this page raised a head's maximum.
        if (kEveryPage || __builtin_amdgcn_ballot_w64(m_page > run.m) != 0)
        {
#pragma unroll
          for (int db = 0; db < HD / 16; ++db)
          {
            run.o[db] *= f_old;
          }
        }
        run.m = m_new;
      }
      const float p_scale = f_page * kPScale;
#pragma unroll
      for (int e = 0; e < 8; ++e)
      {
        _Float16 hi, lo;
        split_half(pv[e] * p_scale, hi, lo);
        p_hi[e] = hi;
        p_lo[e] = lo;
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

    // The per-lane codes and value metadata of one quantised page: rows r
    // and 16 + r, the lane's run of channels.
    template <int HD, int Bits>
    struct QuantRaw
    {
      static constexpr int kRowWords = (HD / 4) * Bits / 8 / 4;
      unsigned kc[2][kRowWords];
      unsigned vc[2][kRowWords];
      unsigned vs[2];
      unsigned vz[2];
    };

    // Adds the key bias's term to a page's scores. The wave turns
    // the bias to the page's first row through its LDS (lane i: angle i), as
    // [b_j | b_j'] and [-b_j' | b_j], so that lane (g, r) forms A (g < 2) or
    // B (g >= 2) of head r as q_j y_j + q_j' y_j' from the first or second
    // copy, over its run of angles j = (g % 2) kRun + 8 s + e, with q_j and
    // q_j' from lanes l and l ^ 32.
    template <int HD>
    __device__ inline void key_bias_scores(f32x4 (&acc)[2], const KeyBias<HD> &b,
                                           const half8 *qb, int r, int g)
    {
      constexpr int S = HD / 32;
      constexpr int kRun = HD / 4;
      constexpr int kHalf = HD / 2;
      // b(t0): b_j cos - b_j' sin, b_j' cos + b_j sin.
      const float turned = b.b * b.turn.x - b.b2 * b.turn.y;
      const float turned2 = b.b2 * b.turn.x + b.b * b.turn.y;
      if (b.lane < kHalf)
      {
        b.lds[b.lane] = turned;
        b.lds[kHalf + b.lane] = turned2;
        b.lds[HD + b.lane] = -turned2;
        b.lds[HD + kHalf + b.lane] = turned;
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
      const float *y = b.lds + (g < 2 ? 0 : HD) + (g & 1) * kRun;
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        const float4 *t1 = reinterpret_cast<const float4 *>(y + 8 * s);
        const float4 *t2 = reinterpret_cast<const float4 *>(y + kHalf + 8 * s);
        const float4 y1a = t1[0], y1b = t1[1], y2a = t2[0], y2b = t2[1];
        const float y1[8] = {y1a.x, y1a.y, y1a.z, y1a.w, y1b.x, y1b.y, y1b.z, y1b.w};
        const float y2[8] = {y2a.x, y2a.y, y2a.z, y2a.w, y2b.x, y2b.y, y2b.z, y2b.w};
        // q_j (the lower lane's) and q_j' (the upper lane's) of the pair.
        const u32x4 own = __builtin_bit_cast(u32x4, qb[s]);
        u32x4 qlo, qhi;
#pragma unroll
        for (int w = 0; w < 4; ++w)
        {
          // (A vector element is copied out before its bits are recast:
          // the compiler recasts the vector's first element otherwise.)
          const unsigned word = own[w];
          float lo, hi;
          lane_pair32(__uint_as_float(word), lo, hi);
          qlo[w] = __float_as_uint(lo);
          qhi[w] = __float_as_uint(hi);
        }
        const half8 q1 = as_half8(qlo), q2 = as_half8(qhi);
        half8 ab_hi, ab_lo;
#pragma unroll
        for (int e = 0; e < 8; ++e)
        {
          // Two mixed-precision fmas, q read as fp16 (q2 y2 rounded once,
          // as a product is).
          const float ab = __builtin_fmaf(static_cast<float>(q1[e]), y1[e],
                                          __builtin_fmaf(static_cast<float>(q2[e]), y2[e], 0.0f));
          _Float16 hi, lo;
          split_half(ab, hi, lo);
          ab_hi[e] = hi;
          ab_lo[e] = lo;
        }
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          const std::uint16_t *row =
              b.rows + (16 * kb + r) * kAngleRowPitch<HD> + g * kRun + 8 * s;
          const half8 e_hi = as_half8(*reinterpret_cast<const u32x4 *>(row));
          const half8 e_lo = as_half8(*reinterpret_cast<const u32x4 *>(row + HD));
          acc[kb] = mfma(e_hi, ab_hi, acc[kb]);
          acc[kb] = mfma(e_hi, ab_lo, acc[kb]);
          acc[kb] = mfma(e_lo, ab_hi, acc[kb]);
        }
      }
    }

    // q.K^T, softmax and P.V of a quantised page from its raw codes, the
    // scores starting from `start`. `ks` and `kz` point at the KV head's key
    // scales and key zeros (HD halves each) in LDS, read 32 channels at a
    // time.
    template <int HD, int Bits, bool kEveryPage = false>
    __device__ inline void quantised_compute(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                             const QuantRaw<HD, Bits> &raw, const unsigned *ks,
                                             const unsigned *kz, const f32x4 (&start)[2])
    {
      constexpr int S = HD / 32;
      constexpr int kRun = HD / 4;
      const int r = c.r, g = c.g;
      f32x4 acc[2] = {start[0], start[1]};
#pragma unroll
      for (int s = 0; s < S; ++s)
      {
        const u32x4 s2 = *reinterpret_cast<const u32x4 *>(ks + (g * kRun + 8 * s) / 2);
        const u32x4 z2 = *reinterpret_cast<const u32x4 *>(kz + (g * kRun + 8 * s) / 2);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          unsigned w0, w1 = 0;
          if constexpr (Bits == 8)
          {
            w0 = raw.kc[kb][2 * s];
            w1 = raw.kc[kb][2 * s + 1];
          }
          else if constexpr (Bits == 4)
          {
            w0 = raw.kc[kb][s];
          }
          else
          {
            w0 = raw.kc[kb][s / 2] >> (16 * (s & 1));
          }
          acc[kb] = mfma(dequant_step<Bits>(w0, w1, s2, z2), qb[s], acc[kb]);
        }
      }
      half8 p_hi, p_lo;
      softmax_page<HD, kEveryPage>(acc, c, run, p_hi, p_lo);
      // Values: one scale and zero a row (token) of this KV head.
      u32x4 sv[2], zv[2];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const unsigned sp = raw.vs[kb] | (raw.vs[kb] << 16), zp = raw.vz[kb] | (raw.vz[kb] << 16);
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
            w0 = raw.vc[kb][2 * s];
            w1 = raw.vc[kb][2 * s + 1];
          }
          else if constexpr (Bits == 4)
          {
            w0 = raw.vc[kb][s];
          }
          else
          {
            w0 = raw.vc[kb][s / 2] >> (16 * (s & 1));
          }
          v[kb] = dequant_step<Bits>(w0, w1, sv[kb], zv[kb]);
        }
        pv_step<HD>(run, s, v[0], v[1], r, g, p_hi, p_lo);
      }
    }

    // A page at INT8/INT4/INT2, read from global memory. `meta` is this
    // wave's 4 * HD bytes of LDS: the key scales and zeros pass through it.
    template <int HD, int Bits, bool kBias = false>
    __device__ inline void quantised_page(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                          const std::uint8_t *page, const PageLayout &L,
                                          std::size_t W, int kvh, int value_kv_heads,
                                          int value_kvh, int lane, unsigned *meta,
                                          const KeyBias<HD> *bias = nullptr)
    {
      using Raw = QuantRaw<HD, Bits>;
      constexpr int kRun = HD / 4;
      constexpr int kRowBytes = Raw::kRowWords * 4;
      constexpr int kMetaLanes = HD / 4; // 8 bytes (4 channels) a lane, a region
      const int r = c.r, g = c.g;
      const std::size_t ch0 = static_cast<std::size_t>(kvh) * HD + g * kRun;
      // Every load first: codes of both rows, the key scales and zeros (two
      // regions, a lane's 8 bytes each), the rows' value scales and zeros.
      Raw raw;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const std::size_t at = (static_cast<std::size_t>(kb * 16 + r) * W + ch0) * Bits / 8;
        load_words<kRowBytes>(raw.kc[kb], page + L.key_codes + at);
        load_words<kRowBytes>(raw.vc[kb], page + L.value_codes + at);
      }
      u32x2 km = {0u, 0u};
      const bool meta_lane = lane < 2 * kMetaLanes;
      if (meta_lane)
      {
        const std::size_t region = lane < kMetaLanes ? L.key_scales : L.key_zeros;
        km = *((g_u32x2)(page + region + 2 * static_cast<std::size_t>(kvh) * HD +
                         8 * (lane % kMetaLanes)));
      }
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const std::size_t grp = static_cast<std::size_t>(kb * 16 + r) * value_kv_heads + value_kvh;
        raw.vs[kb] = *((g_u16)(page + L.value_scales + 2 * grp));
        raw.vz[kb] = *((g_u16)(page + L.value_zeros + 2 * grp));
      }
      // The key bias's scores while the codes are on their way.
      f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      if constexpr (kBias)
      {
        key_bias_scores<HD>(acc, *bias, qb, r, g);
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
      quantised_compute<HD, Bits>(run, c, qb, raw, meta, meta + HD / 2, acc);
    }

    // q.K^T of an FP16 page's two 16-row blocks, added to acc.
    template <int HD>
    __device__ inline void fp16_scores(f32x4 (&acc)[2], const half8 (&k)[2][HD / 32],
                                       const half8 *qb)
    {
#pragma unroll
      for (int s = 0; s < HD / 32; ++s)
      {
        acc[0] = mfma(k[0][s], qb[s], acc[0]);
        acc[1] = mfma(k[1][s], qb[s], acc[1]);
      }
    }

    // P.V of an FP16 page. Rows past the last key may hold anything: their
    // scores are masked, and their values zeroed so that a non-finite one
    // cannot reach P.V.
    template <int HD>
    __device__ inline void fp16_values(Running<HD> &run, const PageCtx &c, half8 (&v)[2][HD / 32],
                                       half8 p_hi, half8 p_lo)
    {
      constexpr int S = HD / 32;
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

    // RoPE of a lane's run of a head's row (HD/4 channels from g HD/4) at
    // one position: the run's raw words and the cos and sin of its angles,
    // asked for first (TurnIn::ask) and turned once they are in (turn). A
    // run's partner channels, hd/2 away, are lane ^ 32's: lane groups 0-1
    // form x1 c - x2 s, groups 2-3 x2 c + x1 s, as rope_pair does.
    template <int HD>
    struct TurnIn
    {
      u32x4 raw[HD / 32];
      f32x4 cs[HD / 8]; // {cos, sin} of two angles a vector

      __device__ void ask(const std::uint16_t *run, const float *table, int position, int g)
      {
        constexpr int kRun = HD / 4;
        const float *angles =
            table + 2 * (static_cast<std::size_t>(position) * (HD / 2) + (g % 2) * kRun);
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
        {
          raw[s] = *((g_u32x4)(run + 8 * s));
        }
#pragma unroll
        for (int i = 0; i < HD / 8; ++i)
        {
          cs[i] = *reinterpret_cast<const f32x4 *>(angles + 4 * i);
        }
      }

      // Lane groups 0-1 hold x1 (own) and need x1 c - x2 s; groups 2-3 hold
      // x2 and need x2 c + x1 s. Both are own c + partner' s, where
      // partner' is x2 with its sign flipped (exact) for groups 0-1 and x1
      // for groups 2-3: the products and the sum round as rope_pair's do.
      __device__ void turn(half8 *dst, const u32x4 *words, int g) const
      {
        const unsigned flip = g < 2 ? 0x80008000u : 0u;
#pragma unroll
        for (int s = 0; s < HD / 32; ++s)
        {
          u32x4 out;
#pragma unroll
          for (int w = 0; w < 4; ++w)
          {
            float lo_word, hi_word;
            lane_pair32(__uint_as_float(words[s][w]), lo_word, hi_word);
            const unsigned own = words[s][w];
            const unsigned partner = __float_as_uint(g < 2 ? hi_word : lo_word) ^ flip;
            const f32x4 a = cs[4 * s + w]; // cos, sin of the word's two angles
            const float r0 = h2f(static_cast<std::uint16_t>(own)) * a[0] +
                             h2f(static_cast<std::uint16_t>(partner)) * a[1];
            const float r1 = h2f(static_cast<std::uint16_t>(own >> 16)) * a[2] +
                             h2f(static_cast<std::uint16_t>(partner >> 16)) * a[3];
            out[w] = static_cast<unsigned>(__half_as_ushort(__float2half(r0))) |
                     (static_cast<unsigned>(__half_as_ushort(__float2half(r1))) << 16);
          }
          dst[s] = as_half8(out);
        }
      }
    };

    // A page of FP16 rows from global memory: keys at k0/k1 (rows r and
    // 16 + r, the lane's run), values at v0/v1, all requested at once so that
    // the page costs one trip to memory. With kCurrent, row `cur_row` (-1:
    // none) is cur_k and cur_v from registers instead.
    struct NoHook
    {
      __device__ void operator()() const {}
    };

    template <int HD, bool kBias = false, bool kCurrent = false, typename Hook = NoHook>
    __device__ inline void fp16_page(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                     const std::uint16_t *k0, const std::uint16_t *k1,
                                     const std::uint16_t *v0, const std::uint16_t *v1,
                                     const KeyBias<HD> *bias = nullptr, int cur_row = -1,
                                     const half8 *cur_k = nullptr, const half8 *cur_v = nullptr,
                                     Hook hook = {})
    {
      constexpr int S = HD / 32;
      half8 k[2][S], v[2][S];
      load_fp16_run<HD>(k[0], k0);
      load_fp16_run<HD>(k[1], k1);
      load_fp16_run<HD>(v[0], v0);
      load_fp16_run<HD>(v[1], v1);
      if constexpr (kCurrent)
      {
        hook(); // work that needs no page byte, while the page's are in flight
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          if (kb * 16 + c.r == cur_row)
          {
#pragma unroll
            for (int s = 0; s < S; ++s)
            {
              k[kb][s] = cur_k[s];
              v[kb][s] = cur_v[s];
            }
          }
        }
      }
      f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      // The key bias's scores while the keys are on their way.
      if constexpr (kBias)
      {
        key_bias_scores<HD>(acc, *bias, qb, c.r, c.g);
      }
      fp16_scores<HD>(acc, k, qb);
      half8 p_hi, p_lo;
      softmax_page<HD>(acc, c, run, p_hi, p_lo);
      fp16_values<HD>(run, c, v, p_hi, p_lo);
    }

    // kCurrent: the row launch's work done here too (the DecodeArgs row_*
    // fields; one split layer, FP16 pages of a cache that does not seal, no
    // key bias, no pack).
    template <int HD, bool kBias, bool kCurrent = false>
    __global__ void __launch_bounds__(kThreads) decode_pages_kernel(DecodeArgs a)
    {
      constexpr int S = HD / 32;  // K steps of q.K^T
      constexpr int DB = HD / 16; // 16-channel blocks of the output
      constexpr int kRun = HD / 4;
      constexpr int kRow = HD + 4;
      extern __shared__ float lds[];

      const int lane = threadIdx.x & 63;
      // Uniform across the wave, as are its pages: their tiers and addresses
      // are scalar loads.
      const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
      const int r = lane & 15;
      const int g = lane >> 4;
      const int split = blockIdx.x;
      const int kvh = blockIdx.y;
      const int li = blockIdx.z;
      const int layer = a.first_layer + li;
      if constexpr (kCurrent)
      {
        // The workgroups past the splits: the first forms RMSNorm(row_x).
        if (split == static_cast<int>(gridDim.x) - 1 && a.row_x != nullptr)
        {
          if (kvh == 0)
          {
            const float scale = inv_rms(a.row_x, a.row_hidden, a.row_eps, lds);
            normed_row(a.row_x, a.row_norm_weight, a.row_normed, a.row_hidden, scale);
          }
          return;
        }
      }
      go_live(a);
      // (The key-bias kernel keeps one split a workgroup: its launches are
      // never bounded.)
      const int busy = !kBias && a.busy_splits > 0 && a.busy_splits < a.live_splits
                           ? a.busy_splits
                           : a.live_splits;
      if (split >= busy)
      {
        return; // past the live pages: the combine reads no partial of this split
      }
      const int G = a.group;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t run0 = static_cast<std::size_t>(kvh) * HD + g * kRun;
      // LDS: each wave's key metadata and turned key bias, then the
      // epilogue's per-wave state.
      unsigned *meta = reinterpret_cast<unsigned *>(lds) + wave * 3 * HD;
      float *s_m = lds + kWaves * 3 * HD;
      float *s_l = s_m + kWaves * G;
      float *s_w = s_l + kWaves * G; // kWaves * G weights, then G maxima
      float *s_o = s_w + kWaves * G + G;

      const unsigned long long *table = a.table + layer * a.table_stride;
      const std::uint8_t *tiers = a.tiers != nullptr ? a.tiers + layer * a.table_stride : nullptr;
      const int own = a.causal ? (a.seq_k - 1) / kPageTokens : -1;
      const int p0 = (split * kWaves + wave) * a.pages_per_wave;
      // The wave's pages: p0 and the next pages_per_wave - 1 (several a
      // wave), or p0 and every kWaves * busy pages on (the pages past the
      // busy splits).
      int p_step = 1, p_count = a.pages_per_wave, p_bound = a.live_pages;
      if constexpr (!kBias)
      {
        if (a.pages_per_wave == 1)
        {
          p_step = kWaves * busy;
          p_count = INT_MAX;
        }
      }
      // A pack's rows: its first KV head's heads, then its second's; lane
      // groups 0-1 hold the first head's 64 channels, 2-3 the second's.
      const int head_row = kvh * G + (r < G ? r : 0);
      const bool pack = a.pack != 0;
      const bool q_off = pack && (r < G ? r : 0) / (G / 2) != g / 2;
      const std::uint16_t *q_row =
          a.q + li * a.q_stride +
          (pack ? static_cast<std::size_t>(head_row) * (HD / 2) + (g % 2) * kRun
                : static_cast<std::size_t>(head_row) * HD + g * kRun);
      // A value row's metadata: the lane's own KV head's.
      const int value_kvh = pack ? 2 * kvh + g / 2 : kvh;
      float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;
      const int SG = a.stat_group;

      Running<HD> run;
      run.m = -INFINITY;
      run.l = 0.0f;
#pragma unroll
      for (int db = 0; db < DB; ++db)
      {
        run.o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }

      // q of head r, the lane's run of channels. Columns past the group
      // repeat the group's first head: their scores and outputs stay in
      // their own columns and are never stored.
      // The zeros are written first and the lanes that keep them do not
      // load: zeroing after the load would wait for it here, before the
      // page table is asked for.
      half8 qb[S];
#pragma unroll
      for (int si = 0; si < S; ++si)
      {
        qb[si] = as_half8(u32x4{0u, 0u, 0u, 0u});
      }
      // The current row (kCurrent): its position, its page and row there,
      // and whether this wave reads that page. q's raw run and angles (and
      // with the page, the row's raw k and its values) are asked for here
      // and turned once the first page's entry is asked for too.
      const int cur_pos = a.seq_k - 1;
      const int cur_page = cur_pos / kPageTokens;
      const int cur_t = cur_pos % kPageTokens;
      half8 cur_k[kCurrent ? S : 1], cur_v[kCurrent ? S : 1];
      u32x4 k_raw[kCurrent ? S : 1];
      TurnIn<kCurrent ? HD : 32> turn_in;
      bool holds_cur = false;
      if constexpr (kCurrent)
      {
        const int ahead = cur_page - p0;
        holds_cur = ahead >= 0 && ahead % p_step == 0 && ahead / p_step < p_count;
        turn_in.ask(q_row, a.row_table, cur_pos, g);
        if (holds_cur)
        {
          const std::uint16_t *k_row =
              a.row_qk + (static_cast<std::size_t>(a.row_q_heads) + kvh) * HD + g * kRun;
#pragma unroll
          for (int si = 0; si < S; ++si)
          {
            k_raw[si] = *((g_u32x4)(k_row + 8 * si));
          }
          load_fp16_run<HD>(cur_v, a.row_v + run0);
        }
      }
      if constexpr (!kCurrent)
      {
        if (!q_off)
        {
          load_fp16_run<HD>(qb, q_row);
        }
      }

      // Where the tiers and addresses are read from: q (always readable)
      // stands in for a table that has no entries (a causal cache with no
      // page sealed yet has no tables at all: both pointers are null).
      const auto *tier_base =
          a.causal && own > 0 ? tiers : reinterpret_cast<const std::uint8_t *>(a.q);
      const auto *page_base =
          !a.causal || own > 0 ? table : reinterpret_cast<const unsigned long long *>(a.q);
      // A page's tier and address, requested together with no branch
      // between them, so that both are one trip to memory. The tier (a
      // byte: a vector load) is made uniform where it is used, so that
      // nothing waits for it before then.
      const auto entry = [&](int p, int &tier_lane, unsigned long long &page_raw) {
        const bool sealed = !a.causal || p < own;
        tier_lane = tier_base[a.causal && p < own ? p : 0];
        page_raw = page_base[sealed ? p : 0];
      };
      // The wave's first page's entry is asked for before the key bias's
      // prologue, whose angle-row copy then shares its trip to memory.
      int first_tier_lane = 0;
      unsigned long long first_page_raw = 0;
      if (p0 < p_bound)
      {
        entry(p0, first_tier_lane, first_page_raw);
      }
      // (kCurrent) q and the current row's k turned, and the turned rows
      // out: split 0's first wave writes q's, the wave that stores the row
      // its k. Run while the wave's first page's bytes are in flight.
      const auto turn_rows = [&]() {
        turn_in.turn(qb, turn_in.raw, g);
        if (holds_cur)
        {
          turn_in.turn(cur_k, k_raw, g);
        }
        if (a.row_qk_out != nullptr && split == 0 && wave == 0 && r < G)
        {
#pragma unroll
          for (int si = 0; si < S; ++si)
          {
            *reinterpret_cast<u32x4 *>(a.row_qk_out + static_cast<std::size_t>(head_row) * HD +
                                       g * kRun + 8 * si) = as_u32x4(qb[si]);
          }
        }
        if (a.row_qk_out != nullptr && holds_cur && r == 0)
        {
#pragma unroll
          for (int si = 0; si < S; ++si)
          {
            *reinterpret_cast<u32x4 *>(a.row_qk_out +
                                       (static_cast<std::size_t>(a.row_q_heads) + kvh) * HD +
                                       g * kRun + 8 * si) = as_u32x4(cur_k[si]);
          }
        }
      };

      // The key bias: lane i holds b_i and b_i' of this KV head; the
      // workgroup's angle rows follow the epilogue's LDS.
      float bias_b = 0.0f, bias_b2 = 0.0f;
      auto *angle_rows = reinterpret_cast<std::uint16_t *>(s_o + kWaves * G * kRow);
      if constexpr (kBias)
      {
        const int i = lane % (HD / 2);
        const std::uint16_t *bh = a.k_bias + static_cast<std::size_t>(kvh) * HD;
        bias_b = static_cast<float>(__builtin_bit_cast(_Float16, bh[i]));
        bias_b2 = static_cast<float>(__builtin_bit_cast(_Float16, bh[HD / 2 + i]));
        copy_angle_rows<HD>(angle_rows, a.rope_angles);
        __syncthreads();
      }
      // The open page's rows, asked for with q, not after the tier.
      const auto *open = a.open_table != nullptr
                             ? reinterpret_cast<const std::uint16_t *>(a.open_table[layer])
                             : a.open;
      if constexpr (kCurrent)
      {
        // FP16 pages of a cache that does not seal: page i of the wave's,
        // its first with the turn while its bytes are in flight (the first
        // page outside the loop, so that the turn's registers end there).
        const auto fp16_at = [&](int i, auto hook) {
          const int p = p0 + i * p_step;
          unsigned long long page_raw = first_page_raw;
          if (i > 0)
          {
            int tier_lane;
            entry(p, tier_lane, page_raw);
          }
          PageCtx c;
          c.r = r;
          c.g = g;
          c.group = G;
          c.last = a.seq_k - 1 - p * kPageTokens;
          c.partial = c.last < kPageTokens - 1;
          c.first = i == 0;
          c.scale = a.scale;
          {
            const int h = kvh * G + r; // rows past the group are never stored
            c.stat = stats + ((static_cast<std::size_t>(h / SG) * a.pages + p) * SG + h % SG) * 2;
          }
          const auto *h = reinterpret_cast<const std::uint16_t *>(page_raw);
          const bool here = holds_cur && p == cur_page;
          fp16_page<HD, false, true>(run, c, qb, h + static_cast<std::size_t>(r) * W + run0,
                                     h + static_cast<std::size_t>(16 + r) * W + run0,
                                     h + static_cast<std::size_t>(kPageTokens + r) * W + run0,
                                     h + static_cast<std::size_t>(kPageTokens + 16 + r) * W + run0,
                                     nullptr, here ? cur_t : -1, cur_k, cur_v, hook);
          // The current row into its page: its four lanes of row cur_t
          // (each row's k and v runs are read by this wave only).
          if (here && (cur_t % 16) == r)
          {
            auto *row = const_cast<std::uint16_t *>(h) + static_cast<std::size_t>(cur_t) * W + run0;
#pragma unroll
            for (int si = 0; si < S; ++si)
            {
              *reinterpret_cast<u32x4 *>(row + 8 * si) = as_u32x4(cur_k[si]);
              *reinterpret_cast<u32x4 *>(row + kPageTokens * W + 8 * si) = as_u32x4(cur_v[si]);
            }
          }
        };
        if (p0 < p_bound)
        {
          fp16_at(0, turn_rows);
          for (int i = 1; i < p_count && p0 + i * p_step < p_bound; ++i)
          {
            fp16_at(i, NoHook{});
          }
        }
      }
      else
      {
        bool first = true;
        for (int i = 0; i < p_count; ++i)
        {
          const int p = p0 + i * p_step;
          if (p >= p_bound)
          {
            break;
          }
          const bool sealed = !a.causal || p < own;
          int tier_lane = first_tier_lane;
          unsigned long long page_raw = first_page_raw;
          if (i > 0)
          {
            entry(p, tier_lane, page_raw);
          }
          const int tier_raw = __builtin_amdgcn_readfirstlane(tier_lane);
          const int tier = !a.causal ? static_cast<int>(kFP16) : (p < own ? tier_raw : kOwnPage);
          const auto *page = reinterpret_cast<const std::uint8_t *>(sealed ? page_raw : 0ull);
          PageCtx c;
          c.r = r;
          c.g = g;
          c.group = G;
          c.last = a.seq_k - 1 - p * kPageTokens;
          c.partial = c.last < kPageTokens - 1;
          c.first = first;
          c.scale = a.scale;
          {
            const int h = kvh * G + r; // rows past the group are never stored
            c.stat = stats + ((static_cast<std::size_t>(h / SG) * a.pages + p) * SG + h % SG) * 2;
          }
          KeyBias<HD> bias;
          if constexpr (kBias)
          {
            bias.b = bias_b;
            bias.b2 = bias_b2;
            bias.lds = reinterpret_cast<float *>(meta + HD);
            bias.lane = lane;
            // cos and sin of the lane's angle at the page's first row.
            bias.turn = *reinterpret_cast<const float2 *>(
                a.rope + 2 * (static_cast<std::size_t>(p) * kPageTokens * (HD / 2) + lane % (HD / 2)));
            bias.rows = angle_rows;
          }
          const KeyBias<HD> *page_bias = &bias;
          if (tier == kUnreadPage)
          {
            if (g == 0 && r < G)
            {
              *reinterpret_cast<float2 *>(c.stat) = make_float2(-INFINITY, 0.0f);
            }
            continue;
          }
          switch (tier)
          {
          case kINT8:
            quantised_page<HD, 8, kBias>(run, c, qb, page, a.lay[kINT8], W, kvh,
                                           a.value_kv_heads, value_kvh, lane, meta, page_bias);
            break;
          case kINT4:
            quantised_page<HD, 4, kBias>(run, c, qb, page, a.lay[kINT4], W, kvh,
                                           a.value_kv_heads, value_kvh, lane, meta, page_bias);
            break;
          case kINT2:
            quantised_page<HD, 2, kBias>(run, c, qb, page, a.lay[kINT2], W, kvh,
                                           a.value_kv_heads, value_kvh, lane, meta, page_bias);
            break;
          case kOwnPage:
          {
            // Rows before `start` from the open page, the rest from the chunk;
            // rows past the last key read row 0 (masked).
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
            fp16_page<HD, kBias>(run, c, qb, rk[0], rk[1], rv[0], rv[1], page_bias);
            break;
          }
          default:
          {
            const auto *h = reinterpret_cast<const std::uint16_t *>(page);
            fp16_page<HD, kBias>(run, c, qb, h + static_cast<std::size_t>(r) * W + run0,
                          h + static_cast<std::size_t>(16 + r) * W + run0,
                          h + static_cast<std::size_t>(kPageTokens + r) * W + run0,
                          h + static_cast<std::size_t>(kPageTokens + 16 + r) * W + run0, page_bias);
            break;
          }
          }
          first = false;
        }
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
              s_o[(wave * G + r) * kRow + out_channel<HD>(s, h, g, i2)] =
                  run.o[2 * s + h][i2] * kPUnscale;
            }
          }
        }
      }
      __syncthreads();
      if (static_cast<int>(threadIdx.x) < kWaves * G)
      {
        const int h = threadIdx.x % G;
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
          top = fmaxf(top, s_m[w * G + h]);
        }
        const float from = top == -INFINITY ? 0.0f : top;
        s_w[threadIdx.x] = exp2_fast(s_m[threadIdx.x] - from);
        if (static_cast<int>(threadIdx.x) < G)
        {
          s_w[kWaves * G + h] = top;
        }
      }
      __syncthreads();
      // A head's partial: its HD channels, or with a pack its own KV head's
      // HD / 2 of the unit's.
      constexpr int kPackHD = HD / 2;
      const int out_hd = pack ? kPackHD : HD;
      float *part = a.partials +
                    ((static_cast<std::size_t>(li) * a.kv_heads + kvh) * a.splits + split) * G * out_hd;
      float *ml = a.split_ml + (static_cast<std::size_t>(li) * a.kv_heads + kvh) * G * a.splits * 2;
      for (int idx = threadIdx.x; idx < G * (out_hd + 2); idx += kThreads)
      {
        const int h = idx / (out_hd + 2);
        const int col = idx % (out_hd + 2);
        const int from = col - 2 + (pack && h >= G / 2 ? kPackHD : 0); // unit channel
        float acc = s_w[kWaves * G + h];
        if (col != 0)
        {
          acc = 0.0f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w)
          {
            const float v = col == 1 ? s_l[w * G + h] : s_o[(w * G + h) * kRow + from];
            acc += v * s_w[w * G + h];
          }
        }
        if (col < 2)
        {
          ml[(static_cast<std::size_t>(h) * a.splits + split) * 2 + col] = acc;
        }
        else
        {
          part[h * out_hd + col - 2] = acc;
        }
      }
      // Splits past the busy ones: empty partials (max -inf, sum and
      // outputs 0), which weigh nothing where they are folded.
      for (int empty = busy + split; !kBias && empty < a.live_splits; empty += busy)
      {
        float *epart = a.partials +
                       ((static_cast<std::size_t>(li) * a.kv_heads + kvh) * a.splits + empty) * G * out_hd;
        for (int idx = threadIdx.x; idx < G * (out_hd + 2); idx += kThreads)
        {
          const int h = idx / (out_hd + 2);
          const int col = idx % (out_hd + 2);
          if (col < 2)
          {
            ml[(static_cast<std::size_t>(h) * a.splits + empty) * 2 + col] =
                col == 0 ? -INFINITY : 0.0f;
          }
          else
          {
            epart[h * out_hd + col - 2] = 0.0f;
          }
        }
      }
    }

    // LDS of decode_pages_kernel, bytes.
    std::size_t pages_kernel_lds(int group, int hd, bool bias)
    {
      const std::size_t angle_rows = bias ? 32 * (2 * hd + 8) * sizeof(std::uint16_t) : 0;
      return (static_cast<std::size_t>(kWaves) * 3 * hd + 3 * kWaves * group + group +
              static_cast<std::size_t>(kWaves) * group * (hd + 4)) *
                 sizeof(float) +
             angle_rows;
    }

    // ---- the streaming kernel: several layers in one launch ----------------

    typedef __attribute__((address_space(3))) void *lds_void;
    // Word 3 of a raw buffer descriptor on gfx9-family parts (gfx950).
    constexpr int kBufferWord3 = 0x00020000;
    typedef const __attribute__((address_space(1))) void *global_void;

    // A direct global-to-LDS copy (global_load_lds): lane l's 16 bytes land
    // at block + 16 l; `block` must be wave-uniform.
    __device__ inline void dma16(const void *src, void *block)
    {
      __builtin_amdgcn_global_load_lds((global_void)src, (lds_void)block, 16, 0, 0);
    }
    // s_waitcnt vmcnt(0): every copy into LDS has landed.
    __device__ inline void wait_copies()
    {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // s_waitcnt lgkmcnt(0): every LDS read has returned, so its slot may be
    // overwritten.
    __device__ inline void wait_reads()
    {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    __device__ inline u32x4 lds16(const void *block, int lane)
    {
      return *reinterpret_cast<const u32x4 *>(static_cast<const std::uint8_t *>(block) + 16 * lane);
    }
    __device__ inline unsigned lds4(const void *block, int lane)
    {
      return *reinterpret_cast<const unsigned *>(static_cast<const std::uint8_t *>(block) + 4 * lane);
    }

    // Where a quantised page's pieces sit in a wave's LDS slot. Codes go in
    // 1 KiB blocks of 16 bytes a lane when a lane's row run is a multiple of
    // 16 bytes, else in 256-byte blocks of 4 bytes a lane; both in the order
    // the lanes read them. Then the KV head's key scales, key zeros (a
    // 256-byte block each) and the page's value scales and zeros.
    template <int HD, int Bits>
    struct SlotLayout
    {
      static constexpr int kRowWords = QuantRaw<HD, Bits>::kRowWords;
      static constexpr bool kWide = kRowWords % 4 == 0;
      static constexpr int kBlocksARow = kWide ? kRowWords / 4 : kRowWords;
      static constexpr int kBlock = kWide ? 1024 : 256;
      static constexpr int kCodes = 4 * kBlocksARow * kBlock; // K rows r, 16+r; V rows
      static constexpr int kKeyScales = kCodes;
      static constexpr int kKeyZeros = kCodes + 256;
      static constexpr int kValueMeta = kCodes + 512;
    };

    // The bytes of one (page, KV head) unit a wave's slot must hold, and the
    // slot's size: an FP16 unit (4 rows of the lane's run, 16 bytes a lane a
    // step) is the largest.
    template <int HD>
    constexpr int stream_slot_bytes()
    {
      return 4 * (HD / 32) * 1024;
    }

    struct Unit
    {
      int li;    // layer within the launch
      int block; // KV-head block: heads [block * ways, (block + 1) * ways)
      int page;
      int kvh;   // the wave's KV head of the block
    };

    __device__ inline Unit unit_of(long long u, int blocks, int pages, int ways, int way)
    {
      const long long group = u / pages;
      const int block = static_cast<int>(group % blocks);
      return {static_cast<int>(group / blocks), block, static_cast<int>(u - group * pages),
              block * ways + way};
    }

    // The unit after u in a range: the next page, or the next group's first.
    __device__ inline void next_unit(Unit &u, int blocks, int pages, int ways)
    {
      if (++u.page == pages)
      {
        u.page = 0;
        if (++u.block == blocks)
        {
          u.block = 0;
          ++u.li;
        }
        u.kvh = u.block * ways + u.kvh % ways;
      }
    }

    // Range of wave w: units [w U / W, (w+1) U / W) (in 32 bits where the
    // product fits).
    __host__ __device__ inline long long range_start(long long w, long long units, int waves)
    {
      const unsigned long long top = static_cast<unsigned long long>(w) * units;
      return top <= 0xFFFFFFFFull
                 ? static_cast<long long>(static_cast<unsigned>(top) / static_cast<unsigned>(waves))
                 : static_cast<long long>(top / static_cast<unsigned long long>(waves));
    }

    // The wave whose range holds unit x: the largest w < waves with
    // floor(w units / waves) <= x, i.e. w units < (x + 1) waves, so
    // w = ((x + 1) waves - 1) / units (waves <= units). One division, in 32
    // bits where the product fits (the scalar unit divides 64-bit values in
    // software).
    __host__ __device__ inline int wave_of(long long x, long long units, int waves)
    {
      const unsigned long long top = static_cast<unsigned long long>(x + 1) * waves - 1;
      const unsigned long long w =
          top <= 0xFFFFFFFFull && units <= 0xFFFFFFFFll
              ? static_cast<unsigned>(top) / static_cast<unsigned>(units)
              : top / static_cast<unsigned long long>(units);
      return static_cast<int>(w < static_cast<unsigned long long>(waves) ? w : waves - 1);
    }

    // The first unit of (layer li, KV head kvh)'s group in the streaming
    // launch's unit order.
    __host__ __device__ inline long long group_base(const DecodeArgs &a, int li, int kvh)
    {
      const int blocks = a.kv_heads / a.stream_ways;
      return (static_cast<long long>(li) * blocks + kvh / a.stream_ways) * a.pages;
    }

    // Splits of (layer li, KV head kvh): fixed, or the streaming ranges that
    // meet its pages.
    __host__ __device__ inline int group_splits(const DecodeArgs &a, int li, int kvh)
    {
      if (a.stream_ranges == 0)
      {
        return a.splits;
      }
      const long long base = group_base(a, li, kvh);
      return wave_of(base + a.pages - 1, a.stream_units, a.stream_ranges) -
             wave_of(base, a.stream_units, a.stream_ranges) + 1;
    }

    // Issues the copies of unit `u` (address `page`, tier `tier`) into `slot`.
    template <int HD>
    __device__ inline void stream_copy(const DecodeArgs &a, const Unit &u, const std::uint8_t *page,
                                       int tier, std::uint8_t *slot, int lane)
    {
      constexpr int S = HD / 32;
      constexpr int kRun = HD / 4;
      const int r = lane & 15, g = lane >> 4;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t run0 = static_cast<std::size_t>(u.kvh) * HD + g * kRun;
      const auto quantised = [&](auto bits_tag) {
        constexpr int Bits = decltype(bits_tag)::value;
        using SL = SlotLayout<HD, Bits>;
        const PageLayout &L = a.lay[Bits == 8 ? kINT8 : Bits == 4 ? kINT4 : kINT2];
        // One buffer over the page (reads past it return zeros); each lane's
        // row offset once, the regions and rows as scalar offsets, the steps
        // as immediates.
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<std::uint8_t *>(page), 0, static_cast<int>(L.page_bytes), kBufferWord3);
        const int lane_row = static_cast<int>((r * W + run0) * Bits / 8);
        const int row16 = static_cast<int>(16 * W * Bits / 8);
#pragma unroll
        for (int half = 0; half < 2; ++half) // keys, values
        {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
          {
            const int region =
                static_cast<int>(half == 0 ? L.key_codes : L.value_codes) + kb * row16;
#pragma unroll
            for (int i = 0; i < SL::kBlocksARow; ++i)
            {
              std::uint8_t *block = slot + ((half * 2 + kb) * SL::kBlocksARow + i) * SL::kBlock;
              if constexpr (SL::kWide)
              {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)block, 16, lane_row,
                                                         region + 16 * i, 0, 0);
              }
              else
              {
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)block, 4, lane_row,
                                                         region + 4 * i, 0, 0);
              }
            }
          }
        }
        // Key scales and zeros of this KV head: HD halves each, 4 bytes a lane.
        const int meta_off = 4 * (lane % (HD / 2));
        const int kvh_meta = 2 * u.kvh * HD;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)(slot + SL::kKeyScales), 4, meta_off,
                                                 static_cast<int>(L.key_scales) + kvh_meta, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)(slot + SL::kKeyZeros), 4, meta_off,
                                                 static_cast<int>(L.key_zeros) + kvh_meta, 0, 0);
        // Value scales then value zeros, all KV heads: 64 * kv bytes each,
        // contiguous in the page (zeros follow scales).
        const int words = 16 * a.kv_heads;
        for (int b = 0; b < (2 * words + 63) / 64; ++b)
        {
          const int w = b * 64 + lane;
          const int wc = w < 2 * words ? w : 2 * words - 1;
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)(slot + SL::kValueMeta + 256 * b),
                                                   4, 4 * wc, static_cast<int>(L.value_scales),
                                                   0, 0);
        }
      };
      if (tier != kOwnPage && tier >= kINT8 && tier <= kINT2)
      {
        switch (tier)
        {
        case kINT8:
          quantised(std::integral_constant<int, 8>{});
          break;
        case kINT4:
          quantised(std::integral_constant<int, 4>{});
          break;
        default:
          quantised(std::integral_constant<int, 2>{});
          break;
        }
        return;
      }
      if (tier != kOwnPage)
      {
        // FP16 rows: keys r, 16+r then values r, 16+r, the lane's run, a
        // 16-byte step at a time, through one buffer over the page.
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<std::uint8_t *>(page), 0, static_cast<int>(4 * kPageTokens * W),
            kBufferWord3);
        const int lane_row = static_cast<int>((r * W + run0) * 2);
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
          const int row = static_cast<int>(((j / 2) * kPageTokens + (j % 2) * 16) * W * 2);
#pragma unroll
          for (int st = 0; st < S; ++st)
          {
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void)(slot + (j * S + st) * 1024), 16,
                                                     lane_row, row + 16 * st, 0, 0);
          }
        }
        return;
      }
      // The own page: rows before `start` from the open page, the rest from
      // the chunk; rows past the last key read row 0.
      const int layer = a.first_layer + u.li;
      const auto *open = a.open_table != nullptr
                             ? reinterpret_cast<const std::uint16_t *>(a.open_table[layer])
                             : a.open;
      const int last = a.seq_k - 1 - u.page * kPageTokens;
      const int t_start = a.start - u.page * kPageTokens;
      const std::uint16_t *ck = a.chunk_k + u.li * a.chunk_stride;
      const std::uint16_t *cv = a.chunk_v + u.li * a.chunk_stride;
      const std::uint16_t *rows[4];
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const int t = kb * 16 + r;
        const int tt = t <= last ? t : 0;
        if (tt < t_start)
        {
          rows[kb] = open + static_cast<std::size_t>(tt) * W + run0;
          rows[2 + kb] = open + static_cast<std::size_t>(kPageTokens + tt) * W + run0;
        }
        else
        {
          rows[kb] = ck + static_cast<std::size_t>(tt - t_start) * W + run0;
          rows[2 + kb] = cv + static_cast<std::size_t>(tt - t_start) * W + run0;
        }
      }
#pragma unroll
      for (int j = 0; j < 4; ++j)
      {
#pragma unroll
        for (int st = 0; st < S; ++st)
        {
          dma16(rows[j] + 8 * st, slot + (j * S + st) * 1024);
        }
      }
    }

    // Reads a quantised unit's codes and value metadata from the slot.
    template <int HD, int Bits>
    __device__ inline void stream_read_quantised(QuantRaw<HD, Bits> &raw, const std::uint8_t *slot,
                                                 int lane, int kvh, int kv_heads)
    {
      using SL = SlotLayout<HD, Bits>;
      const int r = lane & 15;
#pragma unroll
      for (int half = 0; half < 2; ++half)
      {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
        {
          unsigned *dst = half == 0 ? raw.kc[kb] : raw.vc[kb];
#pragma unroll
          for (int i = 0; i < SL::kBlocksARow; ++i)
          {
            const std::uint8_t *block =
                slot + ((half * 2 + kb) * SL::kBlocksARow + i) * SL::kBlock;
            if constexpr (SL::kWide)
            {
              const u32x4 v = lds16(block, lane);
              dst[4 * i + 0] = v.x;
              dst[4 * i + 1] = v.y;
              dst[4 * i + 2] = v.z;
              dst[4 * i + 3] = v.w;
            }
            else
            {
              dst[i] = lds4(block, lane);
            }
          }
        }
      }
      const auto *vmeta = reinterpret_cast<const std::uint16_t *>(slot + SL::kValueMeta);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const int grp = (kb * 16 + r) * kv_heads + kvh;
        raw.vs[kb] = vmeta[grp];
        raw.vz[kb] = vmeta[32 * kv_heads + grp];
      }
    }

    // Writes a wave's running softmax as the partial of its group's split.
    template <int HD>
    __device__ inline void stream_flush(const DecodeArgs &a, const Running<HD> &run, int li, int kvh,
                                        int split, int r, int g)
    {
      const int G = a.group;
      if (r >= G)
      {
        return;
      }
      float *part = a.partials +
                    (((static_cast<std::size_t>(li) * a.kv_heads + kvh) * a.splits + split) * G + r) * HD;
      if (g == 0)
      {
        *reinterpret_cast<float2 *>(
            a.split_ml +
            (((static_cast<std::size_t>(li) * a.kv_heads + kvh) * G + r) * a.splits + split) * 2) =
            make_float2(run.m, run.l);
      }
#pragma unroll
      for (int s = 0; s < HD / 32; ++s)
      {
#pragma unroll
        for (int h = 0; h < 2; ++h)
        {
          *reinterpret_cast<f32x4 *>(part + out_channel<HD>(s, h, g, 0)) =
              run.o[2 * s + h] * kPUnscale;
        }
      }
    }

    // A quantised unit from the slot: codes and value metadata to registers,
    // the key scales and zeros to the wave's metadata area (out of the
    // slot), then `next` (which reuses the slot), then the arithmetic.
    template <int HD, int Bits, typename Next>
    __device__ inline void stream_quantised(Running<HD> &run, const PageCtx &c, const half8 *qb,
                                            const std::uint8_t *slot, std::uint8_t *meta,
                                            int lane, int kvh, int kv_heads, const Next &next)
    {
      using SL = SlotLayout<HD, Bits>;
      QuantRaw<HD, Bits> raw;
      stream_read_quantised<HD, Bits>(raw, slot, lane, kvh, kv_heads);
      const u32x2 km = *reinterpret_cast<const u32x2 *>(slot + SL::kKeyScales + 8 * lane);
      *reinterpret_cast<u32x2 *>(meta + 8 * lane) = km;
      next();
      const f32x4 zero[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
      quantised_compute<HD, Bits, true>(run, c, qb, raw, reinterpret_cast<const unsigned *>(meta),
                                        reinterpret_cast<const unsigned *>(meta + 256), zero);
    }

    // Each range of (layer, KV-head block, page) units (at most 64 of them)
    // is walked by `ways` waves of a workgroup, one KV head of the block
    // each, with one unit in flight a wave: the next unit's bytes are copied
    // into the wave's LDS slot by global_load_lds while the current one,
    // already in registers, is computed. A wave writes one partial per group
    // it touches.
    template <int HD>
    __global__ void __launch_bounds__(kThreads) decode_stream_kernel(DecodeArgs a)
    {
      constexpr int S = HD / 32;
      constexpr int DB = HD / 16;
      constexpr int kRun = HD / 4;
      extern __shared__ float lds[];
      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int r = lane & 15;
      const int g = lane >> 4;
      const int G = a.group;
      const int ways = a.stream_ways;
      const int way = wave % ways;
      const int blocks = a.kv_heads / ways;
      const int gw = blockIdx.x * (kWaves / ways) + wave / ways; // the range
      if (gw >= a.stream_ranges)
      {
        return;
      }
      const long long u0 = range_start(gw, a.stream_units, a.stream_ranges);
      const long long u1 = range_start(gw + 1, a.stream_units, a.stream_ranges);
      const int n = static_cast<int>(u1 - u0);
      if (n <= 0)
      {
        return;
      }
      std::uint8_t *slot = reinterpret_cast<std::uint8_t *>(lds) + wave * stream_slot_bytes<HD>();
      std::uint8_t *meta =
          reinterpret_cast<std::uint8_t *>(lds) + kWaves * stream_slot_bytes<HD>() + wave * 512;
      const int own = a.causal ? (a.seq_k - 1) / kPageTokens : -1;

      // Every unit's address and tier, a lane a unit, read once.
      unsigned long long my_addr = 0;
      int my_tier = kFP16;
      if (lane < n)
      {
        const Unit u = unit_of(u0 + lane, blocks, a.pages, ways, way);
        const long long at = static_cast<long long>(a.first_layer + u.li) * a.table_stride + u.page;
        if (a.causal)
        {
          my_tier = u.page < own ? static_cast<int>(a.tiers[at]) : kOwnPage;
        }
        if (my_tier != kUnreadPage && my_tier != kOwnPage)
        {
          my_addr = a.table[at];
        }
      }
      const auto addr_of = [&](int i) {
        return reinterpret_cast<const std::uint8_t *>(
            (static_cast<unsigned long long>(__builtin_amdgcn_readlane(
                 static_cast<unsigned>(my_addr >> 32), i))
             << 32) |
            static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<unsigned>(my_addr), i)));
      };
      const auto tier_of = [&](int i) { return __builtin_amdgcn_readlane(my_tier, i); };

      Running<HD> run;
      run.m = -INFINITY;
      run.l = 0.0f;
#pragma unroll
      for (int db = 0; db < DB; ++db)
      {
        run.o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }
      half8 qb[S];
      int seg_group = -1;
      bool first = true;

      {
        const int t = tier_of(0);
        if (t != kUnreadPage)
        {
          stream_copy<HD>(a, unit_of(u0, blocks, a.pages, ways, way), addr_of(0), t, slot, lane);
        }
      }
      Unit u = unit_of(u0, blocks, a.pages, ways, way);
      for (int i = 0; i < n; ++i)
      {
        if (i > 0)
        {
          next_unit(u, blocks, a.pages, ways);
        }
        const int group = u.li * a.kv_heads + u.kvh;
        if (group != seg_group)
        {
          seg_group = group;
          first = true;
          const std::uint16_t *q_row =
              a.q + u.li * a.q_stride + static_cast<std::size_t>(u.kvh * G + (r < G ? r : 0)) * HD +
              g * kRun;
          // Zeros first, and only the group's lanes load (zeroing after
          // the load would wait for it before the unit's page is asked for).
#pragma unroll
          for (int s = 0; s < S; ++s)
          {
            qb[s] = as_half8(u32x4{0u, 0u, 0u, 0u});
          }
          if (r < G)
          {
            load_fp16_run<HD>(qb, q_row);
          }
        }
        const int tier = tier_of(i);
        PageCtx c;
        c.r = r;
        c.g = g;
        c.group = G;
        c.last = a.seq_k - 1 - u.page * kPageTokens;
        c.partial = c.last < kPageTokens - 1;
        c.first = first;
        c.scale = a.scale;
        c.stat = a.page_stats +
                 (((static_cast<std::size_t>(u.li) * a.kv_heads + u.kvh) * a.pages + u.page) * G + r) *
                     2;
        // The next unit's copies go out as soon as this one is out of LDS.
        const auto next = [&]() {
          wait_reads();
          if (i + 1 < n)
          {
            const int t = tier_of(i + 1);
            if (t != kUnreadPage)
            {
              Unit v = u;
              next_unit(v, blocks, a.pages, ways);
              stream_copy<HD>(a, v, addr_of(i + 1), t, slot, lane);
            }
          }
        };
        wait_copies();
        switch (tier)
        {
        case kUnreadPage:
          next();
          if (g == 0 && r < G)
          {
            *reinterpret_cast<float2 *>(c.stat) = make_float2(-INFINITY, 0.0f);
          }
          break;
        case kINT8:
          stream_quantised<HD, 8>(run, c, qb, slot, meta, lane, u.kvh, a.kv_heads, next);
          first = false;
          break;
        case kINT4:
          stream_quantised<HD, 4>(run, c, qb, slot, meta, lane, u.kvh, a.kv_heads, next);
          first = false;
          break;
        case kINT2:
          stream_quantised<HD, 2>(run, c, qb, slot, meta, lane, u.kvh, a.kv_heads, next);
          first = false;
          break;
        default:
        {
          half8 k[2][S], v[2][S];
#pragma unroll
          for (int j = 0; j < 4; ++j)
          {
#pragma unroll
            for (int st = 0; st < S; ++st)
            {
              const half8 x = as_half8(lds16(slot + (j * S + st) * 1024, lane));
              if (j < 2)
              {
                k[j][st] = x;
              }
              else
              {
                v[j - 2][st] = x;
              }
            }
          }
          next();
          f32x4 acc[2] = {{0.0f, 0.0f, 0.0f, 0.0f}, {0.0f, 0.0f, 0.0f, 0.0f}};
          fp16_scores<HD>(acc, k, qb);
          half8 p_hi, p_lo;
          softmax_page<HD, true>(acc, c, run, p_hi, p_lo);
          fp16_values<HD>(run, c, v, p_hi, p_lo);
          first = false;
          break;
        }
        }
        // The group's last unit in this wave's range: its partial.
        const bool group_ends = i + 1 == n || u.page + 1 == a.pages;
        if (group_ends)
        {
          const int split =
              gw - wave_of(group_base(a, u.li, u.kvh), a.stream_units, a.stream_ranges);
          if (first)
          {
            // Every unit of the segment was unread: an empty partial.
            run.m = -INFINITY;
            run.l = 0.0f;
#pragma unroll
            for (int db = 0; db < DB; ++db)
            {
              run.o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            }
          }
          stream_flush<HD>(a, run, u.li, u.kvh, split, r, g);
          run.m = -INFINITY;
          run.l = 0.0f;
#pragma unroll
          for (int db = 0; db < DB; ++db)
          {
            run.o[db] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
        }
      }
    }

    // LDS of decode_stream_kernel, bytes: a slot and a metadata area a wave.
    template <int HD>
    constexpr std::size_t stream_kernel_lds()
    {
      return static_cast<std::size_t>(kWaves) * (stream_slot_bytes<HD>() + 512);
    }

    constexpr int kCombineThreads = 256;
    constexpr int kWarmBlocks = 8; // one an XCD
    constexpr int kQuads = 16;                                // 4-channel quads a block
    constexpr int kSplitRows = kCombineThreads / kQuads;      // splits read side by side
    constexpr int kSplitsAhead = 8;                           // a thread's loads before any use

    // Folds (m, l) into a running (max, sum), both softmax partials in base 2.
    __device__ inline void fold_partial(float &top, float &sum, float m, float l)
    {
      const float next = fmaxf(top, m);
      const float from = next == -INFINITY ? 0.0f : next;
      sum = sum * exp2_fast(top - from) + l * exp2_fast(m - from);
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

    // The same over the whole wave, as a uniform value: the four rows'
    // results read out of lanes 0, 16, 32 and 48 (no LDS round trip).
    __device__ inline float lane_value(float v, int lane)
    {
      return __builtin_bit_cast(float,
                                __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
    }
    __device__ inline float wave_max(float v)
    {
      v = row16_max(v);
      return fmaxf(fmaxf(lane_value(v, 0), lane_value(v, 16)),
                   fmaxf(lane_value(v, 32), lane_value(v, 48)));
    }
    __device__ inline float wave_sum(float v)
    {
      v = row16_sum(v);
      return (lane_value(v, 0) + lane_value(v, 16)) + (lane_value(v, 32) + lane_value(v, 48));
    }

    // Blocks x < heads * HD/64: 64 output channels of one head. A split's
    // 64 channels are 16 threads' float4 loads (coalesced), 16 splits side
    // by side, and every thread issues the loads of its next 8 splits before
    // it uses any: the partials come from other XCDs' writes, a far round
    // trip away, so the block's whole read is one trip. Indices past the
    // last split are clamped to it and weighted zero, so no load is
    // conditional. Blocks past that: 256 pages' masses and the layer's scores
    // (importance_scores.cu:31-50: heads summed in order, every operation
    // rounded once). blockIdx.y is the launch's layer.
    // A step's page seal (one workgroup): when the step's position is its
    // page's last row, the page -- rows 0..30 from the open page, the last
    // from the step's k and v -- quantised at its tier (copied at FP16) into
    // its slot, a task a lane (page_tasks.hpp), as the store's seal does.
    template <int HD>
    __device__ inline void seal_step_page(const StepStore &s)
    {
      const int position = *s.position;
      if (position % kPageTokens != kPageTokens - 1)
      {
        return;
      }
      const int page = position / kPageTokens;
      const int W = s.kv_heads * HD;
      const int tier = s.tiers[page];
      RowJob j{};
      j.kind = static_cast<int>(tier == kFP16 ? RowJobKind::kCopy : RowJobKind::kQuantise);
      j.k_lo = s.open;
      j.v_lo = s.open + static_cast<std::size_t>(kPageTokens) * W;
      j.k_hi = s.keys;
      j.v_hi = s.values;
      j.split = kPageTokens - 1;
      j.dst = reinterpret_cast<std::uint8_t *>(s.addresses[page]);
      j.tier = tier;
      for (int task = threadIdx.x; task < W; task += kCombineThreads)
      {
        page_tasks::run_row_task<HD>(j, s.lay, task, s.kv_heads);
      }
    }

    template <int HD, bool Streamed>
    __global__ void __launch_bounds__(kCombineThreads) decode_combine_kernel(const DecodeArgs args)
    {
      if constexpr (!Streamed)
      {
        // The seal reads the launch's own (constant) arguments: its index
        // into the layouts, taken from memory, would otherwise pin the
        // combine's mutable copy below to private memory.
        if (args.seal_block != 0 && static_cast<int>(blockIdx.x) == args.seal_block - 1)
        {
          seal_step_page<HD>(args.seal);
          return;
        }
      }
      DecodeArgs a = args;
      // Fixed splits unless the streaming kernel wrote the partials: the
      // per-layer form carries none of the streaming geometry's code.
      go_live(a);
      const auto splits_of = [&](int li, int kvh) {
        return Streamed ? group_splits(a, li, kvh) : a.live_splits;
      };
      constexpr int kBlocksAHead = HD / (4 * kQuads);
      __shared__ f32x4 s_o[kSplitRows][kQuads];
      __shared__ float s_m[kSplitRows];
      __shared__ float s_l[kSplitRows];
      __shared__ float s_share[kMaxHeads][64];
      const int G = a.group;
      const int li = blockIdx.y;
      const int t = threadIdx.x;
      const int bx = static_cast<int>(blockIdx.x) + a.block_base;
      // Head h's split outputs (split s at s * split_stride) and its splits'
      // (max, sum) pairs, side by side.
      const auto head_out = [&](int h) {
        return a.partials +
               ((static_cast<std::size_t>(li) * a.kv_heads + h / G) * a.splits * G + h % G) * HD;
      };
      const auto head_ml = [&](int h) {
        return reinterpret_cast<const float2 *>(a.split_ml) +
               (static_cast<std::size_t>(li) * a.heads + h) * a.splits;
      };
      const std::size_t split_stride = static_cast<std::size_t>(G) * HD;
      if (bx < a.heads * kBlocksAHead)
      {
        const int h = bx / kBlocksAHead;
        const int c0 = (bx % kBlocksAHead) * 4 * kQuads;
        const int quad = t % kQuads;
        const int row = t / kQuads;
        const int splits = splits_of(li, h / G);
        const float *base = head_out(h);
        const float2 *mls = head_ml(h);
        float top = -INFINITY, l = 0.0f;
        f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
        const auto fold_from = [&](int s0) {
          float mv[kSplitsAhead], lv[kSplitsAhead];
          f32x4 ov[kSplitsAhead];
#pragma unroll
          for (int i = 0; i < kSplitsAhead; ++i)
          {
            const int s = min(s0 + i * kSplitRows, splits - 1);
            const float2 ml = mls[s];
            mv[i] = ml.x;
            lv[i] = ml.y;
            ov[i] = *reinterpret_cast<const f32x4 *>(base + s * split_stride + c0 + 4 * quad);
          }
          float next = top;
#pragma unroll
          for (int i = 0; i < kSplitsAhead; ++i)
          {
            if (s0 + i * kSplitRows < splits)
            {
              next = fmaxf(next, mv[i]);
            }
          }
          const float from = next == -INFINITY ? 0.0f : next;
          const float keep = exp2_fast(top - from);
          acc *= keep;
          l *= keep;
#pragma unroll
          for (int i = 0; i < kSplitsAhead; ++i)
          {
            const float w = s0 + i * kSplitRows < splits ? exp2_fast(mv[i] - from) : 0.0f;
            acc += ov[i] * w;
            l += lv[i] * w;
          }
          top = next;
        };
        // The first kSplitRows * kSplitsAhead splits outside the loop, so
        // that their loads are not held behind a loop head's wait.
        fold_from(row);
        for (int s0 = row + kSplitRows * kSplitsAhead; s0 < splits;
             s0 += kSplitRows * kSplitsAhead)
        {
          fold_from(s0);
        }
        // The rows into one: every row's share at the rows' common max.
        s_o[row][quad] = acc;
        if (quad == 0)
        {
          s_m[row] = top;
          s_l[row] = l;
        }
        __syncthreads();
        if (t < kQuads)
        {
          float all = -INFINITY;
#pragma unroll
          for (int u = 0; u < kSplitRows; ++u)
          {
            all = fmaxf(all, s_m[u]);
          }
          const float from = all == -INFINITY ? 0.0f : all;
          f32x4 sum = {0.0f, 0.0f, 0.0f, 0.0f};
          float total = 0.0f;
#pragma unroll
          for (int u = 0; u < kSplitRows; ++u)
          {
            const float w = exp2_fast(s_m[u] - from);
            sum += s_o[u][t] * w;
            total += s_l[u] * w;
          }
          unsigned short hv[4];
#pragma unroll
          for (int i = 0; i < 4; ++i)
          {
            hv[i] = __half_as_ushort(__float2half(sum[i] / total));
          }
          std::uint16_t *dst =
              a.out + li * a.out_stride + static_cast<std::size_t>(h) * HD + c0 + 4 * t;
          if (reinterpret_cast<std::uintptr_t>(dst) % 8 == 0)
          {
            *reinterpret_cast<u32x2 *>(dst) = u32x2{hv[0] | (static_cast<unsigned>(hv[1]) << 16),
                                                    hv[2] | (static_cast<unsigned>(hv[3]) << 16)};
          }
          else
          {
#pragma unroll
            for (int i = 0; i < 4; ++i)
            {
              dst[i] = hv[i];
            }
          }
        }
        return;
      }
      if (bx >= a.heads * kBlocksAHead + a.mass_blocks)
      {
        // A warm block: the next layer's tiers and page addresses through
        // this XCD's caches (workgroups go to the XCDs in turn, so the
        // kWarmBlocks consecutive blocks cover them all).
        unsigned fold = 0;
        for (int i = t; i < a.warm_count; i += kCombineThreads)
        {
          fold ^= a.warm_tiers[i] ^ static_cast<unsigned>(a.warm_table[i]);
        }
        // The reads are for their side effect on the caches: an empty asm
        // that takes the folded value keeps the compiler from dropping them.
        asm volatile("" ::"v"(fold));
        return;
      }
      // A mass block: 64 pages, a wave a head at a time (heads w, w + 4, ...):
      // the wave requests its heads' split pairs (one coalesced 512-byte read
      // each) and the pages' (max, sum) together, forms each head's total,
      // and leaves each page's share in LDS; then wave 0 sums a page's shares
      // in head order and folds the score.
      const int lane = t & 63;
      const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
      constexpr int kWavesC = kCombineThreads / 64;
      constexpr int kHeadsAWave = kMaxHeads / kWavesC;
      const int first_page = (bx - a.heads * kBlocksAHead) * 64;
      if (first_page >= a.live_pages || (a.score_every > 1 && a.seq_k % a.score_every != 0))
      {
        return; // no live page here, or not a step the scores take
      }
      const int page = first_page + lane;
      const bool has_page = page < a.live_pages;
      const int pg = has_page ? page : a.live_pages - 1; // clamped: loads, never stores
      const float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;
      float *scores = a.scores != nullptr ? a.scores + li * a.scores_stride : nullptr;
      float *mass = a.mass != nullptr ? a.mass + li * a.mass_stride : nullptr;
      const float old = scores != nullptr && wave == 0 ? scores[pg] : 0.0f;
      for (int j0 = 0; j0 < kHeadsAWave && wave + kWavesC * j0 < a.heads; j0 += 4)
      {
        float2 st[4], ml[4][2];
        int splits[4];
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
          const int h = min(wave + kWavesC * (j0 + j), a.heads - 1);
          splits[j] = splits_of(li, h / G);
          const int SG = a.stat_group;
          st[j] = *reinterpret_cast<const float2 *>(
              stats + ((static_cast<std::size_t>(h / SG) * a.pages + pg) * SG + h % SG) * 2);
          const float2 *mls = head_ml(h);
#pragma unroll
          for (int k = 0; k < 2; ++k)
          {
            ml[j][k] = mls[min(lane + 64 * k, splits[j] - 1)];
          }
        }
#pragma unroll
        for (int j = 0; j < 4; ++j)
        {
          const int h = wave + kWavesC * (j0 + j);
          if (h >= a.heads)
          {
            break;
          }
          float top = -INFINITY, sum = 0.0f;
#pragma unroll
          for (int k = 0; k < 2; ++k)
          {
            if (lane + 64 * k < splits[j])
            {
              fold_partial(top, sum, ml[j][k].x, ml[j][k].y);
            }
          }
          // More than 128 splits only when several layers share a launch.
          const float2 *mls = head_ml(h);
          for (int sp = lane + 128; sp < splits[j]; sp += 64)
          {
            const float2 v = mls[sp];
            fold_partial(top, sum, v.x, v.y);
          }
          const float all = wave_max(top);
          const float from = all == -INFINITY ? 0.0f : all;
          const float whole = wave_sum(sum * exp2_fast(top - from));
          const float share = st[j].y * exp2_fast(st[j].x - from) / whole;
          s_share[h][lane] = share;
          if (mass != nullptr && has_page)
          {
            mass[static_cast<std::size_t>(h) * a.live_pages + page] = share;
          }
        }
      }
      __syncthreads();
      if (wave == 0 && has_page && scores != nullptr)
      {
        float total = 0.0f;
        for (int h = 0; h < a.heads; ++h)
        {
          total = __fadd_rn(total, s_share[h][lane]);
        }
        const float observed = __fdiv_rn(total, static_cast<float>(a.heads));
        scores[page] = ewma_step(old, observed, a.alpha);
      }
    }

    // Where a launch's scratch comes from: the caller's workspace source,
    // else the caller's partials buffer when it is known to be large enough,
    // else the stream's library buffer.
    float *decode_scratch(const AttentionArgs &a, std::size_t floats, hipStream_t stream)
    {
      if (a.workspace != nullptr)
      {
        return a.workspace->floats(floats);
      }
      if (a.partials != nullptr && a.partials_floats >= floats)
      {
        return a.partials;
      }
      return stream_workspace(stream, floats);
    }

    bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

    // Waves of the head_dim-64 pages kernel (a wave a page of one KV head)
    // that the current device holds at once, for a workgroup's LDS of `lds`
    // bytes: whole workgroups a CU times the CUs.
    long long resident_pages_waves_64(std::size_t lds)
    {
      static std::mutex lock;
      static std::map<std::pair<int, std::size_t>, long long> known;
      int device = 0;
      hip_check(hipGetDevice(&device), "hipGetDevice");
      std::lock_guard<std::mutex> guard(lock);
      const auto key = std::make_pair(device, lds);
      const auto found = known.find(key);
      if (found != known.end())
      {
        return found->second;
      }
      int blocks = 0;
      hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(
                    &blocks, reinterpret_cast<const void *>(decode_pages_kernel<64, false>),
                    kThreads, lds),
                "hipOccupancyMaxActiveBlocksPerMultiprocessor decode");
      int cus = 0;
      hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                "hipDeviceGetAttribute CUs");
      const long long waves = static_cast<long long>(std::max(blocks, 1)) * kWaves * cus;
      known.emplace(key, waves);
      return waves;
    }

    // Workgroups of a pages-kernel variant the current device holds at once
    // with `lds` bytes of LDS each: whole workgroups a CU times the CUs.
    long long resident_pages_blocks(const void *kernel, std::size_t lds)
    {
      static std::mutex lock;
      static std::map<std::tuple<int, const void *, std::size_t>, long long> known;
      int device = 0;
      hip_check(hipGetDevice(&device), "hipGetDevice");
      std::lock_guard<std::mutex> guard(lock);
      const auto key = std::make_tuple(device, kernel, lds);
      const auto found = known.find(key);
      if (found != known.end())
      {
        return found->second;
      }
      int blocks = 0;
      hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, kThreads, lds),
                "hipOccupancyMaxActiveBlocksPerMultiprocessor decode pages");
      int cus = 0;
      hip_check(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device),
                "hipDeviceGetAttribute CUs");
      const long long held = static_cast<long long>(std::max(blocks, 1)) * cus;
      known.emplace(key, held);
      return held;
    }

  } // namespace

  float *stream_workspace(hipStream_t stream, std::size_t count)
  {
    struct Held
    {
      float *buffer = nullptr;
      std::size_t count = 0;
    };
    static std::mutex lock;
    static std::map<hipStream_t, Held> held;
    static std::vector<float *> retired; // kept: a captured graph may hold one
    std::lock_guard<std::mutex> guard(lock);
    Held &h = held[stream];
    if (count > h.count)
    {
      if (h.buffer != nullptr)
      {
        retired.push_back(h.buffer);
      }
      const std::size_t grown = std::max<std::size_t>(count, 1 << 20);
      float *buffer = nullptr;
      hip_check(hipMalloc(reinterpret_cast<void **>(&buffer), grown * sizeof(float)),
                "hipMalloc decode workspace");
      h.buffer = buffer;
      h.count = grown;
    }
    return h.buffer;
  }

  bool decode_fast_applies(const KVSource &kv, const AttentionArgs &a)
  {
    if (a.seq_q != 1 || kv.layout == Layout::kContiguous ||
        kv.page_tokens != kPageTokens || (a.head_dim != 64 && a.head_dim != 128) ||
        a.kv_heads <= 0 || a.heads % a.kv_heads != 0 || a.heads / a.kv_heads > kMaxGroup ||
        a.heads > kMaxHeads || a.seq_k <= 0)
    {
      return false;
    }
    // The key bias: with the table over every key position and its first
    // page's angles.
    if (a.k_bias != nullptr && (a.rope == nullptr || a.rope_angles == nullptr ||
                                a.rope_positions < a.seq_k || !aligned16(a.rope_angles)))
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
    // The key bias, one layer's, on the one-layer launch only.
    if (a.k_bias != nullptr && (ls.layers != 1 || a.rope == nullptr || a.rope_angles == nullptr))
    {
      throw InvalidArgument("decode: the key bias needs one layer and the RoPE table's angles");
    }
    d.k_bias = a.k_bias;
    d.rope = a.k_bias != nullptr ? a.rope : nullptr;
    d.rope_angles = a.k_bias != nullptr ? a.rope_angles : nullptr;
    d.start = kv.start;
    d.causal = kv.layout == Layout::kCausal;
    d.seq_k = a.seq_k;
    d.heads = a.heads;
    d.kv_heads = a.kv_heads;
    d.group = group;
    d.value_kv_heads = a.kv_heads;
    d.stat_group = group;
    d.pages = pages;
    // Scores in base-2 units: the softmax weights are exp2 of them.
    d.scale = static_cast<float>(1.4426950408889634 / std::sqrt(static_cast<double>(a.head_dim)));
    // One layer: a page a wave, so a launch has a wave for every page of
    // every KV head (or, unsplit, one workgroup a KV head). Several layers:
    // the streaming kernel, equal ranges of units a wave.
    const bool streaming = ls.split && ls.layers > 1;
    if (ls.live_seq_k != nullptr && (!ls.split || ls.layers != 1))
    {
      throw InvalidArgument("a decode whose position lives on the device is one split layer");
    }
    d.live_seq_k = ls.live_seq_k;
    d.score_every = 1;
    if (ls.seal != nullptr)
    {
      if (ls.live_seq_k == nullptr || !ls.split || ls.layers != 1)
      {
        throw InvalidArgument("a step's seal rides with one split layer whose position lives on "
                              "the device");
      }
      d.seal = *ls.seal;
      for (int t = kINT8; t <= kINT2; ++t)
      {
        d.seal.lay[t] = page_layout(t, kPageTokens, d.seal.kv_heads, a.head_dim);
      }
    }
    const RowPrep *row = ls.row;
    if (row != nullptr)
    {
      if (!ls.split || ls.layers != 1 || ls.live_seq_k != nullptr || ls.seal != nullptr ||
          ls.keep_ml != nullptr || kv.layout != Layout::kPaged || a.k_bias != nullptr ||
          a.mass != nullptr || a.scores != nullptr || row->head_dim != a.head_dim ||
          row->kv_heads != a.kv_heads || row->q_heads != a.heads || row->qk != a.q ||
          row->table == nullptr || row->table_positions < a.seq_k || row->values == nullptr ||
          !aligned16(row->values) || !aligned16(row->table) ||
          (row->qk_out != nullptr && !aligned16(row->qk_out)) ||
          (row->x != nullptr &&
           (row->norm_weight == nullptr || row->normed == nullptr || row->hidden <= 0)))
      {
        throw InvalidArgument("the pages launch takes the row launch's work for one split layer "
                              "of FP16 pages with no key bias, mass or scores, q and k rows of "
                              "the cache's shape, 16-byte aligned rows and a RoPE table covering "
                              "the current position");
      }
      d.row_qk = row->qk;
      d.row_qk_out = row->qk_out;
      d.row_v = row->values;
      d.row_table = row->table;
      d.row_q_heads = row->q_heads;
      d.row_x = row->x;
      d.row_norm_weight = row->norm_weight;
      d.row_normed = row->normed;
      d.row_hidden = row->hidden;
      d.row_eps = row->eps;
    }
    int stream_blocks = 0;
    if (streaming)
    {
      // A range's waves: as many of the KV heads as divide a workgroup.
      const int ways = std::gcd(a.kv_heads, kWaves);
      const long long units = static_cast<long long>(ls.layers) * (a.kv_heads / ways) * pages;
      const int per_cu = 1; // 2 waves a SIMD (registers); LDS holds a slot a wave
      long long ranges = static_cast<long long>(device_multiprocessors()) * per_cu * kWaves / ways;
      ranges = std::max(ranges, (units + 63) / 64); // at most 64 units a range
      ranges = std::min(ranges, units);             // no range without a unit
      d.stream_units = units;
      d.stream_ranges = static_cast<int>(ranges);
      d.stream_ways = ways;
      const long long per_block = kWaves / ways;
      stream_blocks = static_cast<int>((ranges + per_block - 1) / per_block);
      d.pages_per_wave = 0;
      d.splits = 1;
      for (int li = 0; li < ls.layers; ++li)
      {
        for (int kvh = 0; kvh < a.kv_heads; ++kvh)
        {
          d.splits = std::max(d.splits, group_splits(d, li, kvh));
        }
      }
    }
    else if (ls.split)
    {
      d.pages_per_wave = 1;
      d.splits = (pages + kWaves - 1) / kWaves;
    }
    else
    {
      d.pages_per_wave = (pages + kWaves - 1) / kWaves;
      d.splits = 1;
    }
    d.live_pages = pages;
    d.live_splits = d.splits;
    // head_dim 64 with an even number of KV heads and no key bias (the
    // Llama shapes): two KV heads a wave, as one 128-channel unit, so that a
    // launch has half the waves, each with a unit of the size the kernel's
    // fixed costs are paid for. Only where a wave a KV head would not all be
    // resident at once: below that, halving the waves halves the launch's
    // parallelism (Qwen2.5-0.5B at 8K: 6.8 us a layer unpacked, 9.9 packed).
    const bool packed =
        !streaming && row == nullptr && a.head_dim == 64 && d.k_bias == nullptr &&
        a.kv_heads % 2 == 0 &&
        2 * group <= kMaxGroup &&
        static_cast<long long>(pages) * a.kv_heads * ls.layers >
            resident_pages_waves_64(pages_kernel_lds(group, 64, false));
    if (packed)
    {
      d.pack = 2;
      d.kv_heads = a.kv_heads / 2;
      d.group = 2 * group;
    }
    const std::size_t part =
        static_cast<std::size_t>(ls.layers) * a.kv_heads * d.splits * group * a.head_dim;
    const bool kept = ls.keep_ml != nullptr;
    const std::size_t ml =
        kept ? 0 : static_cast<std::size_t>(ls.layers) * a.kv_heads * group * d.splits * 2;
    const std::size_t stats = kept ? 0 : static_cast<std::size_t>(ls.layers) * a.heads * pages * 2;
    float *ws = decode_scratch(a, part + ml + stats, stream);
    d.partials = ws;
    // Kept statistics (a decode whose fold comes later) go where the caller
    // keeps them; otherwise they are scratch after the partials.
    d.split_ml = kept ? ls.keep_ml : ws + part;
    d.page_stats = kept ? ls.keep_stats : ws + part + ml;
    if (kept && (a.mass != nullptr || a.scores != nullptr || ls.layers != 1 || !ls.split))
    {
      throw InvalidArgument("a decode that keeps its statistics for a later fold is one split "
                            "layer with no mass or scores of its own");
    }
    const int mass_blocks = (a.mass != nullptr || a.scores != nullptr) ? (pages + 63) / 64 : 0;
    d.mass_blocks = mass_blocks;
    const bool warm = kv.warm_pages != nullptr && ls.layers == 1;
    d.warm_table = warm ? kv.warm_pages : nullptr;
    d.warm_tiers = warm ? kv.warm_tiers : nullptr;
    d.warm_count = warm ? kv.warm_count : 0;
    const auto run = [&](auto pages_kernel, auto stream_kernel, auto combine_kernel,
                         auto combine_streamed, int hd, std::size_t stream_lds,
                         int pages_hd) {
      if (stream_blocks > 0)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(stream_kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(stream_lds)),
                  "hipFuncSetAttribute decode stream LDS");
        hipLaunchKernelGGL(stream_kernel, dim3(stream_blocks), dim3(kThreads), stream_lds, stream,
                           d);
        hip_check(hipGetLastError(), "decode stream kernel launch");
      }
      else
      {
        const std::size_t lds = pages_kernel_lds(d.group, pages_hd, d.k_bias != nullptr);
        if (lds > 64 * 1024)
        {
          hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(pages_kernel),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)),
                    "hipFuncSetAttribute decode LDS");
        }
        // One layer split a page a wave (no key bias): no more workgroups a
        // KV head than the device holds at once (past that, second pages
        // for some waves).
        int grid_splits = d.splits;
        if (ls.split && d.k_bias == nullptr)
        {
          const long long per = resident_pages_blocks(reinterpret_cast<const void *>(pages_kernel),
                                                      lds) /
                                (static_cast<long long>(d.kv_heads) * ls.layers);
          if (per < d.splits)
          {
            d.busy_splits = static_cast<int>(std::max<long long>(per, 1));
            grid_splits = d.busy_splits;
          }
        }
        // With the row's RMSNorm: one more column of workgroups (the first
        // forms it; the rest end at once).
        const int norm_splits = row != nullptr && row->x != nullptr ? 1 : 0;
        hipLaunchKernelGGL(pages_kernel, dim3(grid_splits + norm_splits, d.kv_heads, ls.layers),
                           dim3(kThreads), lds, stream, d);
        hip_check(hipGetLastError(), "decode pages kernel launch");
      }
      const int combine_blocks = a.heads * (hd / (4 * kQuads)) + mass_blocks +
                                 (warm ? kWarmBlocks : 0);
      d.seal_block = ls.seal != nullptr ? combine_blocks + 1 : 0;
      hipLaunchKernelGGL(stream_blocks > 0 ? combine_streamed : combine_kernel,
                         dim3(combine_blocks + (ls.seal != nullptr ? 1 : 0), ls.layers),
                         dim3(kCombineThreads), 0, stream, d);
      hip_check(hipGetLastError(), "decode combine kernel launch");
    };
    if (row != nullptr)
    {
      if (a.head_dim == 128)
      {
        run(decode_pages_kernel<128, false, true>, decode_stream_kernel<128>,
            decode_combine_kernel<128, false>, decode_combine_kernel<128, true>, 128,
            stream_kernel_lds<128>(), 128);
      }
      else
      {
        run(decode_pages_kernel<64, false, true>, decode_stream_kernel<64>,
            decode_combine_kernel<64, false>, decode_combine_kernel<64, true>, 64,
            stream_kernel_lds<64>(), 64);
      }
    }
    else if (a.head_dim == 128)
    {
      if (d.k_bias != nullptr)
      {
        run(decode_pages_kernel<128, true>, decode_stream_kernel<128>,
            decode_combine_kernel<128, false>, decode_combine_kernel<128, true>, 128,
            stream_kernel_lds<128>(), 128);
      }
      else
      {
        run(decode_pages_kernel<128, false>, decode_stream_kernel<128>,
            decode_combine_kernel<128, false>, decode_combine_kernel<128, true>, 128,
            stream_kernel_lds<128>(), 128);
      }
    }
    else if (packed)
    {
      // The pack's unit is 128 channels; each head's output is its own 64.
      run(decode_pages_kernel<128, false>, decode_stream_kernel<64>,
          decode_combine_kernel<64, false>, decode_combine_kernel<64, true>, 64,
          stream_kernel_lds<64>(), 128);
    }
    else if (d.k_bias != nullptr)
    {
      run(decode_pages_kernel<64, true>, decode_stream_kernel<64>, decode_combine_kernel<64, false>,
          decode_combine_kernel<64, true>, 64, stream_kernel_lds<64>(), 64);
    }
    else
    {
      run(decode_pages_kernel<64, false>, decode_stream_kernel<64>,
          decode_combine_kernel<64, false>, decode_combine_kernel<64, true>, 64,
          stream_kernel_lds<64>(), 64);
    }
  }

  std::size_t decode_kept_floats(int heads, int kv_heads, int seq_k)
  {
    const int pages = (seq_k + kPageTokens - 1) / kPageTokens;
    const int splits = (pages + kWaves - 1) / kWaves;
    (void)kv_heads;
    return static_cast<std::size_t>(heads) * splits * 2 + static_cast<std::size_t>(heads) * pages * 2;
  }

  void launch_decode_fold(const DecodeFold &f, hipStream_t stream)
  {
    if (f.layers <= 0)
    {
      return;
    }
    DecodeArgs d{};
    const int pages = (f.seq_k + kPageTokens - 1) / kPageTokens;
    d.heads = f.heads;
    d.kv_heads = f.kv_heads;
    d.group = f.heads / f.kv_heads;
    d.value_kv_heads = f.kv_heads;
    d.stat_group = d.group;
    d.pages = pages;
    d.seq_k = f.seq_k;
    d.splits = (pages + kWaves - 1) / kWaves;
    d.split_ml = f.kept;
    d.page_stats = f.kept + static_cast<std::size_t>(f.layers) * f.heads * d.splits * 2;
    d.mass = f.mass;
    d.mass_stride = f.mass_stride;
    d.scores = f.scores;
    d.scores_stride = f.scores_stride;
    d.alpha = f.alpha;
    d.live_seq_k = f.live_seq_k;
    d.live_pages = pages;
    d.live_splits = d.splits;
    d.pages_per_wave = 1;
    d.score_every = std::max(1, f.score_every);
    d.mass_blocks = (pages + 63) / 64;
    const int blocks_a_head = f.head_dim / (4 * kQuads);
    d.block_base = f.heads * blocks_a_head;
    const auto kernel = f.head_dim == 128 ? decode_combine_kernel<128, false>
                                          : decode_combine_kernel<64, false>;
    hipLaunchKernelGGL(kernel, dim3(d.mass_blocks, f.layers), dim3(kCombineThreads), 0, stream, d);
    hip_check(hipGetLastError(), "decode fold kernel launch");
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
