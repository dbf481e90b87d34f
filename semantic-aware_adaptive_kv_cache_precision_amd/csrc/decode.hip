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
//   - a wave64 owns one 32-token page of a *pack* of NP KV heads, NP chosen
//     so that the pack's query heads (NP x group) fill the 16 columns of a
//     16x16x32 f16 MFMA as far as they go: each page's softmax and its
//     bookkeeping are paid once for the pack, not once a KV head;
//   - q.K^T: the page's keys are the MFMA's rows. Lane group g (lane / 16)
//     holds the contiguous channels [g W'/4, (g+1) W'/4) of the pack's
//     W' = NP hd channels of two key rows, so its codes arrive as whole
//     16-byte (or 8- or 4-byte) global loads straight into registers. A lane
//     group's channels belong to one KV head, so q enters as a block-diagonal
//     operand: zero where a column's head is not that KV head's;
//   - codes are dequantised in registers with packed fp16 arithmetic: bytes
//     spliced into the fp16 1024 + code by v_perm, 1024 subtracted, then one
//     fp16 fma with the scale and zero. The reference forms code * scale +
//     zero in fp32 and rounds that to fp16; rounding the exact value once to
//     fp16 differs from it only where the fp32 value lands on an fp16 tie,
//     by one fp16 ulp;
//   - P.V needs V with the keys along each lane's eight MFMA operands: V
//     goes global -> LDS by direct DMA (global_load_lds), laid out so that
//     gfx950's transposing LDS reads (ds_read_b64_tr_b16 / _b8 / _b4) hand
//     every lane eight consecutive keys of one channel, each read instruction
//     covering one contiguous 512-byte run (no bank conflicts). INT8 and INT4
//     codes are transposed as codes and dequantised after, with each key's
//     value scale and zero; INT2 (no 2-bit transpose exists) is dequantised
//     in rows and written to LDS as fp16 first;
//   - scores are kept in base-2 units (scale * log2 e folded in), so the
//     softmax weights are single exp2 instructions; P is split into an fp16
//     high and low part, two MFMAs, keeping ~22 bits of P;
//   - a wave walks a contiguous run of pages of one (layer, pack) with one
//     page in flight: the next page's K codes (to registers), metadata and V
//     (to LDS) are requested before the current page's P.V is computed;
//   - a workgroup of 8 waves owns a contiguous page range of one (layer,
//     pack) and folds its waves into one partial (m, l, o) per head in LDS;
//     the combine kernel folds the partials, and turns each page's
//     (max, sum) into its mass and the layer's scores.

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
    typedef short i16x4 __attribute__((ext_vector_type(4)));
    typedef int i32x2 __attribute__((ext_vector_type(2)));
    // Global-address-space views: loads through them are global_load_*.
    typedef const __attribute__((address_space(1))) u32x4 *g_u32x4;
    typedef const __attribute__((address_space(1))) u32x2 *g_u32x2;
    typedef const __attribute__((address_space(1))) unsigned *g_u32;
    typedef __attribute__((address_space(3))) void *lds_void;
    typedef __attribute__((address_space(3))) i16x4 *lds_i16x4;
    typedef __attribute__((address_space(3))) i32x2 *lds_i32x2;
    typedef const __attribute__((address_space(1))) void *global_void;

    constexpr int kWaves = 8;
    constexpr int kThreads = 64 * kWaves;
    constexpr int kPageTokens = 32;
    constexpr int kMaxGroup = 16;
    constexpr int kMaxHeads = 64;
    constexpr int kMaxKvHeads = 16;
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
      int splits;   // workgroups a (layer, pack): blockIdx.x
      float scale;  // 1/sqrt(hd) * log2 e: scores in base-2 units
      float *partials;   // [launch layer][kv_heads][splits][group][kSlotHead + hd]
      float *page_stats; // [launch layer][heads][pages][2]: each page's max and sum
    };

    __device__ inline half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

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
    constexpr int kSlotHead = 32;

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

    // Eight INT4 codes of one word (nibble t the t-th) in the order
    // (0, 4, 1, 5, 2, 6, 3, 7): one mask-and-merge a pair, no reordering.
    // s2/z2 pair the scales the same way.
    __device__ inline half8 dequant_int4_interleaved(unsigned w, u32x4 s2, u32x4 z2)
    {
      u32x4 out;
      out[0] = dq2((w & 0x000F000Fu) | 0x64006400u, s2[0], z2[0]);
      out[1] = dq2(((w >> 4) & 0x000F000Fu) | 0x64006400u, s2[1], z2[1]);
      out[2] = dq2(((w >> 8) & 0x000F000Fu) | 0x64006400u, s2[2], z2[2]);
      out[3] = dq2(((w >> 12) & 0x000F000Fu) | 0x64006400u, s2[3], z2[3]);
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

    // Direct global-to-LDS copies (global_load_lds): lane l's 16 (or 4)
    // bytes land at block + 16 l (4 l); `block` must be wave-uniform.
    __device__ inline void dma16(const void *src, void *block)
    {
      __builtin_amdgcn_global_load_lds((global_void)src, (lds_void)block, 16, 0, 0);
    }
    __device__ inline void dma4(const void *src, void *block)
    {
      __builtin_amdgcn_global_load_lds((global_void)src, (lds_void)block, 4, 0, 0);
    }
    // s_waitcnt vmcnt(0): every load, to registers or into LDS, has landed.
    __device__ inline void wait_copies()
    {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_waitcnt(0x0F70);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // s_waitcnt lgkmcnt(0): every LDS access has completed, so the slot may
    // be overwritten.
    __device__ inline void wait_reads()
    {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_s_waitcnt(0xC07F);
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
    // Orders this wave's LDS writes before its later LDS reads (LDS
    // operations of one wave are performed in order; this keeps the
    // compiler from moving them).
    __device__ inline void lds_order()
    {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }

    // The lane index, opaque to the compiler: address arithmetic derived from
    // it inside the page loop stays there instead of being hoisted out and
    // held in registers across the loop, one set per tier.
    __device__ inline int opaque(int v)
    {
      asm volatile("" : "+v"(v));
      return v;
    }

    // Global loads from a wave-uniform base plus a 32-bit per-lane offset
    // (the scalar-base form of global_load).
    template <int Bytes>
    __device__ inline void load_at(unsigned *w, const std::uint8_t *base, unsigned offset)
    {
      load_words<Bytes>(w, base + offset);
    }

    __device__ inline u32x2 tr16(const std::uint8_t *p)
    {
      return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(p)));
    }
    __device__ inline u32x2 tr8(const std::uint8_t *p)
    {
      return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr8_b64_v2i32((lds_i32x2)(p)));
    }
    __device__ inline u32x2 tr4(const std::uint8_t *p)
    {
      return __builtin_bit_cast(u32x2, __builtin_amdgcn_ds_read_tr4_b64_v2i32((lds_i32x2)(p)));
    }

    // Sizes of one (HD, NP) instantiation. W' = NP * HD channels a page row
    // of the pack.
    template <int HD, int NP>
    struct Cfg
    {
      static constexpr int kWp = NP * HD;
      static constexpr int kRun = kWp / 4;         // channels a lane group holds of a row
      static constexpr int kSteps = kRun / 8;      // q.K^T steps of 32 channels
      static constexpr int kCB = HD / 16;          // 16-channel output blocks
      static constexpr int kVBytes = NP * HD * 64; // V as fp16: 32 rows of W' halves
      static constexpr int kKMeta = 4 * NP * HD;   // key scales, then key zeros, of the pack
      static constexpr int kRaw = NP * HD / 4;     // words of a lane's two FP16 key rows
      static constexpr int kVt = NP * HD / 4;      // words of a lane's transposed FP16 V
    };

    // The key row behind MFMA row m (0..15) of key block kb. C's rows 4g..4g+3
    // of both blocks then hold keys 8g..8g+7 in the order P.V reads them:
    // natural, or (0, 4, 1, 5, 2, 6, 3, 7) for an INT4 page, whose values
    // dequantise in that order.
    template <bool Interleaved>
    __device__ inline int key_of(int m, int kb)
    {
      const int i = m & 3;
      const int j = Interleaved ? (i & 1) * 4 + (i >> 1) + 2 * kb : 4 * kb + i;
      return 8 * (m >> 2) + j;
    }

    // Where key t sits in the FP16 V image: the 16 keys of one half h
    // ((t / 4) % 2) together, so a transposing read of one half is one run.
    __device__ inline int fp16_image_row(int t)
    {
      return 16 * ((t >> 2) & 1) + 4 * (t >> 3) + (t & 3);
    }
    __device__ inline int fp16_image_key(int row)
    {
      return 8 * ((row >> 2) & 3) + 4 * (row >> 4) + (row & 3);
    }

    // The running softmax of one wave over its pages, for the lane's column.
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
      int g;
      bool live;    // the lane's column is one of the pack's heads
      int last;     // the page's last valid row
      bool partial; // rows past `last` exist on this page (natural key order)
      bool first;   // the wave's first page: it starts the running softmax
      float scale;
      float *stat;  // this page's (max, sum) slot for the lane's head
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
          if (8 * c.g + e > c.last)
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
        pv[e] = exp2_fast(sc[e] - m_from);
        l_page += pv[e];
      }
      l_page += __shfl_xor(l_page, 16);
      l_page += __shfl_xor(l_page, 32);
      if (c.g == 0 && c.live)
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
        const float f_old = exp2_fast(run.m - m_new_from);
        f_page = exp2_fast(m_page - m_new_from);
        run.l = run.l * f_old + l_page * f_page;
        // o needs rescaling only where this page raised a head's maximum.
        if (__builtin_amdgcn_ballot_w64(m_page > run.m) != 0)
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
        const float pe = pv[e] * p_scale;
        const _Float16 hi = static_cast<_Float16>(pe);
        p_hi[e] = hi;
        p_lo[e] = static_cast<_Float16>(pe - static_cast<float>(hi));
      }
    }

    // The rows one unit (a page of a pack) is read from.
    struct Rows
    {
      const std::uint8_t *page;     // sealed page (any tier)
      const std::uint16_t *open;    // own page: rows before t_start
      const std::uint16_t *chunk_k; // own page: rows from t_start
      const std::uint16_t *chunk_v;
      int t_start;
      int last;
    };

    // Key row t of an FP16 unit (a sealed page, or the own page: the open page
    // before t_start, the chunk from there; rows past `last` read row 0).
    __device__ inline const std::uint16_t *key_row(const Rows &u, int tier, int t, std::size_t W)
    {
      if (tier != kOwnPage)
      {
        return reinterpret_cast<const std::uint16_t *>(u.page) + static_cast<std::size_t>(t) * W;
      }
      const int tt = t <= u.last ? t : 0;
      return tt < u.t_start ? u.open + static_cast<std::size_t>(tt) * W
                            : u.chunk_k + static_cast<std::size_t>(tt - u.t_start) * W;
    }
    __device__ inline const std::uint16_t *value_row(const Rows &u, int tier, int t, std::size_t W)
    {
      if (tier != kOwnPage)
      {
        return reinterpret_cast<const std::uint16_t *>(u.page) +
               static_cast<std::size_t>(kPageTokens + t) * W;
      }
      const int tt = t <= u.last ? t : 0;
      return tt < u.t_start ? u.open + static_cast<std::size_t>(kPageTokens + tt) * W
                            : u.chunk_v + static_cast<std::size_t>(tt - u.t_start) * W;
    }

    // The per-wave LDS of one instantiation: V image, key metadata, value
    // metadata (all KV heads' value scales then zeros).
    template <int HD, int NP>
    struct Slot
    {
      std::uint8_t *v;
      std::uint8_t *kmeta;
      std::uint8_t *vmeta;
    };

    // The pack's value scales and zeros: for each of the 32 keys, the
    // dwords holding the pack's NP halves (one dword when NP is 1 or 2).
    template <int NP>
    constexpr int value_meta_dwords() { return NP > 2 ? NP / 2 : 1; }

    template <int HD, int NP>
    __host__ __device__ constexpr int slot_bytes()
    {
      return Cfg<HD, NP>::kVBytes + Cfg<HD, NP>::kKMeta + 256 * value_meta_dwords<NP>();
    }

    // Requests the LDS part of unit `u` at `tier`: the pack's key metadata
    // and every value scale and zero to the slot's metadata, V to the slot's
    // image (INT8, INT4, FP16). No registers are held while these fly.
    template <int HD, int NP>
    __device__ inline void issue_lds(const DecodeArgs &a, const Rows &u, int tier, int kp,
                                     const Slot<HD, NP> &slot, int lane)
    {
      using C = Cfg<HD, NP>;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t pack0 = static_cast<std::size_t>(kp) * C::kWp; // pack's first channel
      if (tier == kFP16 || tier == kOwnPage)
      {
        // V image: chunk q = 64 d + lane is (c8, k, row) with row = q % 32.
        const int row = lane & 31;
        const int t = fp16_image_key(row);
        if (tier == kFP16)
        {
          const unsigned off =
              static_cast<unsigned>(((kPageTokens + t) * W + pack0) * 2);
#pragma unroll
          for (int d = 0; d < C::kVBytes / 1024; ++d)
          {
            const int idx = 2 * d + (lane >> 5); // c8 * NP + k
            const int k = idx % NP, c8 = idx / NP;
            dma16(u.page + off + (k * HD + 8 * c8) * 2, slot.v + 1024 * d);
          }
          return;
        }
        const std::uint16_t *vrow = value_row(u, tier, t, W) + pack0;
#pragma unroll
        for (int d = 0; d < C::kVBytes / 1024; ++d)
        {
          const int idx = 2 * d + (lane >> 5); // c8 * NP + k
          const int k = idx % NP, c8 = idx / NP;
          dma16(vrow + k * HD + 8 * c8, slot.v + 1024 * d);
        }
        return;
      }
      const auto quantised = [&](auto bits_tag) {
        constexpr int Bits = decltype(bits_tag)::value;
        const PageLayout &L = a.lay[Bits == 8 ? kINT8 : Bits == 4 ? kINT4 : kINT2];
        const std::uint8_t *p = u.page;
        if constexpr (Bits != 2)
        {
          // V codes: chunk q = 64 d + lane is 16 bytes of row q % 32 at chunk
          // index q / 32 = (c * NP + k), c a 16-byte column of the row.
          constexpr int kChunkChannels = 128 / Bits;
          const int t = lane & 31;
          const unsigned vrow = static_cast<unsigned>(L.value_codes + (t * W + pack0) * Bits / 8);
#pragma unroll
          for (int d = 0; d < C::kWp * 32 * Bits / 8 / 1024; ++d)
          {
            const int idx = 2 * d + (lane >> 5);
            const int k = idx % NP, c = idx / NP;
            dma16(p + vrow + (k * HD + kChunkChannels * c) * Bits / 8, slot.v + 1024 * d);
          }
        }
        // Key scales then key zeros of the pack: 2 * W' bytes each.
        constexpr int kMetaLanes = C::kKMeta / 16;
#pragma unroll
        for (int d = 0; d < (kMetaLanes + 63) / 64; ++d)
        {
          const int ml = 64 * d + lane;
          if (ml < kMetaLanes)
          {
            const int half = ml / (kMetaLanes / 2);
            const unsigned region = static_cast<unsigned>(half == 0 ? L.key_scales : L.key_zeros);
            dma16(p + region + static_cast<unsigned>(2 * pack0 + 16 * (ml % (kMetaLanes / 2))),
                  slot.kmeta + 1024 * d);
          }
        }
        // The pack's value scales then zeros: dword q = 64 d + lane is
        // (region, key t, j) with j < D, the pack's halves of key t.
        constexpr int D = value_meta_dwords<NP>();
#pragma unroll
        for (int d = 0; d < D; ++d)
        {
          const int q = 64 * d + lane;
          const int region = q / (32 * D), t = (q / D) % 32, j = q % D;
          const int half = t * a.kv_heads + kp * NP; // the pack's first half of key t
          const unsigned region_at =
              static_cast<unsigned>(region == 0 ? L.value_scales : L.value_zeros);
          dma4(p + region_at + static_cast<unsigned>(4 * (half / 2 + j)), slot.vmeta + 256 * d);
        }
      };
      switch (tier)
      {
      case kINT8:
        quantised(std::integral_constant<int, 8>{});
        break;
      case kINT4:
        quantised(std::integral_constant<int, 4>{});
        break;
      case kINT2:
        quantised(std::integral_constant<int, 2>{});
        break;
      default:
        break;
      }
    }

    // The register part of a sealed unit: the lane's two key rows (and, at
    // INT2, its two value rows) as eight 16-byte blocks, kraw slot kb * 4 + q
    // for row kb. Every tier issues the same eight loads into the same
    // registers, only the offsets differ: FP16 rows are 64 bytes (q = 0..3);
    // INT8 rows 32 (q = 0, 1, then again); INT4 rows 16 (q = 0, then again);
    // INT2 key and value rows 8 bytes each, in the 16-byte blocks holding
    // them (q = 0 keys, q = 1 values, then again). The repeats hit the cache;
    // one instruction sequence means the loads land in fixed registers with
    // nothing to merge between tiers.
    template <int HD, int NP>
    __device__ inline void issue_regs(const DecodeArgs &a, const std::uint8_t *page, int tier,
                                      int kp, unsigned *kraw, int lane)
    {
      using C = Cfg<HD, NP>;
      static_assert(C::kRun == 32, "a lane group holds 32 channels of a row");
      const int r = lane & 15, g = lane >> 4;
      const unsigned W = static_cast<unsigned>(a.kv_heads * HD);
      const unsigned gc = static_cast<unsigned>(kp * C::kWp + g * C::kRun);
      const int bits = tier == kINT8 ? 8 : tier == kINT4 ? 4 : tier == kINT2 ? 2 : 16;
      const unsigned vcodes = static_cast<unsigned>(a.lay[kINT2].value_codes);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const int t = tier == kINT4 ? key_of<true>(r, kb) : key_of<false>(r, kb);
        const unsigned key_at = (t * W + gc) * bits / 8; // key codes start the page
        const unsigned value_at = vcodes + (key_of<false>(r, kb) * W + gc) * 2 / 8;
        // Offsets without branches: block q of the row is 16 q (FP16),
        // 16 (q & 1) (INT8), 0 (INT4); INT2 takes keys at even q, values at
        // odd, each in its aligned block.
        const unsigned stride = bits >= 8 ? 16u : 0u;
        const unsigned qmask = bits == 16 ? 3u : 1u;
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
          const unsigned wide = key_at + stride * (static_cast<unsigned>(q) & qmask);
          const unsigned narrow = ((q & 1) != 0 ? value_at : key_at) & ~15u;
          load_at<16>(kraw + 4 * (kb * 4 + q), page, bits == 2 ? narrow : wide);
        }
      }
    }

    // The own page's key rows, FP16, as sealed FP16 rows sit in kraw: rows
    // before t_start from the open page, from t_start on from the chunk;
    // rows past the last key read row 0 (their scores are masked).
    template <int HD, int NP>
    __device__ inline void issue_regs_own(const DecodeArgs &a, const Rows &u, int kp,
                                          unsigned *kraw, int lane)
    {
      using C = Cfg<HD, NP>;
      const int r = lane & 15, g = lane >> 4;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t gc = static_cast<std::size_t>(kp) * C::kWp + g * C::kRun;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        load_words<2 * C::kRun>(kraw + kb * 16, key_row(u, kOwnPage, key_of<false>(r, kb), W) + gc);
      }
    }

    // q.K^T of a unit: acc[kb] = the scores of C rows (keys key_of(., kb)),
    // the keys read from kraw's slots (see issue_regs).
    template <int HD, int NP, int Bits>
    __device__ inline void unit_scores(f32x4 (&acc)[2], const unsigned *kraw, const half8 *qb,
                                       const std::uint8_t *kmeta, int g)
    {
      using C = Cfg<HD, NP>;
      acc[0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      acc[1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (Bits == 16)
      {
#pragma unroll
        for (int s = 0; s < C::kSteps; ++s)
        {
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
          {
            const unsigned *w = kraw + 4 * (kb * 4 + s);
            acc[kb] = mfma(as_half8(u32x4{w[0], w[1], w[2], w[3]}), qb[s], acc[kb]);
          }
        }
      }
      else
      {
        const auto *ks = reinterpret_cast<const u32x4 *>(kmeta) + g * (C::kRun / 8);
        const auto *kz = reinterpret_cast<const u32x4 *>(kmeta + 2 * C::kWp) + g * (C::kRun / 8);
        // INT2: an odd lane group's 8 bytes are its block's upper half; picked
        // by masking values, never by indexing, so kraw stays in registers.
        const unsigned upper = (g & 1) != 0 ? 0xFFFFFFFFu : 0u;
#pragma unroll
        for (int s = 0; s < C::kSteps; ++s)
        {
          const u32x4 s2 = ks[s];
          const u32x4 z2 = kz[s];
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
          {
            unsigned w0, w1 = 0;
            if constexpr (Bits == 8)
            {
              const unsigned *w = kraw + 4 * (kb * 4 + s / 2) + 2 * (s & 1);
              w0 = w[0];
              w1 = w[1];
            }
            else if constexpr (Bits == 4)
            {
              w0 = kraw[4 * (kb * 4) + s];
            }
            else
            {
              const unsigned *w = kraw + 4 * (kb * 4);
              const unsigned lo = w[s / 2], hi = w[2 + s / 2];
              w0 = (lo ^ ((lo ^ hi) & upper)) >> (16 * (s & 1));
            }
            acc[kb] = mfma(dequant_step<Bits>(w0, w1, s2, z2), qb[s], acc[kb]);
          }
        }
      }
    }

    // Value scale (region 0) or zero (region 1) of key t, KV head k of the
    // pack, from the slot's value metadata, as fp16 bits.
    template <int NP>
    __device__ inline unsigned value_meta(const std::uint8_t *vmeta, int region, int t, int k,
                                          int kp, int kv_heads)
    {
      constexpr int D = value_meta_dwords<NP>();
      const int half = NP == 1 ? ((t * kv_heads + kp) & 1) : (k & 1);
      const auto *w = reinterpret_cast<const unsigned *>(vmeta) + (region * 32 + t) * D +
                      (NP == 1 ? 0 : k / 2);
      return (*w >> (16 * half)) & 0xFFFFu;
    }

    // Value scales (or zeros) of keys 8g .. 8g+7 of the pack's KV head k, as
    // four packed pairs: natural (t, t+1), or (t, t+4) for INT4's order. The
    // keys' dwords are read together, the halves paired by byte permutes.
    template <int NP, bool Interleaved>
    __device__ inline u32x4 value_pairs(const std::uint8_t *vmeta, int region, int g, int k,
                                        int kp, int kv_heads)
    {
      constexpr int D = value_meta_dwords<NP>();
      // The dword of key 8g + j holding KV head k: j * D + k / 2.
      const auto *base = reinterpret_cast<const unsigned *>(vmeta) + (region * 32 + 8 * g) * D;
      unsigned w[8];
#pragma unroll
      for (int j = 0; j < 8; ++j)
      {
        w[j] = base[j * D + (NP == 1 ? 0 : k / 2)];
      }
      u32x4 out;
#pragma unroll
      for (int u = 0; u < 4; ++u)
      {
        const int j0 = Interleaved ? u : 2 * u;
        const int j1 = j0 + (Interleaved ? 4 : 1);
        const int h0 = NP == 1 ? (((8 * g + j0) * kv_heads + kp) & 1) : (k & 1);
        const int h1 = NP == 1 ? (((8 * g + j1) * kv_heads + kp) & 1) : (k & 1);
        const unsigned sel = static_cast<unsigned>(2 * h0) |
                             (static_cast<unsigned>(2 * h0 + 1) << 8) |
                             (static_cast<unsigned>(4 + 2 * h1) << 16) |
                             (static_cast<unsigned>(5 + 2 * h1) << 24);
        out[u] = __builtin_amdgcn_perm(w[j1], w[j0], sel);
      }
      return out;
    }

    // INT2 values: the lane's two value rows dequantised in registers and
    // written to the slot's FP16 image, for the same transposing reads as an
    // FP16 page.
    template <int HD, int NP>
    __device__ inline void int2_values_to_image(const unsigned *kraw, const Slot<HD, NP> &slot,
                                                int kp, int kv_heads, int lane)
    {
      using C = Cfg<HD, NP>;
      const int r = lane & 15, g = lane >> 4;
      const int k = g * C::kRun / HD;                // KV head within the pack
      const int c0 = (g * C::kRun) % HD;             // first channel within it
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
      {
        const int t = key_of<false>(r, kb);
        const unsigned s = value_meta<NP>(slot.vmeta, 0, t, k, kp, kv_heads);
        const unsigned z = value_meta<NP>(slot.vmeta, 1, t, k, kp, kv_heads);
        const unsigned sp = s | (s << 16), zp = z | (z << 16);
        const u32x4 s2 = {sp, sp, sp, sp}, z2 = {zp, zp, zp, zp};
        const unsigned *vc = kraw + 4 * (kb * 4 + 1);
        const unsigned upper = (g & 1) != 0 ? 0xFFFFFFFFu : 0u; // see unit_scores
        const int row = fp16_image_row(t);
#pragma unroll
        for (int s8 = 0; s8 < C::kRun / 8; ++s8)
        {
          const unsigned lo = vc[s8 / 2], hi = vc[2 + s8 / 2];
          const half8 v = dequant_step<2>((lo ^ ((lo ^ hi) & upper)) >> (16 * (s8 & 1)), 0u, s2, z2);
          const int c8 = c0 / 8 + s8;
          *reinterpret_cast<half8 *>(slot.v + 16 * ((c8 * NP + k) * 32 + row)) = v;
        }
      }
    }

    // P.V of a unit, V read transposed out of the slot block by block: per
    // 16-channel block and KV head k of the pack, eight keys of one channel
    // a lane (FP16 and INT2 from the fp16 image, two 4-key reads; INT8 one
    // 8-code read; INT4 one 16-code read serving two (block, k) pairs),
    // dequantised with each key's value scale and zero, times that head's
    // P (zero in other heads' columns), high and low parts.
    template <int HD, int NP, int Bits>
    __device__ inline void unit_pv(Running<HD> &run, const Slot<HD, NP> &slot,
                                   const half8 (&b_hi)[NP], const half8 (&b_lo)[NP], int kp,
                                   int kv_heads, int lane, const PageCtx &c)
    {
      using C = Cfg<HD, NP>;
      const int g = lane >> 4, s = lane & 15;
      if constexpr (Bits == 16 || Bits == 2)
      {
        const std::uint8_t *base =
            slot.v + 16 * (((s & 3) >> 1) * NP * 32 + 4 * g + (s >> 2)) + 8 * (s & 1);
        // A partial page (a cache that does not seal: its last page) may hold
        // anything past its last key: those values are zeroed, so that a
        // non-finite one cannot reach P.V through a zero weight.
        unsigned keep = 0xFFu;
        if (c.partial)
        {
          const int valid = c.last + 1 - 8 * g; // keys 8g .. 8g+7 of this lane
          keep = valid <= 0 ? 0u : valid >= 8 ? 0xFFu : (1u << valid) - 1u;
        }
#pragma unroll
        for (int cb = 0; cb < C::kCB; ++cb)
        {
#pragma unroll
          for (int k = 0; k < NP; ++k)
          {
            const std::uint8_t *p = base + 16 * (2 * cb * NP + k) * 32;
            const u32x2 x0 = tr16(p);
            const u32x2 x1 = tr16(p + 16 * 16);
            u32x4 w = {x0.x, x0.y, x1.x, x1.y};
            if (c.partial)
            {
#pragma unroll
              for (int e = 0; e < 4; ++e)
              {
                const unsigned lo = (keep >> (2 * e)) & 1u ? 0x0000FFFFu : 0u;
                const unsigned hi = (keep >> (2 * e + 1)) & 1u ? 0xFFFF0000u : 0u;
                w[e] &= lo | hi;
              }
            }
            const half8 v = as_half8(w);
            run.o[cb] = mfma(v, b_hi[k], run.o[cb]);
            run.o[cb] = mfma(v, b_lo[k], run.o[cb]);
          }
        }
      }
      else
      {
        u32x4 vs[NP], vz[NP];
#pragma unroll
        for (int k = 0; k < NP; ++k)
        {
          vs[k] = value_pairs<NP, Bits == 4>(slot.vmeta, 0, g, k, kp, kv_heads);
          vz[k] = value_pairs<NP, Bits == 4>(slot.vmeta, 1, g, k, kp, kv_heads);
        }
        if constexpr (Bits == 8)
        {
#pragma unroll
          for (int cb = 0; cb < C::kCB; ++cb)
          {
#pragma unroll
            for (int k = 0; k < NP; ++k)
            {
              const u32x2 x = tr8(slot.v + 512 * (cb * NP + k) + 8 * lane);
              const half8 v = dequant_step<8>(x.x, x.y, vs[k], vz[k]);
              run.o[cb] = mfma(v, b_hi[k], run.o[cb]);
              run.o[cb] = mfma(v, b_lo[k], run.o[cb]);
            }
          }
        }
        else
        {
          // Read rho: source lanes s < 8 carry pair 2 rho, s >= 8 pair
          // 2 rho + 1 (pair = cb * NP + k); source lane s reads key 8 g + s % 8.
#pragma unroll
          for (int rho = 0; rho < NP * C::kCB / 2; ++rho)
          {
            const int mine = 2 * rho + (s >> 3);
            const int mcb = mine / NP, mk = mine % NP;
            const u32x2 x = tr4(slot.v + 16 * (((mcb >> 1) * NP + mk) * 32 + 8 * g + (s & 7)) +
                                8 * (mcb & 1));
#pragma unroll
            for (int h = 0; h < 2; ++h)
            {
              const int pair = 2 * rho + h;
              const int cb = pair / NP, k = pair % NP;
              const half8 v = dequant_int4_interleaved(h == 0 ? x.x : x.y, vs[k], vz[k]);
              run.o[cb] = mfma(v, b_hi[k], run.o[cb]);
              run.o[cb] = mfma(v, b_lo[k], run.o[cb]);
            }
          }
        }
      }
    }

    template <int HD, int NP>
    __device__ inline Slot<HD, NP> slot_in(std::uint8_t *buffer, int wave)
    {
      Slot<HD, NP> slot;
      slot.v = buffer + wave * slot_bytes<HD, NP>();
      slot.kmeta = slot.v + Cfg<HD, NP>::kVBytes;
      slot.vmeta = slot.kmeta + Cfg<HD, NP>::kKMeta;
      return slot;
    }

    template <int HD, int NP>
    __global__ void __launch_bounds__(kThreads) decode_pages_kernel(DecodeArgs a)
    {
      using C = Cfg<HD, NP>;
      constexpr int kRow = HD + 4;
      // Two LDS buffers a wave: the unit being computed reads one while the
      // next unit's V and metadata land in the other. Two distinct arrays, so
      // that the compiler sees the copies into one cannot alias reads of the
      // other and adds no waits for them.
      __shared__ __attribute__((aligned(16))) std::uint8_t buf_a[kWaves * slot_bytes<HD, NP>()];
      __shared__ __attribute__((aligned(16))) std::uint8_t buf_b[kWaves * slot_bytes<HD, NP>()];

      const int lane = threadIdx.x & 63;
      // The wave index, and all that follows from it (pages, tiers, page
      // addresses), is uniform across the wave: said so, the tier switch is
      // scalar branching and only one tier's registers are live at a time.
      const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x >> 6));
      const int r = lane & 15;
      const int g = lane >> 4;
      const int split = blockIdx.x;
      const int kp = blockIdx.y;
      const int li = blockIdx.z;
      const int layer = a.first_layer + li;
      const int G = a.group;
      const int n_live = NP * G;
      const bool live = r < n_live;
      const int kn = live ? r / G : NP; // the column's KV head within the pack
      const Slot<HD, NP> sa = slot_in<HD, NP>(buf_a, wave);
      const Slot<HD, NP> sb = slot_in<HD, NP>(buf_b, wave);

      const unsigned long long *table = a.table + layer * a.table_stride;
      const std::uint8_t *tiers = a.tiers != nullptr ? a.tiers + layer * a.table_stride : nullptr;
      const int own = a.causal ? (a.seq_k - 1) / kPageTokens : -1;
      // The workgroup's pages, then this wave's share of them.
      const int wg0 = static_cast<int>(static_cast<long long>(split) * a.pages / a.splits);
      const int wg1 = static_cast<int>(static_cast<long long>(split + 1) * a.pages / a.splits);
      const int p0 = wg0 + (wg1 - wg0) * wave / kWaves;
      const int p1 = wg0 + (wg1 - wg0) * (wave + 1) / kWaves;
      float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;
      const int head = kp * n_live + (live ? r : 0);

      // q of the lane's column, block-diagonal: zero unless the lane group's
      // channels are the column's KV head's.
      half8 qb[C::kSteps];
      {
        const int kg = g * NP / 4; // the lane group's KV head within the pack
        const std::uint16_t *q_row = a.q + li * a.q_stride + static_cast<std::size_t>(head) * HD +
                                     (g * C::kRun) % HD;
        unsigned qw[C::kRun / 2];
        load_words<2 * C::kRun>(qw, q_row);
#pragma unroll
        for (int s = 0; s < C::kSteps; ++s)
        {
          qb[s] = (live && kg == kn)
                      ? as_half8(u32x4{qw[4 * s], qw[4 * s + 1], qw[4 * s + 2], qw[4 * s + 3]})
                      : as_half8(u32x4{0u, 0u, 0u, 0u});
        }
      }

      Running<HD> run;
      run.m = -INFINITY;
      run.l = 0.0f;
#pragma unroll
      for (int cb = 0; cb < C::kCB; ++cb)
      {
        run.o[cb] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
      }

      const auto *open = a.open_table != nullptr
                             ? reinterpret_cast<const std::uint16_t *>(a.open_table[layer])
                             : a.open;
      const auto own_rows = [&](int p) {
        Rows u;
        u.page = nullptr;
        u.open = open;
        u.chunk_k = a.chunk_k + li * a.chunk_stride;
        u.chunk_v = a.chunk_v + li * a.chunk_stride;
        u.t_start = a.start - p * kPageTokens;
        u.last = a.seq_k - 1 - p * kPageTokens;
        return u;
      };
      // Sealed pages of this wave: [p0, q1); the own page, if this wave's,
      // after them. Their tiers and addresses are read once, a lane a page,
      // 64 pages at a time, and taken out of the lanes as the loop goes.
      const int q1 = a.causal ? min(p1, own) : p1;
      unsigned long long my_addr = 0;
      int my_tier = kUnreadPage;
      const auto preload = [&](int from) {
        const int pl = from + lane;
        my_tier = kUnreadPage;
        my_addr = 0;
        if (pl < q1)
        {
          my_tier = a.causal ? static_cast<int>(tiers[pl]) : static_cast<int>(kFP16);
          if (my_tier != kUnreadPage)
          {
            my_addr = table[pl];
          }
        }
      };
      const auto tier_at = [&](int p) {
        return p < q1 ? __builtin_amdgcn_readlane(my_tier, (p - p0) & 63) : kUnreadPage;
      };
      const auto page_at = [&](int p) {
        const int i = (p - p0) & 63;
        return reinterpret_cast<const std::uint8_t *>(
            (static_cast<unsigned long long>(
                 __builtin_amdgcn_readlane(static_cast<unsigned>(my_addr >> 32), i))
             << 32) |
            static_cast<unsigned>(__builtin_amdgcn_readlane(static_cast<unsigned>(my_addr), i)));
      };

      unsigned kraw[C::kRaw];
      bool first = true;
      // A readable stand-in for a next unit that does not exist: the key
      // loads read the start of the decode workspace (at least 4 MiB; an
      // FP16 unit's offsets stay below 64 W bytes, 32 KiB at most) and
      // nothing uses what they return.
      const auto *stand_in = reinterpret_cast<const std::uint8_t *>(a.partials);
      const auto masks = [&](const half8 &p_hi, const half8 &p_lo, half8 (&b_hi)[NP],
                             half8 (&b_lo)[NP]) {
        // Each KV head of the pack multiplies its own heads' P only.
#pragma unroll
        for (int k = 0; k < NP; ++k)
        {
          b_hi[k] = kn == k ? p_hi : as_half8(u32x4{0u, 0u, 0u, 0u});
          b_lo[k] = kn == k ? p_lo : as_half8(u32x4{0u, 0u, 0u, 0u});
        }
      };
      const auto context = [&](int p) {
        PageCtx c;
        c.g = g;
        c.live = live;
        c.last = a.seq_k - 1 - p * kPageTokens;
        c.partial = c.last < kPageTokens - 1;
        c.first = first;
        c.scale = a.scale;
        c.stat = stats + (static_cast<std::size_t>(head) * a.pages + p) * 2;
        return c;
      };
      const auto unread = [&](int p) {
        if (g == 0 && live)
        {
          float *stat = stats + (static_cast<std::size_t>(head) * a.pages + p) * 2;
          stat[0] = -INFINITY;
          stat[1] = 0.0f;
        }
      };
      // One sealed unit: page p at `tier`, its V and metadata in x, its key
      // rows in kraw. The next sealed unit (page p + 1 at next_tier, at
      // next_page) is requested into y and kraw as soon as this unit's keys
      // are used, to fly while this unit's softmax and P.V are computed. The
      // key rows are requested from one place, whatever the tiers, so that
      // kraw's registers are the same on every path (with no next unit, a
      // page of the q rows stands in and is never read).
      const auto step = [&](int p, int tier, int next_tier, const std::uint8_t *next_page,
                            const Slot<HD, NP> &x, const Slot<HD, NP> &y) {
        const int ln = opaque(lane);
        f32x4 acc[2];
        // Every path waits here, so that no load is in flight into kraw when
        // the next unit's loads reuse its registers.
        wait_copies();
        if (tier != kUnreadPage)
        {
          switch (tier)
          {
          case kINT8:
            unit_scores<HD, NP, 8>(acc, kraw, qb, x.kmeta, ln >> 4);
            break;
          case kINT4:
            unit_scores<HD, NP, 4>(acc, kraw, qb, x.kmeta, ln >> 4);
            break;
          case kINT2:
            unit_scores<HD, NP, 2>(acc, kraw, qb, x.kmeta, ln >> 4);
            int2_values_to_image<HD, NP>(kraw, x, kp, a.kv_heads, ln);
            lds_order();
            break;
          default:
            unit_scores<HD, NP, 16>(acc, kraw, qb, x.kmeta, ln >> 4);
            break;
          }
        }
        const bool has_next = next_tier != kUnreadPage;
        if (has_next)
        {
          Rows u{};
          u.page = next_page;
          issue_lds<HD, NP>(a, u, next_tier, kp, y, ln);
        }
        issue_regs<HD, NP>(a, has_next ? next_page : stand_in, has_next ? next_tier : kFP16, kp,
                           kraw, ln);
        if (tier == kUnreadPage)
        {
          unread(p);
          return;
        }
        const PageCtx c = context(p);
        half8 p_hi, p_lo;
        softmax_page<HD>(acc, c, run, p_hi, p_lo);
        half8 b_hi[NP], b_lo[NP];
        masks(p_hi, p_lo, b_hi, b_lo);
        switch (tier)
        {
        case kINT8:
          unit_pv<HD, NP, 8>(run, x, b_hi, b_lo, kp, a.kv_heads, ln, c);
          break;
        case kINT4:
          unit_pv<HD, NP, 4>(run, x, b_hi, b_lo, kp, a.kv_heads, ln, c);
          break;
        case kINT2:
          unit_pv<HD, NP, 2>(run, x, b_hi, b_lo, kp, a.kv_heads, ln, c);
          break;
        default:
          unit_pv<HD, NP, 16>(run, x, b_hi, b_lo, kp, a.kv_heads, ln, c);
          break;
        }
        first = false;
      };

      preload(p0);
      int tier = tier_at(p0);
      {
        const bool has = tier != kUnreadPage;
        Rows u{};
        u.page = has ? page_at(p0) : stand_in;
        if (has)
        {
          issue_lds<HD, NP>(a, u, tier, kp, sa, lane);
        }
        issue_regs<HD, NP>(a, u.page, has ? tier : kFP16, kp, kraw, lane);
      }
      for (int p = p0; p < q1; p += 2)
      {
        // Every 64 pages the next 64 pages' tiers and addresses; the page
        // that starts the block was read with the block before.
        int t1 = kUnreadPage;
        const std::uint8_t *a1 = nullptr;
        if (p + 1 < q1)
        {
          if (((p + 1 - p0) & 63) == 0)
          {
            preload(p + 1);
          }
          t1 = tier_at(p + 1);
          a1 = page_at(p + 1);
        }
        step(p, tier, t1, a1, sa, sb);
        if (p + 1 >= q1)
        {
          break;
        }
        int t2 = kUnreadPage;
        const std::uint8_t *a2 = nullptr;
        if (p + 2 < q1)
        {
          if (((p + 2 - p0) & 63) == 0)
          {
            preload(p + 2);
          }
          t2 = tier_at(p + 2);
          a2 = page_at(p + 2);
        }
        step(p + 1, t1, t2, a2, sb, sa);
        tier = t2;
      }
      if (a.causal && own >= p0 && own < p1)
      {
        // The query's own page, FP16 from the open page and the chunk rows:
        // the last page, after the sealed ones (all of whose loads are done).
        const Rows u = own_rows(own);
        issue_lds<HD, NP>(a, u, kOwnPage, kp, sa, lane);
        issue_regs_own<HD, NP>(a, u, kp, kraw, lane);
        const PageCtx c = context(own);
        wait_copies();
        f32x4 acc[2];
        unit_scores<HD, NP, 16>(acc, kraw, qb, sa.kmeta, g);
        half8 p_hi, p_lo;
        softmax_page<HD>(acc, c, run, p_hi, p_lo);
        half8 b_hi[NP], b_lo[NP];
        masks(p_hi, p_lo, b_hi, b_lo);
        unit_pv<HD, NP, 16>(run, sa, b_hi, b_lo, kp, a.kv_heads, lane, c);
        first = false;
      }
      wait_reads();

      // The workgroup's waves into one partial: each wave's state to LDS
      // (buffer a is free once every wave is past its loop), then each
      // (wave, column)'s weight at the columns' common max, once.
      __syncthreads();
      auto *lf = reinterpret_cast<float *>(buf_a);
      float *s_m = lf;
      float *s_l = s_m + kWaves * 16;
      float *s_w = s_l + kWaves * 16; // kWaves * 16 weights, then 16 maxima
      float *s_o = s_w + kWaves * 16 + 16;
      static_assert((3 * kWaves * 16 + 16 + kWaves * 16 * kRow) * 4 <=
                        kWaves * slot_bytes<HD, NP>(),
                    "the epilogue's state fits buffer a");
      if (g == 0)
      {
        s_m[wave * 16 + r] = first ? -INFINITY : run.m;
        s_l[wave * 16 + r] = first ? 0.0f : run.l;
      }
#pragma unroll
      for (int cb = 0; cb < C::kCB; ++cb)
      {
#pragma unroll
        for (int i = 0; i < 4; ++i)
        {
          s_o[(wave * 16 + r) * kRow + 16 * cb + 4 * g + i] =
              first ? 0.0f : run.o[cb][i] * kPUnscale;
        }
      }
      __syncthreads();
      if (threadIdx.x < kWaves * 16)
      {
        const int h = threadIdx.x % 16;
        float top = -INFINITY;
#pragma unroll
        for (int w = 0; w < kWaves; ++w)
        {
          top = fmaxf(top, s_m[w * 16 + h]);
        }
        const float from = top == -INFINITY ? 0.0f : top;
        s_w[threadIdx.x] = exp2_fast(s_m[threadIdx.x] - from);
        if (threadIdx.x < 16)
        {
          s_w[kWaves * 16 + h] = top;
        }
      }
      __syncthreads();
      for (int idx = threadIdx.x; idx < n_live * (HD + 2); idx += kThreads)
      {
        const int h = idx / (HD + 2);
        const int col = idx % (HD + 2);
        float acc = s_w[kWaves * 16 + h];
        if (col != 0)
        {
          acc = 0.0f;
#pragma unroll
          for (int w = 0; w < kWaves; ++w)
          {
            const float v = col == 1 ? s_l[w * 16 + h] : s_o[(w * 16 + h) * kRow + col - 2];
            acc += v * s_w[w * 16 + h];
          }
        }
        const int kvh = kp * NP + h / G;
        float *part = a.partials +
                      (((static_cast<std::size_t>(li) * a.kv_heads + kvh) * a.splits + split) * G +
                       h % G) *
                          (kSlotHead + HD);
        part[col < 2 ? col : kSlotHead + col - 2] = acc;
      }
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
      const int splits = a.splits;
      const auto slot = [&](int h, int s) {
        return a.partials +
               (((static_cast<std::size_t>(li) * a.kv_heads + h / G) * splits + s) * G + h % G) *
                   (kSlotHead + HD);
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
        for (int s0 = j; s0 < splits; s0 += kSplitLanes * kLoadsAhead)
        {
          float mv[kLoadsAhead], lv[kLoadsAhead], ov[kLoadsAhead];
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            const int s = s0 + i * kSplitLanes;
            mv[i] = -INFINITY;
            lv[i] = 0.0f;
            ov[i] = 0.0f;
            if (s < splits)
            {
              const float *p = slot(h, s);
              mv[i] = p[0];
              lv[i] = p[1];
              ov[i] = p[kSlotHead + d0 + c];
            }
          }
          float next = top;
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            next = fmaxf(next, mv[i]);
          }
          const float from = next == -INFINITY ? 0.0f : next;
          const float keep = exp2_fast(top - from);
          acc *= keep;
          l *= keep;
#pragma unroll
          for (int i = 0; i < kLoadsAhead; ++i)
          {
            const float w = exp2_fast(mv[i] - from);
            acc += ov[i] * w;
            l += lv[i] * w;
          }
          top = next;
        }
        // Across the block: the common max, then every thread's share at it.
        const float all = block_reduce<true>(top, s_red);
        const float from = all == -INFINITY ? 0.0f : all;
        const float keep = exp2_fast(top - from);
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
      // This block's page: its (max, sum) of the first kHeadsAPass heads and
      // its old score are loaded now, while the head totals are formed.
      const int page = (blockIdx.x - a.heads * kChunks) * kCombineThreads + t;
      const bool has_page = page < a.pages;
      const float *stats = a.page_stats + static_cast<std::size_t>(li) * a.heads * a.pages * 2;
      float *scores = a.scores != nullptr ? a.scores + li * a.scores_stride : nullptr;
      const float old = has_page && scores != nullptr ? scores[page] : 0.0f;
      float2 st0[kHeadsAPass];
#pragma unroll
      for (int i = 0; i < kHeadsAPass; ++i)
      {
        if (has_page && i < a.heads)
        {
          st0[i] = *reinterpret_cast<const float2 *>(
              stats + (static_cast<std::size_t>(i) * a.pages + page) * 2);
        }
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
          for (int s0 = q; s0 < splits; s0 += 16 * kLoadsAhead)
          {
            float mv[kLoadsAhead], lv[kLoadsAhead];
#pragma unroll
            for (int i = 0; i < kLoadsAhead; ++i)
            {
              const int s = s0 + 16 * i;
              mv[i] = -INFINITY;
              lv[i] = 0.0f;
              if (s < splits)
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
        const float total = row16_sum(sum * exp2_fast(top - from));
        if (q == 0 && h < a.heads)
        {
          s_top[h] = from;
          s_sum[h] = total;
        }
      }
      __syncthreads();
      if (!has_page)
      {
        return;
      }
      float *mass = a.mass != nullptr ? a.mass + li * a.mass_stride : nullptr;
      float total = 0.0f;
      for (int h0 = 0; h0 < a.heads; h0 += kHeadsAPass)
      {
        // The page's (max, sum) of kHeadsAPass heads, loaded together.
        float2 st[kHeadsAPass];
#pragma unroll
        for (int i = 0; i < kHeadsAPass; ++i)
        {
          if (h0 == 0)
          {
            st[i] = st0[i];
          }
          else if (h0 + i < a.heads)
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
            const float share = st[i].y * exp2_fast(st[i].x - s_top[h]) / s_sum[h];
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
        a.kv_heads <= 0 || a.kv_heads > kMaxKvHeads || a.heads % a.kv_heads != 0 ||
        a.heads / a.kv_heads > kMaxGroup || a.heads > kMaxHeads || a.seq_k <= 0)
    {
      return false;
    }
    // A wave's pack is 128 channels: one KV head at head_dim 128; two at 64,
    // whose query heads must then fit the MFMA's 16 columns together.
    if (a.head_dim == 64 && (a.kv_heads % 2 != 0 || 2 * (a.heads / a.kv_heads) > kMaxGroup))
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
        if ((L.key_scales | L.key_zeros | L.value_codes | L.value_scales | L.page_bytes) % 16 != 0)
        {
          return false;
        }
      }
    }
    const int pages = (a.seq_k + kPageTokens - 1) / kPageTokens;
    return pages <= 65535 * kWaves;
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
    // A pack is 128 channels of a row: one KV head at head_dim 128, two at 64.
    const int cus = device_multiprocessors();
    const int wave_pages = (pages + kWaves - 1) / kWaves; // workgroups a group could have
    const int np = 128 / a.head_dim;
    const int packs = a.kv_heads / np;
    const long long groups = static_cast<long long>(ls.layers) * packs;
    if (!ls.split)
    {
      d.splits = 1; // no partials given: one workgroup a (layer, pack)
    }
    else
    {
      // Workgroups a group: the compute units shared out, at most a page a wave.
      const long long share = std::max<long long>(1, cus / groups);
      d.splits = static_cast<int>(std::min<long long>(share, wave_pages));
    }
    const std::size_t part = static_cast<std::size_t>(ls.layers) * a.kv_heads * d.splits * group *
                             (kSlotHead + a.head_dim);
    const std::size_t stats = static_cast<std::size_t>(ls.layers) * a.heads * pages * 2;
    float *ws = decode_workspace(part + stats);
    d.partials = ws;
    d.page_stats = ws + part;
    const int mass_blocks = (a.mass != nullptr || a.scores != nullptr)
                                ? (pages + kCombineThreads - 1) / kCombineThreads
                                : 0;
    const auto run = [&](auto pages_kernel, auto combine_kernel, int hd) {
      hipLaunchKernelGGL(pages_kernel, dim3(d.splits, packs, ls.layers), dim3(kThreads), 0,
                         stream, d);
      hip_check(hipGetLastError(), "decode pages kernel launch");
      hipLaunchKernelGGL(combine_kernel,
                         dim3(a.heads * (hd / kCombineDims) + mass_blocks, ls.layers),
                         dim3(kCombineThreads), 0, stream, d);
      hip_check(hipGetLastError(), "decode combine kernel launch");
    };
    if (a.head_dim == 128)
    {
      run(decode_pages_kernel<128, 1>, decode_combine_kernel<128>, 128);
    }
    else
    {
      run(decode_pages_kernel<64, 2>, decode_combine_kernel<64>, 64);
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
