// Attention of a chunk of queries on the matrix cores: QK^T and PV as
// v_mfma_f32_16x16x32_f16 over 32-key pages (reference: attention.cu:449-746,
// the prefill tile of qpb = 16 queries, and kv_pages.h:86-93, the causal
// reading of a cache that seals).
//
// The arithmetic is the general kernel's: a query reads each page before its
// own at the tier the page table records, dequantised exactly as
// dequantise_page does, and its own page at FP16 from the open page and the
// chunk's rows; an unread page is skipped; the key bias is completed as
// k + RoPE(k_bias, j); online softmax; split-K runs folded by the combine.
//
// Work decomposition. A workgroup takes one KV head, `qb` consecutive queries
// and, when the keys are split, one run of whole pages. Its rows are the
// (query, head) pairs of those queries and the KV head's `group` query heads,
// row r = query r / group, head r % group, sixteen rows an MFMA tile. For each
// page the workgroup stages the KV head's 32 keys and values once in LDS, as
// fp16 (dequantised, plus the bias if any), and every wave multiplies its
// tiles against them:
//
//   S^T (32 keys x 16 rows) = K (keys x d) . Q^T   (A = K from LDS, B = Q^T
//                                                    held in registers)
//   O^T (d x 16 rows)      += V^T (d x keys) . P^T  (A = V^T from LDS, B = P^T)
//
// With S^T in the accumulator layout, lane l holds row l % 16 and keys
// 4(l/16)+i and 16+4(l/16)+i: each lane's scores are its own row's, so the
// softmax needs no transpose, a row's maximum is two lane exchanges, and the
// lane's eight probabilities are the B operand of PV directly when V^T's key
// order in LDS is permuted to match (slot 8g+e holds key 4g+e for e < 4 and
// 16+4g+e-4 after).
//
// Precision. Q, the dequantised K and V are exact in fp16. With a key bias,
// k + bias is formed in fp32 as the general kernel forms it and split into a
// high and a low fp16 part, two MFMAs. The probabilities are split the same
// way (high and low fp16 of p * 2^14) so PV keeps fp32-level accuracy; the
// scale leaves no low part subnormal that matters. Scores are taken to base 2
// (x log2(e)/sqrt(hd)) and exponentiated with v_exp_f32.
//
// Causality per row: against page p a row whose own page o is after p reads
// p sealed (all 32 keys); the row whose own page is p reads p's FP16 rows up
// to its position; a later page is masked. A workgroup therefore visits its
// pages in order, a page before every row's own page once (sealed), and a
// page in its rows' own-page range twice: sealed for the rows past it, FP16
// for the rows on it.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>

namespace mi
{
  namespace
  {

    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

    constexpr int kP = 32;              // keys a page, and a key tile
    constexpr int kVS = kP + 8;         // V^T row stride in halves (80 B: no bank conflicts)
    constexpr float kPScale = 16384.0f; // probabilities are held x2^14 for PV
    constexpr float kPUnscale = 1.0f / 16384.0f;
    constexpr float kLn2 = 0.693147180559945309f;
    constexpr int kMaxWaves = 8;
    constexpr int kMinThreads = 256; // a workgroup stages with at least this many threads

    enum : int
    {
      kSealed = 0, // a page before the row's own, at its recorded tier
      kOwn = 1,    // the row's own page at FP16 (or any FP16/contiguous page)
    };

    struct PrefillArgs
    {
      KVSource kv;
      PageLayout lay[kTierCount];
      const std::uint16_t *q;
      std::uint16_t *out;
      const std::uint16_t *k_bias;
      const float *rope;
      float *partials; // null: one run, the output written directly
      int seq_q;
      int seq_k;
      int heads;
      int kv_heads;
      int group;
      int qb;              // queries a workgroup
      int rows;            // qb * group
      int pages_per_split; // pages a run
      float scale2;        // log2(e) / sqrt(head_dim)
    };

    __device__ inline float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }

    __device__ inline f32x4 mfma(half8 a, half8 b, f32x4 c)
    {
      return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }

    __device__ inline half8 as_half8(u32x4 v) { return __builtin_bit_cast(half8, v); }

    // The LDS slot of key t in V^T's row (the PV operand's key order).
    __device__ inline int v_slot(int t)
    {
      return 8 * ((t & 15) >> 2) + (t & 3) + ((t >> 4) << 2);
    }

    // The key lane l's accumulator element (tile kt, index i) holds.
    __device__ inline int key_of(int kt, int g, int i) { return 16 * kt + 4 * g + i; }

    // What one thread fetched for one (key, 8-channel chunk) of a page:
    // raw K and V (fp16 rows, or codes), and for a quantised page the key
    // channels' scales and zeros and the value row's scale and zero.
    struct Fetched
    {
      u32x4 k;
      u32x4 v;
      u32x4 ks;
      u32x4 kz;
      unsigned vsz; // value scale | value zero << 16
      int tier;     // kFP16, a quantised tier, or -1 for zeros
    };

    template <int HD>
    struct Geometry
    {
      static constexpr int kKS = HD + 8;           // K row stride in halves (no bank conflicts)
      static constexpr int kChunks = HD / 8;       // 8-channel chunks a key row
      static constexpr int kItems = kP * kChunks;  // (key, chunk) pairs a page
    };

    template <int HD, bool kBias>
    __host__ __device__ constexpr int stage_halves()
    {
      return (kBias ? 2 : 1) * kP * Geometry<HD>::kKS + HD * kVS;
    }

    // Fetches one (key t, chunk c) of the item (page p, version) for KV head
    // kvh: global loads only; what it needs to dequantise comes with it.
    template <int HD>
    __device__ inline void fetch(const PrefillArgs &a, int p, int version, int kvh, int t, int c,
                                 Fetched &f)
    {
      const KVSource &kv = a.kv;
      const std::size_t row = static_cast<std::size_t>(a.kv_heads) * HD;
      const std::size_t at = static_cast<std::size_t>(kvh) * HD + 8 * c;
      const int j = p * kP + t;
      f.tier = -1;
      const std::uint16_t *k_row = nullptr;
      const std::uint16_t *v_row = nullptr;
      if (kv.layout == Layout::kCausal && version == kSealed)
      {
        const int tier = kv.tiers[p];
        const auto *page = reinterpret_cast<const std::uint8_t *>(kv.pages[p]);
        if (tier == kFP16)
        {
          const auto *h = reinterpret_cast<const std::uint16_t *>(page);
          k_row = h + t * row;
          v_row = h + (kP + t) * row;
        }
        else
        {
          const PageLayout &L = a.lay[tier];
          const int bits = tier == kINT8 ? 8 : tier == kINT4 ? 4 : 2;
          const std::size_t e = static_cast<std::size_t>(t) * row + at; // first element
          const std::uint8_t *kc = page + L.key_codes + e * bits / 8;
          const std::uint8_t *vc = page + L.value_codes + e * bits / 8;
          // 8 codes: 8 bytes at INT8, 4 at INT4, 2 at INT2.
          f.k = u32x4{0, 0, 0, 0};
          f.v = u32x4{0, 0, 0, 0};
          if (bits == 8)
          {
            const auto *k2 = reinterpret_cast<const unsigned *>(kc);
            const auto *v2 = reinterpret_cast<const unsigned *>(vc);
            f.k.x = k2[0];
            f.k.y = k2[1];
            f.v.x = v2[0];
            f.v.y = v2[1];
          }
          else if (bits == 4)
          {
            f.k.x = *reinterpret_cast<const unsigned *>(kc);
            f.v.x = *reinterpret_cast<const unsigned *>(vc);
          }
          else
          {
            f.k.x = *reinterpret_cast<const unsigned short *>(kc);
            f.v.x = *reinterpret_cast<const unsigned short *>(vc);
          }
          f.ks = *reinterpret_cast<const u32x4 *>(page + L.key_scales + 2 * at);
          f.kz = *reinterpret_cast<const u32x4 *>(page + L.key_zeros + 2 * at);
          const std::size_t group = static_cast<std::size_t>(t) * a.kv_heads + kvh;
          const auto *vs = reinterpret_cast<const std::uint16_t *>(page + L.value_scales);
          const auto *vz = reinterpret_cast<const std::uint16_t *>(page + L.value_zeros);
          f.vsz = static_cast<unsigned>(vs[group]) | (static_cast<unsigned>(vz[group]) << 16);
          f.tier = tier;
          return;
        }
      }
      else if (j < a.seq_k)
      {
        switch (kv.layout)
        {
        case Layout::kContiguous:
          k_row = kv.k + static_cast<std::size_t>(j) * row;
          v_row = kv.v + static_cast<std::size_t>(j) * row;
          break;
        case Layout::kPaged:
        {
          const auto *h = reinterpret_cast<const std::uint16_t *>(kv.pages[p]);
          k_row = h + t * row;
          v_row = h + (kP + t) * row;
          break;
        }
        case Layout::kCausal:
          if (j >= kv.start)
          {
            k_row = kv.chunk_k + static_cast<std::size_t>(j - kv.start) * row;
            v_row = kv.chunk_v + static_cast<std::size_t>(j - kv.start) * row;
          }
          else
          {
            k_row = kv.open + t * row;
            v_row = kv.open + (kP + t) * row;
          }
          break;
        }
      }
      if (k_row != nullptr)
      {
        f.k = *reinterpret_cast<const u32x4 *>(k_row + at);
        f.v = *reinterpret_cast<const u32x4 *>(v_row + at);
        f.tier = kFP16;
      }
      else
      {
        f.k = u32x4{0, 0, 0, 0};
        f.v = u32x4{0, 0, 0, 0};
      }
    }

    // Code e of 8 packed codes (first in the low bits).
    template <int Bits>
    __device__ inline unsigned code_at(const u32x4 &w, int e)
    {
      const int bit = e * Bits;
      const unsigned word = bit < 32 ? w.x : w.y;
      return (word >> (bit & 31)) & ((1u << Bits) - 1);
    }

    __device__ inline std::uint16_t half_of(const u32x4 &w, int e)
    {
      const unsigned word = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
      return static_cast<std::uint16_t>(word >> (16 * (e & 1)));
    }

    __device__ inline std::uint16_t dequant(unsigned code, std::uint16_t s, std::uint16_t z)
    {
      return __half_as_ushort(
          __float2half_rn(fmaf(static_cast<float>(code), h2f(s), h2f(z))));
    }

    // The 8 fp16 K and V values of a fetch.
    __device__ inline void values_of(const Fetched &f, std::uint16_t k[8], std::uint16_t v[8])
    {
      if (f.tier == kFP16 || f.tier < 0)
      {
        for (int e = 0; e < 8; ++e)
        {
          k[e] = half_of(f.k, e);
          v[e] = half_of(f.v, e);
        }
        return;
      }
      const std::uint16_t vs = static_cast<std::uint16_t>(f.vsz);
      const std::uint16_t vz = static_cast<std::uint16_t>(f.vsz >> 16);
      for (int e = 0; e < 8; ++e)
      {
        unsigned kc, vc;
        if (f.tier == kINT8)
        {
          kc = code_at<8>(f.k, e);
          vc = code_at<8>(f.v, e);
        }
        else if (f.tier == kINT4)
        {
          kc = code_at<4>(f.k, e);
          vc = code_at<4>(f.v, e);
        }
        else
        {
          kc = code_at<2>(f.k, e);
          vc = code_at<2>(f.v, e);
        }
        k[e] = dequant(kc, half_of(f.ks, e), half_of(f.kz, e));
        v[e] = dequant(vc, vs, vz);
      }
    }

    // RoPE of the key bias at position j for channels d0..d0+7 (reference:
    // attention.cu:104-116): d < hd/2 pairs with d + hd/2.
    template <int HD>
    __device__ inline void rotated_bias8(const std::uint16_t *bias, const float *rope, int j,
                                         int d0, float rb[8])
    {
      constexpr int half = HD / 2;
      const int j0 = d0 < half ? d0 : d0 - half;
      const float *cs = rope + 2 * (static_cast<std::size_t>(j) * half + j0);
      for (int e = 0; e < 8; ++e)
      {
        const float c = cs[2 * e];
        const float s = cs[2 * e + 1];
        const float b1 = h2f(bias[j0 + e]);
        const float b2 = h2f(bias[j0 + e + half]);
        rb[e] = d0 < half ? b1 * c - b2 * s : b2 * c + b1 * s;
      }
    }

    // Writes a fetch into a stage: K (hi, and lo with a bias) row t, and V^T.
    template <int HD, bool kBias>
    __device__ inline void commit(const PrefillArgs &a, const Fetched &f, int kvh, int j, int t,
                                  int c, std::uint16_t *stage)
    {
      constexpr int KS = Geometry<HD>::kKS;
      std::uint16_t k[8], v[8];
      values_of(f, k, v);
      std::uint16_t *k_hi = stage;
      std::uint16_t *vt = stage + (kBias ? 2 : 1) * kP * KS;
      if constexpr (kBias)
      {
        std::uint16_t *k_lo = stage + kP * KS;
        std::uint16_t hi[8], lo[8];
        if (f.tier >= 0)
        {
          float rb[8];
          rotated_bias8<HD>(a.k_bias + static_cast<std::size_t>(kvh) * HD, a.rope, j, 8 * c, rb);
          for (int e = 0; e < 8; ++e)
          {
            const float x = h2f(k[e]) + rb[e];
            const __half h = __float2half_rn(x);
            hi[e] = __half_as_ushort(h);
            lo[e] = __half_as_ushort(__float2half_rn(x - __half2float(h)));
          }
        }
        else
        {
          for (int e = 0; e < 8; ++e)
          {
            hi[e] = 0;
            lo[e] = 0;
          }
        }
        u32x4 wh, wl;
        wh.x = hi[0] | (unsigned(hi[1]) << 16);
        wh.y = hi[2] | (unsigned(hi[3]) << 16);
        wh.z = hi[4] | (unsigned(hi[5]) << 16);
        wh.w = hi[6] | (unsigned(hi[7]) << 16);
        wl.x = lo[0] | (unsigned(lo[1]) << 16);
        wl.y = lo[2] | (unsigned(lo[3]) << 16);
        wl.z = lo[4] | (unsigned(lo[5]) << 16);
        wl.w = lo[6] | (unsigned(lo[7]) << 16);
        *reinterpret_cast<u32x4 *>(k_hi + t * KS + 8 * c) = wh;
        *reinterpret_cast<u32x4 *>(k_lo + t * KS + 8 * c) = wl;
      }
      else
      {
        u32x4 w;
        w.x = k[0] | (unsigned(k[1]) << 16);
        w.y = k[2] | (unsigned(k[3]) << 16);
        w.z = k[4] | (unsigned(k[5]) << 16);
        w.w = k[6] | (unsigned(k[7]) << 16);
        *reinterpret_cast<u32x4 *>(k_hi + t * KS + 8 * c) = w;
      }
      const int slot = v_slot(t);
      for (int e = 0; e < 8; ++e)
      {
        vt[(8 * c + e) * kVS + slot] = v[e];
      }
    }

    // The pages a workgroup visits, in order, as (page, version) items.
    struct Walk
    {
      int p;
      int version;
      int p_end;
      int o_lo;
      int o_hi;
      bool causal;

      __device__ bool done() const { return p >= p_end; }

      __device__ void start(int p_begin)
      {
        p = p_begin;
        version = causal && p < o_hi ? kSealed : kOwn;
      }

      __device__ void next()
      {
        if (version == kSealed && p >= o_lo)
        {
          version = kOwn;
        }
        else
        {
          ++p;
          version = causal && p < o_hi ? kSealed : kOwn;
        }
      }
    };

    template <int HD, int TPW, bool kBias>
    __global__ void __launch_bounds__(kMaxWaves * 64)
        prefill_kernel(PrefillArgs a)
    {
      constexpr int KS = Geometry<HD>::kKS;
      constexpr int kChunks = Geometry<HD>::kChunks;
      constexpr int kItems = Geometry<HD>::kItems;
      constexpr int kStage = stage_halves<HD, kBias>();
      constexpr int kFetch = (kItems + kMinThreads - 1) / kMinThreads; // fetches a thread holds
      extern __shared__ std::uint16_t smem[];

      const int lane = threadIdx.x & 63;
      const int wave = threadIdx.x >> 6;
      const int waves = blockDim.x >> 6;
      const int threads = blockDim.x;
      const int g = lane >> 4;
      const int col = lane & 15;
      const int kvh = blockIdx.y;
      const int split = blockIdx.z;
      const int q_first = blockIdx.x * a.qb;
      const int q_last = min(q_first + a.qb, a.seq_q) - 1;
      const int shift = a.seq_k - a.seq_q;
      const bool causal = a.kv.layout == Layout::kCausal;
      // A wave whose first tile is past the rows only stages.
      const bool computes = wave * 16 < a.rows;
      const std::size_t token_stride = static_cast<std::size_t>(a.heads) * HD;

      // This wave's rows: position (or -1), own page, output offset.
      int pos[TPW];
      int own[TPW];
      int qrow[TPW];
      int head[TPW];
      half8 qf[TPW][HD / 32];
      f32x4 o[TPW][HD / 16];
      float m[TPW];
      float l[TPW];
      for (int tt = 0; tt < TPW; ++tt)
      {
        const int r = (wave + tt * waves) * 16 + col;
        const int ql = r / a.group;
        const bool valid = r < a.rows && q_first + ql <= q_last;
        qrow[tt] = q_first + ql;
        head[tt] = kvh * a.group + r % a.group;
        pos[tt] = valid ? shift + qrow[tt] : -1;
        own[tt] = valid ? pos[tt] / kP : -1;
        for (int cc = 0; cc < HD / 32; ++cc)
        {
          u32x4 w = u32x4{0, 0, 0, 0};
          if (valid)
          {
            w = *reinterpret_cast<const u32x4 *>(a.q + qrow[tt] * token_stride +
                                                 static_cast<std::size_t>(head[tt]) * HD +
                                                 32 * cc + 8 * g);
          }
          qf[tt][cc] = as_half8(w);
        }
        for (int dt = 0; dt < HD / 16; ++dt)
        {
          o[tt][dt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
        }
        m[tt] = -INFINITY;
        l[tt] = 0.0f;
      }

      // The pages this workgroup visits.
      const int x_lo = shift + q_first;
      const int x_hi = shift + q_last;
      Walk walk;
      walk.causal = causal;
      walk.o_lo = x_lo / kP;
      walk.o_hi = x_hi / kP;
      const int p_begin = split * a.pages_per_split;
      walk.p_end = min(p_begin + a.pages_per_split, x_hi / kP + 1);
      walk.start(p_begin);

      // Stage the first item.
      Fetched f[kFetch];
      const auto fetch_item = [&](const Walk &w) {
        for (int u = 0; u < kFetch; ++u)
        {
          const int item = threadIdx.x + u * threads;
          if (item < kItems)
          {
            fetch<HD>(a, w.p, w.version, kvh, item / kChunks, item % kChunks, f[u]);
          }
        }
      };
      const auto commit_item = [&](const Walk &w, std::uint16_t *stage) {
        for (int u = 0; u < kFetch; ++u)
        {
          const int item = threadIdx.x + u * threads;
          if (item < kItems)
          {
            const int t = item / kChunks;
            commit<HD, kBias>(a, f[u], kvh, w.p * kP + t, t, item % kChunks, stage);
          }
        }
      };
      // Whether an item has anything to read: an unread sealed page has not.
      const auto readable = [&](const Walk &w) {
        return !(causal && w.version == kSealed && a.kv.tiers[w.p] == kUnreadPage);
      };

      int buf = 0;
      if (!walk.done() && readable(walk))
      {
        fetch_item(walk);
        commit_item(walk, smem);
      }
      __syncthreads();

      while (!walk.done())
      {
        Walk next = walk;
        next.next();
        const bool has_next = !next.done() && readable(next);
        if (has_next)
        {
          fetch_item(next);
        }
        if (computes && readable(walk))
        {
          const std::uint16_t *stage = smem + buf * kStage;
          const std::uint16_t *k_hi = stage;
          const std::uint16_t *k_lo = stage + kP * KS;
          const std::uint16_t *vt = stage + (kBias ? 2 : 1) * kP * KS;
          // Each row's last visible key position on this item (-1: none).
          int limit[TPW];
          for (int tt = 0; tt < TPW; ++tt)
          {
            if (!causal)
            {
              limit[tt] = pos[tt];
            }
            else if (walk.version == kSealed)
            {
              limit[tt] = walk.p < own[tt] ? 0x7fffffff : -1;
            }
            else
            {
              limit[tt] = walk.p == own[tt] ? pos[tt] : -1;
            }
          }
          // S^T = K . Q^T, two 16-key tiles.
          f32x4 s[TPW][2];
          for (int tt = 0; tt < TPW; ++tt)
          {
            s[tt][0] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
            s[tt][1] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
          }
          for (int kt = 0; kt < 2; ++kt)
          {
            for (int cc = 0; cc < HD / 32; ++cc)
            {
              const int off = (16 * kt + col) * KS + 32 * cc + 8 * g;
              const half8 ka = as_half8(*reinterpret_cast<const u32x4 *>(k_hi + off));
              for (int tt = 0; tt < TPW; ++tt)
              {
                s[tt][kt] = mfma(ka, qf[tt][cc], s[tt][kt]);
              }
              if constexpr (kBias)
              {
                const half8 kb = as_half8(*reinterpret_cast<const u32x4 *>(k_lo + off));
                for (int tt = 0; tt < TPW; ++tt)
                {
                  s[tt][kt] = mfma(kb, qf[tt][cc], s[tt][kt]);
                }
              }
            }
          }
          // Online softmax per row, then P^T as the B operand of PV.
          half8 p_hi[TPW], p_lo[TPW];
          for (int tt = 0; tt < TPW; ++tt)
          {
            float sc[8];
            float top = -INFINITY;
            for (int kt = 0; kt < 2; ++kt)
            {
              for (int i = 0; i < 4; ++i)
              {
                const int j = walk.p * kP + key_of(kt, g, i);
                const float x = s[tt][kt][i] * a.scale2;
                const float v = j <= limit[tt] ? x : -INFINITY;
                sc[4 * kt + i] = v;
                top = fmaxf(top, v);
              }
            }
            top = fmaxf(top, __shfl_xor(top, 16));
            top = fmaxf(top, __shfl_xor(top, 32));
            const float m_new = fmaxf(m[tt], top);
            const float from = m_new == -INFINITY ? 0.0f : m_new;
            const float keep = exp2_fast(m[tt] - from);
            m[tt] = m_new;
            float sum = 0.0f;
            for (int e = 0; e < 8; ++e)
            {
              const float pe = exp2_fast(sc[e] - from);
              sum += pe;
              const float ps = pe * kPScale;
              const _Float16 h = static_cast<_Float16>(ps);
              p_hi[tt][e] = h;
              p_lo[tt][e] = static_cast<_Float16>(ps - static_cast<float>(h));
            }
            l[tt] = l[tt] * keep + sum;
            if (keep != 1.0f)
            {
              for (int dt = 0; dt < HD / 16; ++dt)
              {
                o[tt][dt] *= keep;
              }
            }
          }
          // O^T += V^T . P^T.
          for (int dt = 0; dt < HD / 16; ++dt)
          {
            const half8 va = as_half8(
                *reinterpret_cast<const u32x4 *>(vt + (16 * dt + col) * kVS + 8 * g));
            for (int tt = 0; tt < TPW; ++tt)
            {
              o[tt][dt] = mfma(va, p_hi[tt], o[tt][dt]);
              o[tt][dt] = mfma(va, p_lo[tt], o[tt][dt]);
            }
          }
        }
        if (has_next)
        {
          commit_item(next, smem + (buf ^ 1) * kStage);
        }
        __syncthreads();
        buf ^= 1;
        walk = next;
      }

      // Each row's sum over its four lanes; then the output or the run's slot.
      for (int tt = 0; tt < TPW; ++tt)
      {
        float total = l[tt];
        total += __shfl_xor(total, 16);
        total += __shfl_xor(total, 32);
        if (pos[tt] < 0)
        {
          continue;
        }
        if (a.partials == nullptr)
        {
          const float inv = kPUnscale / total;
          std::uint16_t *dst = a.out + qrow[tt] * token_stride +
                               static_cast<std::size_t>(head[tt]) * HD + 4 * g;
          for (int dt = 0; dt < HD / 16; ++dt)
          {
            unsigned lo = __half_as_ushort(__float2half_rn(o[tt][dt][0] * inv)) |
                          (unsigned(__half_as_ushort(__float2half_rn(o[tt][dt][1] * inv))) << 16);
            unsigned hi = __half_as_ushort(__float2half_rn(o[tt][dt][2] * inv)) |
                          (unsigned(__half_as_ushort(__float2half_rn(o[tt][dt][3] * inv))) << 16);
            *reinterpret_cast<uint2 *>(dst + 16 * dt) = make_uint2(lo, hi);
          }
        }
        else
        {
          float *slot = a.partials + ((static_cast<std::size_t>(split) * a.seq_q + qrow[tt]) *
                                          a.heads + head[tt]) * (HD + 2);
          if (g == 0)
          {
            slot[0] = m[tt] == -INFINITY ? -INFINITY : m[tt] * kLn2;
            slot[1] = total;
          }
          for (int dt = 0; dt < HD / 16; ++dt)
          {
            for (int i = 0; i < 4; ++i)
            {
              slot[2 + 16 * dt + 4 * g + i] = o[tt][dt][i] * kPUnscale;
            }
          }
        }
      }
    }

    bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

    template <int HD, int TPW, bool kBias>
    void run(const PrefillArgs &args, dim3 grid, int waves, hipStream_t stream)
    {
      const std::size_t lds = 2 * stage_halves<HD, kBias>() * sizeof(std::uint16_t);
      auto kernel = prefill_kernel<HD, TPW, kBias>;
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute prefill LDS");
      }
      hipLaunchKernelGGL(kernel, grid, dim3(64 * waves), lds, stream, args);
    }

    template <int HD>
    void dispatch(const PrefillArgs &args, dim3 grid, int waves, int tpw, bool bias,
                  hipStream_t stream)
    {
      if (bias)
      {
        tpw == 2 ? run<HD, 2, true>(args, grid, waves, stream)
                 : run<HD, 1, true>(args, grid, waves, stream);
      }
      else
      {
        tpw == 2 ? run<HD, 2, false>(args, grid, waves, stream)
                 : run<HD, 1, false>(args, grid, waves, stream);
      }
    }

  } // namespace

  bool prefill_applies(const KVSource &kv, const AttentionArgs &a)
  {
    if (a.mass != nullptr || a.scores != nullptr)
    {
      return false;
    }
    if (a.head_dim != 64 && a.head_dim != 128)
    {
      return false;
    }
    if (a.kv_heads <= 0 || a.heads / a.kv_heads > 128)
    {
      return false; // one query's rows must fit a workgroup's tiles
    }
    if (kv.layout != Layout::kContiguous && kv.page_tokens != kP)
    {
      return false;
    }
    const bool ok = aligned16(a.q) && aligned16(a.out) &&
                    (a.k_bias == nullptr || aligned16(a.k_bias)) &&
                    (kv.layout != Layout::kContiguous || (aligned16(kv.k) && aligned16(kv.v))) &&
                    (kv.layout != Layout::kCausal ||
                     (aligned16(kv.chunk_k) && aligned16(kv.chunk_v) && aligned16(kv.open)));
    return ok;
  }

  void launch_prefill(const KVSource &kv, const AttentionArgs &a, hipStream_t stream)
  {
    const int hd = a.head_dim;
    const int group = a.heads / a.kv_heads;
    PrefillArgs args{};
    args.kv = kv;
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        args.lay[t] = page_layout(t, kP, a.kv_heads, hd);
      }
    }
    args.q = a.q;
    args.out = a.out;
    args.k_bias = a.k_bias;
    args.rope = a.rope;
    args.seq_q = a.seq_q;
    args.seq_k = a.seq_k;
    args.heads = a.heads;
    args.kv_heads = a.kv_heads;
    args.group = group;
    args.qb = std::max(1, std::min(a.seq_q, std::max(1, 128 / group)));
    args.rows = args.qb * group;
    args.scale2 = 1.4426950408889634f / std::sqrt(static_cast<float>(hd));
    const int tiles = (args.rows + 15) / 16;
    const int tpw = tiles >= 4 ? 2 : 1;
    const int waves = std::max((tiles + tpw - 1) / tpw, kMinThreads / 64);
    if (waves > kMaxWaves)
    {
      throw InvalidArgument("prefill: " + std::to_string(tiles) + " row tiles exceed a workgroup");
    }
    const int qblocks = (a.seq_q + args.qb - 1) / args.qb;
    const int pages = (a.seq_k + kP - 1) / kP;
    int splits = 1;
    if (a.partials != nullptr)
    {
      const long blocks = static_cast<long>(qblocks) * a.kv_heads;
      const long target = 2L * device_multiprocessors();
      const long cap = static_cast<long>(attention_partials_floats(hd) / (hd + 2)) /
                       (static_cast<long>(a.seq_q) * a.heads);
      const long want = std::min<long>({(target + blocks - 1) / blocks, pages / 4, cap});
      splits = static_cast<int>(std::max<long>(1, want));
    }
    args.pages_per_split = (pages + splits - 1) / splits;
    splits = (pages + args.pages_per_split - 1) / args.pages_per_split;
    args.partials = splits > 1 ? a.partials : nullptr;
    const dim3 grid(qblocks, a.kv_heads, splits);
    if (hd == 64)
    {
      dispatch<64>(args, grid, waves, tpw, a.k_bias != nullptr, stream);
    }
    else
    {
      dispatch<128>(args, grid, waves, tpw, a.k_bias != nullptr, stream);
    }
    hip_check(hipGetLastError(), "prefill kernel launch");
    if (splits > 1)
    {
      launch_attention_combine(a.partials, a.out, a.seq_q, a.heads, hd, splits, stream);
    }
  }

} // namespace mi
