// Attention of a chunk of queries on the matrix cores: QK^T and PV as
// v_mfma_f32_16x16x32_f16 over 32-key pages (reference: attention.cu:449-746,
// the prefill tile of qpb = 16 queries, and kv_pages.h:86-93, the causal
// reading of a cache that seals).
//
// The arithmetic is the general kernel's: a query reads each page before its
// own at the tier the page table records, dequantised as dequantise_page
// does (up to one fp16 ulp where the reference's fp32 value lands on an fp16
// tie), and its own page at FP16 from the open page and the
// chunk's rows; an unread page is skipped; the key bias is completed as
// k + RoPE(k_bias, j); online softmax; split-K runs of whole pages folded by
// a combine.
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
// lane's eight probabilities are the B operand of PV directly. V is staged
// in key rows and read transposed (ds_read_b64_tr_b16) in that key order.
//
// Staging. A step stages NP pages (two at head_dim 64 without a key bias)
// behind one barrier, double-buffered: the next step's pages are fetched to
// registers while this step's are multiplied, then dequantised (packed
// fp16, one rounding of code * scale + zero) into the other buffer.
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
#include "dequant.hpp"
#include "kernels.hpp"
#include "lane_ops.hpp"

#include <algorithm>
#include <cmath>

namespace mi
{
  namespace
  {

    typedef _Float16 half8 __attribute__((ext_vector_type(8)));
    typedef float f32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

    constexpr int kP = 32;              // keys a page, and a key tile
    // Probabilities are held x2^14 for PV (14 added in the exponent).
    constexpr float kPUnscale = 1.0f / 16384.0f;
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

    // A load from device memory through a global-address-space pointer.
    // Pages are reached through addresses held as integers, which the
    // compiler would otherwise read with flat instructions; a flat load
    // counts against the LDS wait counter as well, so every LDS read of the
    // products would wait for the next step's page fetch.
    template <typename T>
    __device__ inline T load_global(const void *p)
    {
      return *((const __attribute__((address_space(1))) T *)(p));
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

    // A page's stage: K rows (high parts, then low parts with a key bias),
    // kKS halves apart; then V as 16-byte chunks (key t, channels 8c ..
    // 8c+7) at chunk c * 32 + t, which the transposing LDS read hands out as
    // keys of one channel.
    template <int HD, bool kBias>
    __host__ __device__ constexpr int stage_halves()
    {
      return (kBias ? 2 : 1) * kP * Geometry<HD>::kKS + HD * kP;
    }

    typedef short i16x4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) i16x4 *lds_i16x4;

    // gfx950's transposing LDS read: the 16 lanes of a row group address a
    // 4-row x 16-channel block (lane s: row s / 4, channels 4 (s % 4) ..
    // +3) and lane s receives channel s of the four rows.
    __device__ inline uint2 tr16(const std::uint16_t *p)
    {
      return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_i16x4)(p)));
    }

    // Fetches one (key t, chunk c) of the item (page p, version) for KV head
    // kvh: global loads only; what it needs to dequantise comes with it.
    // The page-table entry of an item: the sealed page's address and tier
    // (or an FP16 page's address); loaded two items ahead of its data.
    struct Entry
    {
      unsigned long long page;
      int tier;
    };

    __device__ inline Entry entry_of(const KVSource &kv, int p, int version, int p_end)
    {
      Entry e{0, kFP16};
      if (p >= p_end)
      {
        return e;
      }
      if (kv.layout == Layout::kCausal && version == kSealed)
      {
        e.page = load_global<unsigned long long>(kv.pages + p);
        e.tier = load_global<std::uint8_t>(kv.tiers + p);
      }
      else if (kv.layout == Layout::kPaged)
      {
        e.page = load_global<unsigned long long>(kv.pages + p);
      }
      return e;
    }

    template <int HD>
    __device__ inline void fetch(const PrefillArgs &a, int p, int version, const Entry &entry,
                                 int kvh, int t, int c, Fetched &f)
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
        const int tier = entry.tier;
        const auto *page = reinterpret_cast<const std::uint8_t *>(entry.page);
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
            f.k.x = load_global<unsigned>(kc);
            f.k.y = load_global<unsigned>(kc + 4);
            f.v.x = load_global<unsigned>(vc);
            f.v.y = load_global<unsigned>(vc + 4);
          }
          else if (bits == 4)
          {
            f.k.x = load_global<unsigned>(kc);
            f.v.x = load_global<unsigned>(vc);
          }
          else
          {
            f.k.x = load_global<unsigned short>(kc);
            f.v.x = load_global<unsigned short>(vc);
          }
          f.ks = load_global<u32x4>(page + L.key_scales + 2 * at);
          f.kz = load_global<u32x4>(page + L.key_zeros + 2 * at);
          const std::size_t group = static_cast<std::size_t>(t) * a.kv_heads + kvh;
          const auto *vs = reinterpret_cast<const std::uint16_t *>(page + L.value_scales);
          const auto *vz = reinterpret_cast<const std::uint16_t *>(page + L.value_zeros);
          f.vsz = static_cast<unsigned>(load_global<std::uint16_t>(vs + group)) |
                  (static_cast<unsigned>(load_global<std::uint16_t>(vz + group)) << 16);
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
          const auto *h = reinterpret_cast<const std::uint16_t *>(entry.page);
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
        f.k = load_global<u32x4>(k_row + at);
        f.v = load_global<u32x4>(v_row + at);
        f.tier = kFP16;
      }
      else
      {
        f.k = u32x4{0, 0, 0, 0};
        f.v = u32x4{0, 0, 0, 0};
      }
    }

    // Word 3 of a raw buffer descriptor on gfx9-family parts (gfx950).
    constexpr int kBufferWord3 = 0x00020000;

    // A thread's byte offsets into a sealed page for its (key t, chunk c),
    // the same at every step: an FP16 page's key and value rows, the codes'
    // element index (the row's first channel), the key channels' scales
    // and zeros, the value row's scale and zero.
    struct ItemOffsets
    {
      int fp16_k;
      int fp16_v;
      int elem;
      int kmeta;
      int vgroup;
    };

    template <int HD>
    __device__ inline ItemOffsets item_offsets(int kv_heads, int kvh, int t, int c)
    {
      const int row = kv_heads * HD;
      const int at = kvh * HD + 8 * c;
      ItemOffsets o;
      o.elem = t * row + at;
      o.fp16_k = 2 * o.elem;
      o.fp16_v = 2 * ((kP + t) * row + at);
      o.kmeta = 2 * at;
      o.vgroup = 2 * (t * kv_heads + kvh);
      return o;
    }

    // fetch's sealed-page branch for a page the whole wave stages: its
    // address and tier uniform, so one buffer over the page with the
    // regions as scalar offsets and the thread's offsets fixed; the same
    // words as fetch reads. An FP16 page (no quantised layout: lay[kFP16]
    // is left empty) is its 2 x 32 rows of kv_heads * HD halves.
    template <int HD>
    __device__ inline void fetch_sealed(const PrefillArgs &a, unsigned long long page, int tier,
                                        const ItemOffsets &o, Fetched &f)
    {
      if (tier == kFP16)
      {
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            reinterpret_cast<void *>(page), 0, 4 * kP * a.kv_heads * HD, kBufferWord3);
        f.k = __builtin_amdgcn_raw_buffer_load_b128(rs, o.fp16_k, 0, 0);
        f.v = __builtin_amdgcn_raw_buffer_load_b128(rs, o.fp16_v, 0, 0);
        f.tier = kFP16;
        return;
      }
      const PageLayout &L = a.lay[tier];
      const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
          reinterpret_cast<void *>(page), 0, static_cast<int>(L.page_bytes), kBufferWord3);
      const int kc = static_cast<int>(L.key_codes);
      const int vc = static_cast<int>(L.value_codes);
      f.k = u32x4{0, 0, 0, 0};
      f.v = u32x4{0, 0, 0, 0};
      if (tier == kINT8)
      {
        const u32x2 k2 = __builtin_amdgcn_raw_buffer_load_b64(rs, o.elem, kc, 0);
        const u32x2 v2 = __builtin_amdgcn_raw_buffer_load_b64(rs, o.elem, vc, 0);
        f.k.x = k2.x;
        f.k.y = k2.y;
        f.v.x = v2.x;
        f.v.y = v2.y;
      }
      else if (tier == kINT4)
      {
        f.k.x = __builtin_amdgcn_raw_buffer_load_b32(rs, o.elem / 2, kc, 0);
        f.v.x = __builtin_amdgcn_raw_buffer_load_b32(rs, o.elem / 2, vc, 0);
      }
      else
      {
        f.k.x = __builtin_amdgcn_raw_buffer_load_b16(rs, o.elem / 4, kc, 0);
        f.v.x = __builtin_amdgcn_raw_buffer_load_b16(rs, o.elem / 4, vc, 0);
      }
      f.ks = __builtin_amdgcn_raw_buffer_load_b128(rs, o.kmeta, static_cast<int>(L.key_scales), 0);
      f.kz = __builtin_amdgcn_raw_buffer_load_b128(rs, o.kmeta, static_cast<int>(L.key_zeros), 0);
      f.vsz = static_cast<unsigned>(__builtin_amdgcn_raw_buffer_load_b16(
                  rs, o.vgroup, static_cast<int>(L.value_scales), 0)) |
              (static_cast<unsigned>(__builtin_amdgcn_raw_buffer_load_b16(
                   rs, o.vgroup, static_cast<int>(L.value_zeros), 0))
               << 16);
      f.tier = tier;
    }

    __device__ inline std::uint16_t half_of(const u32x4 &w, int e)
    {
      const unsigned word = e < 2 ? w.x : e < 4 ? w.y : e < 6 ? w.z : w.w;
      return static_cast<std::uint16_t>(word >> (16 * (e & 1)));
    }

    // The 8 fp16 K and V values of a fetch, as words: FP16 rows as read,
    // zeros for nothing read, codes dequantised in packed fp16 (one rounding
    // of code * scale + zero). Every lane that reaches the quantised branch
    // holds the same tier (a sealed page's).
    __device__ inline void values_of(const Fetched &f, u32x4 &k, u32x4 &v)
    {
      if (f.tier == kFP16)
      {
        k = f.k;
        v = f.v;
        return;
      }
      if (f.tier < 0)
      {
        k = u32x4{0, 0, 0, 0};
        v = u32x4{0, 0, 0, 0};
        return;
      }
      const unsigned sp = (f.vsz & 0xFFFFu) * 0x10001u;
      const unsigned zp = (f.vsz >> 16) * 0x10001u;
      const u32x4 vs2 = {sp, sp, sp, sp};
      const u32x4 vz2 = {zp, zp, zp, zp};
      switch (__builtin_amdgcn_readfirstlane(f.tier))
      {
      case kINT8:
        k = __builtin_bit_cast(u32x4, dq::dequant_step<8>(f.k.x, f.k.y, f.ks, f.kz));
        v = __builtin_bit_cast(u32x4, dq::dequant_step<8>(f.v.x, f.v.y, vs2, vz2));
        break;
      case kINT4:
        k = __builtin_bit_cast(u32x4, dq::dequant_step<4>(f.k.x, 0u, f.ks, f.kz));
        v = __builtin_bit_cast(u32x4, dq::dequant_step<4>(f.v.x, 0u, vs2, vz2));
        break;
      default:
        k = __builtin_bit_cast(u32x4, dq::dequant_step<2>(f.k.x, 0u, f.ks, f.kz));
        v = __builtin_bit_cast(u32x4, dq::dequant_step<2>(f.v.x, 0u, vs2, vz2));
        break;
      }
    }

    // The cos/sin pairs of position j for channels d0..d0+7 (the rope table
    // holds {cos, sin} per (position, j < hd/2)).
    template <int HD>
    __device__ inline void fetch_rope(const float *rope, int j, int d0, f32x4 cs[4])
    {
      constexpr int half = HD / 2;
      const int j0 = d0 < half ? d0 : d0 - half;
      const float *src = rope + 2 * (static_cast<std::size_t>(j) * half + j0);
      for (int i = 0; i < 4; ++i)
      {
        cs[i] = load_global<f32x4>(src + 4 * i);
      }
    }

    // RoPE of the key bias at one position for channels d0..d0+7 (reference:
    // attention.cu:104-116): channel d < hd/2 pairs with d + hd/2. b_first
    // holds bias[j0 .. j0+7] and b_second bias[j0+hd/2 .. +7], j0 the pair index.
    __device__ inline void rotated_bias8(const u32x4 &b_first, const u32x4 &b_second,
                                         const f32x4 cs[4], bool first_half, float rb[8])
    {
      for (int e = 0; e < 8; ++e)
      {
        const float c = cs[e / 2][2 * (e % 2)];
        const float s = cs[e / 2][2 * (e % 2) + 1];
        const float b1 = h2f(half_of(b_first, e));
        const float b2 = h2f(half_of(b_second, e));
        rb[e] = first_half ? b1 * c - b2 * s : b2 * c + b1 * s;
      }
    }

    // Writes a fetch into a stage: K (hi, and lo with a bias) row t, and V
    // chunk (t, c).
    template <int HD, bool kBias>
    __device__ inline void commit(const Fetched &f, const f32x4 cs[4], const u32x4 &b_first,
                                  const u32x4 &b_second, int t, int c, std::uint16_t *stage)
    {
      constexpr int KS = Geometry<HD>::kKS;
      u32x4 kw, vw;
      values_of(f, kw, vw);
      std::uint16_t *k_hi = stage;
      std::uint16_t *v_chunks = stage + (kBias ? 2 : 1) * kP * KS;
      if constexpr (kBias)
      {
        std::uint16_t *k_lo = stage + kP * KS;
        std::uint16_t hi[8], lo[8];
        if (f.tier >= 0)
        {
          float rb[8];
          rotated_bias8(b_first, b_second, cs, 8 * c < HD / 2, rb);
          for (int e = 0; e < 8; ++e)
          {
            const float x = h2f(half_of(kw, e)) + rb[e];
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
        *reinterpret_cast<u32x4 *>(k_hi + t * KS + 8 * c) = kw;
      }
      *reinterpret_cast<u32x4 *>(v_chunks + 8 * (c * kP + t)) = vw;
    }

    // The (page, version) items a workgroup visits, in order: a page before
    // every row's own page once, sealed; a page in the rows' own-page range
    // [o_lo, o_hi] sealed (when a row is past it) and then at FP16. Without
    // a cache that seals, every page once.
    __device__ inline int first_version(int p, bool causal, int o_hi)
    {
      return causal && p < o_hi ? kSealed : kOwn;
    }

    __device__ inline void advance(int &p, int &version, bool causal, int o_lo, int o_hi)
    {
      if (version == kSealed && p >= o_lo)
      {
        version = kOwn;
      }
      else
      {
        ++p;
        version = first_version(p, causal, o_hi);
      }
    }

    // The (page, version) items of a step, item j in element j: its table
    // entry, and whether it has keys to read (inside the workgroup's pages,
    // not an unread page). Vectors, not arrays of structures, so that a
    // thread's item index, which varies across the workgroup, selects in
    // registers.
    typedef int i32x2 __attribute__((ext_vector_type(2)));
    typedef unsigned long long u64x2 __attribute__((ext_vector_type(2)));
    constexpr int kMaxStepPages = 2;

    struct Step
    {
      i32x2 p;
      i32x2 version;
      i32x2 tier;
      i32x2 live;
      u64x2 page;
    };

    template <int HD, int TPW, int NP, bool kBias>
    __global__ void __launch_bounds__(kMaxWaves * 64)
        prefill_kernel(PrefillArgs a)
    {
      constexpr int KS = Geometry<HD>::kKS;
      constexpr int kItems = Geometry<HD>::kItems;
      constexpr int kStage = stage_halves<HD, kBias>();
      constexpr int kStepItems = NP * kItems;
      constexpr int kFetch = (kStepItems + kMinThreads - 1) / kMinThreads; // fetches a thread holds
      static_assert(NP >= 1 && NP <= kMaxStepPages, "pages a step");
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
      float l[TPW]; // in units of 2^-14 (the probabilities' scale)
      #pragma unroll
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
      const int o_lo = (shift + q_first) / kP;
      const int o_hi = (shift + q_last) / kP;
      const int p_begin = split * a.pages_per_split;
      const int p_end = min(p_begin + a.pages_per_split, o_hi + 1);

      // Staging items run key-fastest within a page: item = key + 32 *
      // chunk, page j of the step at j * kItems. A wave then stores V^T rows
      // of two chunks for all 32 keys at once, 32 distinct LDS dwords a
      // store, where key-major order put several chunks on one bank. A
      // thread's items keep their channel chunks from step to step, so its
      // bias channels are loaded once.
      u32x4 b_first[kFetch];
      u32x4 b_second[kFetch];
      #pragma unroll
      for (int u = 0; u < kFetch; ++u)
      {
        b_first[u] = u32x4{0, 0, 0, 0};
        b_second[u] = u32x4{0, 0, 0, 0};
        const int item = threadIdx.x + u * threads;
        if constexpr (kBias)
        {
          if (item < kStepItems)
          {
            const int d0 = 8 * ((item % kItems) / kP);
            const int j0 = d0 < HD / 2 ? d0 : d0 - HD / 2;
            const std::uint16_t *b = a.k_bias + static_cast<std::size_t>(kvh) * HD;
            b_first[u] = *reinterpret_cast<const u32x4 *>(b + j0);
            b_second[u] = *reinterpret_cast<const u32x4 *>(b + j0 + HD / 2);
          }
        }
      }

      // The items of the steps, NP a step, in visiting order from a cursor.
      int cursor_p = p_begin;
      int cursor_v = first_version(cursor_p, causal, o_hi);
      const auto take = [&](Step &st) {
        st.p = i32x2{p_end, p_end};
        st.version = i32x2{kOwn, kOwn};
        st.tier = i32x2{kFP16, kFP16};
        st.live = i32x2{0, 0};
        st.page = u64x2{0ull, 0ull};
#pragma unroll
        for (int j = 0; j < NP; ++j)
        {
          const Entry e = entry_of(a.kv, cursor_p, cursor_v, p_end);
          st.p[j] = cursor_p;
          st.version[j] = cursor_v;
          st.tier[j] = e.tier;
          st.page[j] = e.page;
          advance(cursor_p, cursor_v, causal, o_lo, o_hi);
        }
      };
      // Whether an item has anything to read: an unread sealed page has not.
      // Its table entry (every lane read the same one, a step earlier) is
      // made uniform here, so that what follows it branches on scalars.
      const auto settle = [&](Step &st) {
#pragma unroll
        for (int j = 0; j < NP; ++j)
        {
          st.tier[j] = __builtin_amdgcn_readfirstlane(st.tier[j]);
          const unsigned long long raw = st.page[j];
          st.page[j] =
              static_cast<unsigned long long>(
                  static_cast<unsigned>(__builtin_amdgcn_readfirstlane(static_cast<int>(raw)))) |
              (static_cast<unsigned long long>(static_cast<unsigned>(
                   __builtin_amdgcn_readfirstlane(static_cast<int>(raw >> 32))))
               << 32);
          st.live[j] = st.p[j] < p_end &&
                       !(causal && st.version[j] == kSealed && st.tier[j] == kUnreadPage);
        }
      };

      // A thread's items keep their (key, chunk) from step to step, and a
      // page's items are whole waves (kItems is a multiple of 64): each
      // wave stages one page a slot, its entry uniform.
      static_assert(kItems % 64 == 0, "a page's staging items are whole waves");
      Fetched f[kFetch];
      f32x4 cs[kFetch][4];
      const auto fetch_step = [&](const Step &st) {
        #pragma unroll
        for (int u = 0; u < kFetch; ++u)
        {
          const int item = threadIdx.x + u * threads;
          if (item < kStepItems)
          {
            const int j = __builtin_amdgcn_readfirstlane(item / kItems);
            const int t = (item % kItems) % kP;
            const int c = (item % kItems) / kP;
            const int p = st.p[j];
            f[u].tier = -1;
            // (With a key bias the general fetch: the buffer path's registers
            // would spill there.)
            if (!kBias && st.live[j] && causal && st.version[j] == kSealed)
            {
              fetch_sealed<HD>(a, st.page[j], st.tier[j], item_offsets<HD>(a.kv_heads, kvh, t, c),
                           f[u]);
            }
            else if (st.live[j])
            {
              const Entry e{st.page[j], st.tier[j]};
              fetch<HD>(a, p, st.version[j], e, kvh, t, c, f[u]);
            }
            if (st.live[j])
            {
              if constexpr (kBias)
              {
                if (p * kP + t < a.seq_k)
                {
                  fetch_rope<HD>(a.rope, p * kP + t, 8 * c, cs[u]);
                }
              }
            }
          }
        }
      };
      const auto commit_step = [&](const Step &st, std::uint16_t *stages) {
        #pragma unroll
        for (int u = 0; u < kFetch; ++u)
        {
          const int item = threadIdx.x + u * threads;
          if (item < kStepItems)
          {
            const int j = __builtin_amdgcn_readfirstlane(item / kItems);
            if (st.live[j])
            {
              commit<HD, kBias>(f[u], cs[u], b_first[u], b_second[u], (item % kItems) % kP,
                                (item % kItems) / kP, stages + j * kStage);
            }
          }
        }
      };

      // The step being computed, the next (being fetched) and the one after
      // (its table entries in flight).
      Step cur, nxt, nn;
      take(cur);
      take(nxt);
      settle(cur);
      int buf = 0;
      fetch_step(cur);
      commit_step(cur, smem);
      __syncthreads();

      while (cur.p[0] < p_end)
      {
        take(nn);
        settle(nxt);
        bool has_next = false;
#pragma unroll
        for (int j = 0; j < NP; ++j)
        {
          has_next = has_next || nxt.live[j];
        }
        if (has_next)
        {
          fetch_step(nxt);
        }
        if (computes)
        {
          const std::uint16_t *stages = smem + buf * NP * kStage;
          // S^T = K . Q^T, two 16-key tiles a page, each started from the
          // product's zero operand; a dead item's scores are zeros (the
          // softmax masks it whole).
          const f32x4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
          f32x4 s[TPW][2 * NP];
#pragma unroll
          for (int j = 0; j < NP; ++j)
          {
            if (!cur.live[j])
            {
              #pragma unroll
              for (int tt = 0; tt < TPW; ++tt)
              {
                s[tt][2 * j] = zero;
                s[tt][2 * j + 1] = zero;
              }
              continue;
            }
            const std::uint16_t *k_hi = stages + j * kStage;
            const std::uint16_t *k_lo = k_hi + kP * KS;
#pragma unroll
            for (int kt = 0; kt < 2; ++kt)
            {
#pragma unroll
              for (int cc = 0; cc < HD / 32; ++cc)
              {
                const int off = (16 * kt + col) * KS + 32 * cc + 8 * g;
                const half8 ka = as_half8(*reinterpret_cast<const u32x4 *>(k_hi + off));
                #pragma unroll
                for (int tt = 0; tt < TPW; ++tt)
                {
                  s[tt][2 * j + kt] = mfma(ka, qf[tt][cc], cc == 0 ? zero : s[tt][2 * j + kt]);
                }
                if constexpr (kBias)
                {
                  const half8 kb = as_half8(*reinterpret_cast<const u32x4 *>(k_lo + off));
                  #pragma unroll
                  for (int tt = 0; tt < TPW; ++tt)
                  {
                    s[tt][2 * j + kt] = mfma(kb, qf[tt][cc], s[tt][2 * j + kt]);
                  }
                }
              }
            }
          }
          // Online softmax per row over the step's keys, then P^T as the B
          // operand of PV. An item every row sees whole (a sealed page before
          // every row's own page, or without sealing a page wholly before the
          // first query) is not masked; a dead item is masked whole.
          half8 p_hi[TPW][NP], p_lo[TPW][NP];
          #pragma unroll
          for (int tt = 0; tt < TPW; ++tt)
          {
            // A masked key's score becomes -inf in place; an item every row
            // sees whole keeps its scores as they are.
            float top = -INFINITY;
#pragma unroll
            for (int j = 0; j < NP; ++j)
            {
              const int p = cur.p[j];
              const bool live = cur.live[j];
              const bool sealed = cur.version[j] == kSealed;
              const bool full = causal ? sealed && p < o_lo
                                       : p * kP + kP - 1 <= shift + q_first;
              // The row's last visible key position on this item (-1: none).
              int limit;
              if (!causal)
              {
                limit = pos[tt];
              }
              else if (sealed)
              {
                limit = p < own[tt] ? 0x7fffffff : -1;
              }
              else
              {
                limit = p == own[tt] ? pos[tt] : -1;
              }
              if (!live)
              {
                limit = -1;
              }
              if (!(live && full))
              {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                {
                  const int key = p * kP + key_of(e / 4, g, e % 4);
                  s[tt][2 * j + e / 4][e % 4] =
                      key <= limit ? s[tt][2 * j + e / 4][e % 4] : -INFINITY;
                }
              }
#pragma unroll
              for (int e = 0; e < 8; ++e)
              {
                top = fmaxf(top, s[tt][2 * j + e / 4][e % 4]);
              }
            }
            // Scores to base 2: the scale is positive, so the scaled maximum
            // is the maximum scaled.
            top = lane_max32(lane_max16(top)) * a.scale2;
            const float m_new = fmaxf(m[tt], top);
            const float from = m_new == -INFINITY ? 0.0f : m_new;
            const float keep = exp2_fast(m[tt] - from);
            m[tt] = m_new;
            // The probabilities come out x2^14 (the shift in the exponent).
            const float bias2 = 14.0f - from;
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < NP; ++j)
            {
#pragma unroll
              for (int e = 0; e < 8; ++e)
              {
                const float ps = exp2_fast(fmaf(s[tt][2 * j + e / 4][e % 4], a.scale2, bias2));
                sum += ps;
                _Float16 h, h_lo;
                split_half(ps, h, h_lo);
                p_hi[tt][j][e] = h;
                p_lo[tt][j][e] = h_lo;
              }
            }
            l[tt] = l[tt] * keep + sum;
            // Most steps leave every row's maximum where it was: rescale only
            // when some lane's moved.
            if (__any(keep != 1.0f))
            {
              for (int dt = 0; dt < HD / 16; ++dt)
              {
                o[tt][dt] *= keep;
              }
            }
          }
          // O^T += V^T . P^T, the high parts of every row tile before the
          // low parts, so that no product waits on the one before it.
#pragma unroll
          for (int j = 0; j < NP; ++j)
          {
            if (!cur.live[j])
            {
              continue;
            }
            // Lane (g, col) reads keys 4g .. 4g+3 and 16+4g .. 16+4g+3 of
            // channel 16 dt + col: P's key order.
            const std::uint16_t *vt = stages + j * kStage + (kBias ? 2 : 1) * kP * KS +
                                      8 * (((col & 3) >> 1) * kP + 4 * g + (col >> 2)) +
                                      4 * (col & 1);
            for (int dt = 0; dt < HD / 16; ++dt)
            {
              const uint2 x0 = tr16(vt + 8 * (2 * dt * kP));
              const uint2 x1 = tr16(vt + 8 * (2 * dt * kP + 16));
              const half8 va = as_half8(u32x4{x0.x, x0.y, x1.x, x1.y});
              #pragma unroll
              for (int tt = 0; tt < TPW; ++tt)
              {
                o[tt][dt] = mfma(va, p_hi[tt][j], o[tt][dt]);
              }
              #pragma unroll
              for (int tt = 0; tt < TPW; ++tt)
              {
                o[tt][dt] = mfma(va, p_lo[tt][j], o[tt][dt]);
              }
            }
          }
        }
        if (has_next)
        {
          commit_step(nxt, smem + (buf ^ 1) * NP * kStage);
        }
        __syncthreads();
        buf ^= 1;
        cur = nxt;
        nxt = nn;
      }

      // Each row's sum over its four lanes; then the output or the run's slot.
      #pragma unroll
      for (int tt = 0; tt < TPW; ++tt)
      {
        float total = l[tt];
        total = lane_sum32(lane_sum16(total));
        if (pos[tt] < 0)
        {
          continue;
        }
        if (a.partials == nullptr)
        {
          const float inv = 1.0f / total;
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
            slot[0] = m[tt]; // base 2, -inf for a run that saw no key
            slot[1] = total * kPUnscale;
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

    // Folds the runs of one (query, head) row: weights 2^(m_s - max m) (a
    // run that saw no key has m = -inf and weighs 0), out = sum(w o) /
    // sum(w l). kCombineThreads / HD groups of HD threads, a thread a channel,
    // share the runs; their sums meet in LDS. Runs' slots are (run, query,
    // head) apart, run_stride floats.
    constexpr int kCombineThreads = 1024;

    template <int HD>
    __global__ void __launch_bounds__(kCombineThreads)
        prefill_combine_kernel(const float *__restrict__ partials, std::uint16_t *__restrict__ out,
                               std::size_t run_stride, int splits)
    {
      constexpr int kGroups = kCombineThreads / HD;
      __shared__ float s_top[kCombineThreads / 64];
      __shared__ float s_acc[kGroups][HD];
      __shared__ float s_l[kGroups];
      const float *row = partials + static_cast<std::size_t>(blockIdx.x) * (HD + 2);
      float top = -INFINITY;
      for (int s = threadIdx.x; s < splits; s += kCombineThreads)
      {
        top = fmaxf(top, row[s * run_stride]);
      }
      for (int off = 32; off > 0; off >>= 1)
      {
        top = fmaxf(top, __shfl_xor(top, off));
      }
      if (threadIdx.x % 64 == 0)
      {
        s_top[threadIdx.x / 64] = top;
      }
      __syncthreads();
      top = s_top[0];
      for (int w = 1; w < kCombineThreads / 64; ++w)
      {
        top = fmaxf(top, s_top[w]);
      }
      const int group = threadIdx.x / HD;
      const int d = threadIdx.x % HD;
      float l = 0.0f;
      float acc = 0.0f;
#pragma unroll 4
      for (int s = group; s < splits; s += kGroups)
      {
        const float *slot = row + s * run_stride;
        const float w = exp2_fast(slot[0] - top);
        l += slot[1] * w;
        acc += slot[2 + d] * w;
      }
      s_acc[group][d] = acc;
      if (d == 0)
      {
        s_l[group] = l;
      }
      __syncthreads();
      if (group == 0)
      {
        float sum = 0.0f;
        float total = 0.0f;
        for (int g = 0; g < kGroups; ++g)
        {
          sum += s_acc[g][d];
          total += s_l[g];
        }
        out[static_cast<std::size_t>(blockIdx.x) * HD + d] =
            __half_as_ushort(__float2half_rn(sum / total));
      }
    }

    bool aligned16(const void *p) { return (reinterpret_cast<std::uintptr_t>(p) & 15) == 0; }

    // Launches the kernel for `args` (pages_per_split and partials still to
    // set): the keys split into runs of whole pages when the attention
    // workspace is given and the query blocks alone would not fill every
    // workgroup slot the kernel's occupancy allows, then a combine.
    template <int HD, int TPW, int NP, bool kBias>
    void run(PrefillArgs args, float *partials, int qblocks, int waves, hipStream_t stream)
    {
      const std::size_t lds = 2 * NP * stage_halves<HD, kBias>() * sizeof(std::uint16_t);
      auto kernel = prefill_kernel<HD, TPW, NP, kBias>;
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute prefill LDS");
      }
      const int pages = (args.seq_k + kP - 1) / kP;
      int splits = 1;
      if (partials != nullptr)
      {
        int resident = 0;
        hip_check(hipOccupancyMaxActiveBlocksPerMultiprocessor(&resident, kernel, 64 * waves, lds),
                  "hipOccupancyMaxActiveBlocksPerMultiprocessor prefill");
        const long blocks = static_cast<long>(qblocks) * args.kv_heads;
        const long target = static_cast<long>(std::max(resident, 1)) * device_multiprocessors();
        const long cap = static_cast<long>(attention_partials_floats(HD) / (HD + 2)) /
                         (static_cast<long>(args.seq_q) * args.heads);
        splits = static_cast<int>(
            std::max<long>(1, std::min<long>({target / blocks, pages / 2, cap})));
      }
      args.pages_per_split = (pages + splits - 1) / splits;
      splits = (pages + args.pages_per_split - 1) / args.pages_per_split;
      args.partials = splits > 1 ? partials : nullptr;
      hipLaunchKernelGGL(kernel, dim3(qblocks, args.kv_heads, splits), dim3(64 * waves), lds,
                         stream, args);
      hip_check(hipGetLastError(), "prefill kernel launch");
      if (splits > 1)
      {
        const std::size_t run_stride = static_cast<std::size_t>(args.seq_q) * args.heads * (HD + 2);
        hipLaunchKernelGGL(prefill_combine_kernel<HD>, dim3(args.seq_q * args.heads),
                           dim3(kCombineThreads), 0, stream, partials, args.out, run_stride,
                           splits);
        hip_check(hipGetLastError(), "prefill combine kernel launch");
      }
    }

    template <int HD, int TPW>
    void dispatch(const PrefillArgs &args, float *partials, int qblocks, int waves, bool bias,
                  hipStream_t stream)
    {
      if (bias)
      {
        run<HD, TPW, 1, true>(args, partials, qblocks, waves, stream);
      }
      else
      {
        // Two pages a barrier where the registers allow (no key bias).
        run<HD, TPW, HD == 64 ? 2 : 1, false>(args, partials, qblocks, waves, stream);
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
    // Rows a workgroup: up to 128 (eight tiles), 256 at head_dim 64 for a
    // long chunk (eight waves of two tiles), so each staged page feeds more
    // matrix work.
    const int row_target = hd == 64 && a.seq_q >= 256 ? 256 : 128;
    args.qb = std::max(1, std::min(a.seq_q, std::max(1, row_target / group)));
    args.rows = args.qb * group;
    args.scale2 = 1.4426950408889634f / std::sqrt(static_cast<float>(hd));
    const int tiles = (args.rows + 15) / 16;
    // Two tiles a wave share each K and V operand read; at head_dim 128 the
    // second tile's accumulators do not fit the registers.
    const int tpw = hd == 64 && tiles >= 4 ? 2 : 1;
    const int waves = std::max((tiles + tpw - 1) / tpw, kMinThreads / 64);
    if (waves > kMaxWaves)
    {
      throw InvalidArgument("prefill: " + std::to_string(tiles) + " row tiles exceed a workgroup");
    }
    const int qblocks = (a.seq_q + args.qb - 1) / args.qb;
    const bool bias = a.k_bias != nullptr;
    if (hd == 128)
    {
      dispatch<128, 1>(args, a.partials, qblocks, waves, bias, stream);
    }
    else if (tpw == 2)
    {
      dispatch<64, 2>(args, a.partials, qblocks, waves, bias, stream);
    }
    else
    {
      dispatch<64, 1>(args, a.partials, qblocks, waves, bias, stream);
    }
  }

} // namespace mi
