// Page jobs: the byte and requantisation work a cache's stores, tier moves
// and compaction make, on gfx950.
//
//   - copy_refs / requant_refs: batches named by 32-bit page references
//     (a tier range's slot, or a shadow's number); the kernels form the
//     addresses, so a batch of thousands of moves sends 8 bytes a pair;
//   - row_jobs: one store's seals, open-page fills and the Halves
//     diagnostic's round trips, every kind in one launch, the jobs passed by
//     value (a decode step's store uploads nothing);
//   - table_edits: a page table's changed entries applied on the device.
//
// The register quantiser. A 32-token page of W = kv_heads * head_dim
// channels (head_dim 64 or 128) is split into W tasks of 64 elements, a lane
// each, none staged through LDS:
//   - key task (j, g), W/2 of them: channels [8j, 8j + 8) of rows
//     [8g, 8g + 8), eight 16-byte loads. A key channel's range is over all
//     32 rows, so the four tasks of a chunk (adjacent lanes) fold their
//     minima and maxima with two lane exchanges; each then codes its own
//     8 rows, one 2/4/8-byte store a row;
//   - value task (r, h, part), W/2 of them: channels [64 part, 64 part + 64)
//     of head h in row r, eight 16-byte loads; at head_dim 128 the two
//     parts of a (row, head) group fold their range with one exchange; the
//     codes leave in 16-byte stores.
// Every input byte is read once and every output byte written once; a page
// is W lanes (a workgroup of 256 covers one 1.5B page, two 0.5B pages), so a
// batch of pages fills the device with no serial walk over rows.
//
// Codes, scales and zeros follow quant_core.hpp (the reference's rules,
// quant.cu:44-199) to the bit.

#include "common.hpp"
#include "kernels.hpp"
#include "quant_core.hpp"

#include <algorithm>

namespace mi
{
  namespace
  {
    constexpr int kThreads = 256;
    constexpr int kP = 32; // the register quantiser's page

    __device__ inline std::uint8_t *resolve(const PageSpaces &s, std::uint32_t ref)
    {
      const std::uint32_t space = ref >> kRefIndexBits;
      const std::uint32_t index = ref & kRefIndexMask;
      if (space == kShadowSpace)
      {
        return reinterpret_cast<std::uint8_t *>(s.shadows[index]);
      }
      if (space == kStagingSpace)
      {
        return reinterpret_cast<std::uint8_t *>(s.staging + s.shadow_bytes * index);
      }
      return reinterpret_cast<std::uint8_t *>(s.base[space] + s.bytes[space] * index);
    }

    __device__ inline unsigned long long page_size(const PageSpaces &s, std::uint32_t ref)
    {
      const std::uint32_t space = ref >> kRefIndexBits;
      return space >= kShadowSpace ? s.shadow_bytes : s.bytes[space];
    }

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

    __device__ inline uint4 load16(const std::uint16_t *p)
    {
      return *reinterpret_cast<const uint4 *>(p);
    }
    __device__ inline void store16(std::uint16_t *p, uint4 v) { *reinterpret_cast<uint4 *>(p) = v; }

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
        *reinterpret_cast<uint2 *>(at) =
            uint2{static_cast<unsigned>(packed), static_cast<unsigned>(packed >> 32)};
      }
      else if constexpr (Bits == 4)
      {
        *reinterpret_cast<unsigned *>(at) = static_cast<unsigned>(packed);
      }
      else
      {
        *reinterpret_cast<std::uint16_t *>(at) = static_cast<std::uint16_t>(packed);
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
    // of chunk j sit in lanes 4j .. 4j + 3 of one wave. Two passes: the
    // ranges, with all eight rows' loads in flight at once; then the codes a
    // row at a time, each row read again (from cache: the first pass just
    // brought it), so that the 64 divisions never hold all eight rows.
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
    // At head_dim 128 the group's two parts sit in adjacent lanes. The same
    // two passes as a key task, over the row's eight 16-byte runs.
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
          reinterpret_cast<std::uint16_t *>(dst + L.value_scales)[group] = sbits;
          reinterpret_cast<std::uint16_t *>(dst + L.value_zeros)[group] =
              static_cast<std::uint16_t>(half_of(lo));
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
          *reinterpret_cast<uint4 *>(at + 4 * w) =
              uint4{words[w], words[w + 1], words[w + 2], words[w + 3]};
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

    // ---- batches by reference ------------------------------------------------

    // Page blockIdx.y of the batch: the blocks of x stride over its bytes.
    __global__ void __launch_bounds__(kThreads)
        copy_refs_kernel(const RefPair *__restrict__ pairs, PageSpaces s)
    {
      const RefPair p = pairs[blockIdx.y];
      const auto *src = reinterpret_cast<const uint4 *>(resolve(s, p.from));
      auto *dst = reinterpret_cast<uint4 *>(resolve(s, p.to));
      const unsigned long long bytes = page_size(s, p.to);
      const unsigned long long units = bytes / 16;
      for (unsigned long long i = static_cast<unsigned long long>(blockIdx.x) * kThreads + threadIdx.x;
           i < units; i += static_cast<unsigned long long>(gridDim.x) * kThreads)
      {
        dst[i] = src[i];
      }
      // A page size that is not a multiple of 16: its last bytes one by one.
      if (blockIdx.x == 0 && threadIdx.x < bytes % 16)
      {
        const unsigned long long at = 16 * units + threadIdx.x;
        reinterpret_cast<std::uint8_t *>(dst)[at] = reinterpret_cast<const std::uint8_t *>(src)[at];
      }
    }

    // The register quantiser over a batch: lane (blockIdx.x * 256 + tid)
    // is task (lane % W) of pair (lane / W).
    template <int Bits, int HD>
    __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
        requant_refs_kernel(const RefPair *__restrict__ pairs, int count, PageSpaces s,
                            PageLayout L, int kv_heads)
    {
      const int W = kv_heads * HD;
      const long long lane = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
      const long long pair = lane / W;
      if (pair >= count)
      {
        return; // whole waves: W is a multiple of 64
      }
      const RefPair p = pairs[pair];
      const auto *src = reinterpret_cast<const std::uint16_t *>(resolve(s, p.from));
      std::uint8_t *dst = resolve(s, p.to);
      const Rows keys{src, src, kP, W};
      const Rows values{src + static_cast<std::size_t>(kP) * W, src + static_cast<std::size_t>(kP) * W,
                        kP, W};
      page_task<Bits, HD>(static_cast<int>(lane % W), keys, values, kv_heads, dst, L, Emit::kCodes,
                          Emit::kCodes);
    }

    // The register quantiser over pages named by address (the batch API):
    // page i's keys at rows[i] (or row0), its values `values_offset` bytes
    // on, quantised into pages[i] (or page0); lane (blockIdx.x * 256 + tid)
    // is task (lane % W) of page (lane / W).
    template <int Bits, int HD>
    __global__ void __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(4)))
        quantise_ptrs_kernel(const void *const *__restrict__ rows, void *const *__restrict__ pages,
                             const void *row0, void *page0, std::ptrdiff_t values_offset,
                             int count, PageLayout L, int kv_heads)
    {
      const int W = kv_heads * HD;
      const long long lane = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
      const long long page = lane / W;
      if (page >= count)
      {
        return; // whole waves: W is a multiple of 64
      }
      const auto *src = static_cast<const std::uint8_t *>(rows ? rows[page] : row0);
      auto *dst = static_cast<std::uint8_t *>(pages ? pages[page] : page0);
      const auto *k = reinterpret_cast<const std::uint16_t *>(src);
      const auto *v = reinterpret_cast<const std::uint16_t *>(src + values_offset);
      const Rows keys{k, k, kP, W};
      const Rows values{v, v, kP, W};
      page_task<Bits, HD>(static_cast<int>(lane % W), keys, values, kv_heads, dst, L, Emit::kCodes,
                          Emit::kCodes);
    }

    // The LDS quantiser for any other shape: a workgroup a page, the page
    // staged whole (quant_core::quantise_in_lds).
    template <int Bits>
    __global__ void __launch_bounds__(kThreads)
        requant_refs_lds_kernel(const RefPair *__restrict__ pairs, PageSpaces s, PageLayout L,
                                int page_tokens, int kv_heads, int head_dim)
    {
      extern __shared__ uint4 lds_raw[];
      const RefPair p = pairs[blockIdx.x];
      const std::size_t half = static_cast<std::size_t>(page_tokens) * kv_heads * head_dim * 2;
      auto *in = reinterpret_cast<std::uint8_t *>(lds_raw);
      std::uint8_t *out = in + ((2 * half + 15) / 16) * 16;
      quant_core::block_copy(in, resolve(s, p.from), 2 * half);
      __syncthreads();
      quant_core::quantise_in_lds<Bits>(reinterpret_cast<const std::uint16_t *>(in), out, L,
                                        page_tokens, kv_heads, head_dim);
      __syncthreads();
      quant_core::block_copy(resolve(s, p.to), out, L.page_bytes);
    }

    // ---- a store's row jobs ---------------------------------------------------

    struct RowJobs
    {
      RowJob job[kRowJobsALaunch];
      PageLayout lay[kTierCount];
    };

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

    // Job blockIdx.y, tasks blockIdx.x * 256 + tid (of W).
    template <int HD>
    __global__ void __launch_bounds__(kThreads) row_jobs_kernel(RowJobs jobs, int kv_heads)
    {
      const int task = blockIdx.x * kThreads + threadIdx.x;
      if (task >= kv_heads * HD)
      {
        return;
      }
      run_row_task<HD>(jobs.job[blockIdx.y], jobs.lay, task, kv_heads);
    }

    // A decode step's store, its position read on the device: the one row
    // fills row position % P of the open page, or, on a page's last row,
    // the page is sealed from the open page's rows and this one.
    template <int HD>
    __global__ void __launch_bounds__(kThreads) step_store_kernel(StepStore s)
    {
      const int task = blockIdx.x * kThreads + threadIdx.x;
      const int W = s.kv_heads * HD;
      if (task >= W)
      {
        return;
      }
      const int position = *s.position;
      const int row = position % kP;
      const int page = position / kP;
      RowJob j{};
      if (row < kP - 1)
      {
        j.kind = static_cast<int>(RowJobKind::kFill);
        j.k_lo = j.k_hi = s.keys;
        j.v_lo = j.v_hi = s.values;
        j.rows = 1;
        j.dst_row = row;
        j.dst = reinterpret_cast<std::uint8_t *>(s.open);
        j.tier = kFP16;
      }
      else
      {
        const int tier = s.tiers[page];
        j.kind = static_cast<int>(tier == kFP16 ? RowJobKind::kCopy : RowJobKind::kQuantise);
        j.k_lo = s.open;
        j.v_lo = s.open + static_cast<std::size_t>(kP) * W;
        j.k_hi = s.keys;
        j.v_hi = s.values;
        j.split = kP - 1;
        j.dst = reinterpret_cast<std::uint8_t *>(s.addresses[page]);
        j.tier = tier;
      }
      run_row_task<HD>(j, s.lay, task, s.kv_heads);
    }

    // The step's RoPE and its store in one workgroup: every (head, angle)
    // pair of q and k rotated into qk (the RoPE kernel's arithmetic, the
    // angle's cos and sin from the table), then, once the workgroup has
    // them, the store or seal of the rotated k row and the values.
    template <int HD>
    __global__ void __launch_bounds__(1024) step_rope_store_kernel(StepRopeStore s)
    {
      constexpr int kHalf = HD / 2;
      const int position = *s.store.position;
      const int pairs = (s.heads + s.store.kv_heads) * kHalf;
      const float *cs = s.rope + static_cast<std::size_t>(position) * kHalf * 2;
      for (int i = threadIdx.x; i < pairs; i += blockDim.x)
      {
        const int head = i / kHalf;
        const int j = i % kHalf;
        const std::size_t at = static_cast<std::size_t>(head) * HD + j;
        const float c = cs[2 * j];
        const float sn = cs[2 * j + 1];
        const float x1 = f16_bits(s.qk_raw[at]);
        const float x2 = f16_bits(s.qk_raw[at + kHalf]);
        s.qk[at] = static_cast<std::uint16_t>(half_of(x1 * c - x2 * sn));
        s.qk[at + kHalf] = static_cast<std::uint16_t>(half_of(x2 * c + x1 * sn));
      }
      __syncthreads();
      const int task = threadIdx.x;
      const int W = s.store.kv_heads * HD;
      if (task >= W)
      {
        return;
      }
      const std::uint16_t *keys = s.qk + static_cast<std::size_t>(s.heads) * HD;
      const int row = position % kP;
      const int page = position / kP;
      RowJob j{};
      if (row < kP - 1)
      {
        j.kind = static_cast<int>(RowJobKind::kFill);
        j.k_lo = j.k_hi = keys;
        j.v_lo = j.v_hi = s.store.values;
        j.rows = 1;
        j.dst_row = row;
        j.dst = reinterpret_cast<std::uint8_t *>(s.store.open);
        j.tier = kFP16;
      }
      else
      {
        const int tier = s.store.tiers[page];
        j.kind = static_cast<int>(tier == kFP16 ? RowJobKind::kCopy : RowJobKind::kQuantise);
        j.k_lo = s.store.open;
        j.v_lo = s.store.open + static_cast<std::size_t>(kP) * W;
        j.k_hi = keys;
        j.v_hi = s.store.values;
        j.split = kP - 1;
        j.dst = reinterpret_cast<std::uint8_t *>(s.store.addresses[page]);
        j.tier = tier;
      }
      run_row_task<HD>(j, s.store.lay, task, s.store.kv_heads);
    }

    // Any other shape: a workgroup a job, the rows staged in LDS.
    __global__ void __launch_bounds__(kThreads)
        row_jobs_lds_kernel(RowJobs jobs, int page_tokens, int kv_heads, int head_dim)
    {
      extern __shared__ uint4 lds_raw[];
      const RowJob &j = jobs.job[blockIdx.y];
      const RowJobKind kind = static_cast<RowJobKind>(j.kind);
      const int W = kv_heads * head_dim;
      const std::size_t half = static_cast<std::size_t>(page_tokens) * W;
      auto *rows = reinterpret_cast<std::uint16_t *>(lds_raw); // keys then values, FP16
      auto *out = reinterpret_cast<std::uint8_t *>(lds_raw) + ((4 * half + 15) / 16) * 16;
      auto *dst16 = reinterpret_cast<std::uint16_t *>(j.dst);
      if (kind == RowJobKind::kFill)
      {
        for (std::size_t i = threadIdx.x; i < static_cast<std::size_t>(j.rows) * W; i += kThreads)
        {
          const std::size_t at = static_cast<std::size_t>(j.dst_row) * W + i;
          dst16[at] = j.k_hi[i];
          dst16[half + at] = j.v_hi[i];
        }
        return;
      }
      for (std::size_t i = threadIdx.x; i < half; i += kThreads)
      {
        const int t = static_cast<int>(i / W);
        const std::size_t c = i % W;
        const std::size_t from = t < j.split ? i : static_cast<std::size_t>(t - j.split) * W + c;
        rows[i] = (t < j.split ? j.k_lo : j.k_hi)[from];
        rows[half + i] = (t < j.split ? j.v_lo : j.v_hi)[from];
      }
      __syncthreads();
      if (kind == RowJobKind::kCopy)
      {
        for (std::size_t i = threadIdx.x; i < 2 * half; i += kThreads)
        {
          dst16[i] = rows[i];
        }
        return;
      }
      const PageLayout &L = jobs.lay[j.tier];
      switch (L.bits)
      {
      case 8: quant_core::quantise_in_lds<8>(rows, out, L, page_tokens, kv_heads, head_dim); break;
      case 4: quant_core::quantise_in_lds<4>(rows, out, L, page_tokens, kv_heads, head_dim); break;
      default: quant_core::quantise_in_lds<2>(rows, out, L, page_tokens, kv_heads, head_dim); break;
      }
      __syncthreads();
      if (kind == RowJobKind::kQuantise)
      {
        quant_core::block_copy(j.dst, out, L.page_bytes);
        return;
      }
      // The Halves diagnostic: one half dequantised from the codes in LDS
      // (dequantise_page's rounding), the other as it came.
      const bool keys_round = kind == RowJobKind::kRoundKeys;
      const int bits = L.bits;
      const int per_byte = 8 / bits;
      const unsigned mask = (1u << bits) - 1;
      const auto meta = [&](std::size_t off) {
        return reinterpret_cast<const std::uint16_t *>(out + off);
      };
      for (std::size_t i = threadIdx.x; i < 2 * half; i += kThreads)
      {
        const bool is_key = i < half;
        if (is_key != keys_round)
        {
          dst16[i] = rows[i];
          continue;
        }
        const std::size_t e = is_key ? i : i - half;
        const std::uint8_t byte = out[(is_key ? L.key_codes : L.value_codes) + e / per_byte];
        const float q = static_cast<float>((byte >> ((e % per_byte) * bits)) & mask);
        const std::size_t group = is_key ? e % W : e / head_dim;
        const float s = half_bits_to_float(meta(is_key ? L.key_scales : L.value_scales)[group]);
        const float z = half_bits_to_float(meta(is_key ? L.key_zeros : L.value_zeros)[group]);
        dst16[i] = static_cast<std::uint16_t>(half_of(fmaf(q, s, z)));
      }
    }

    __global__ void table_edits_kernel(const TableEdit *__restrict__ edits, int count,
                                       unsigned long long *__restrict__ addresses,
                                       std::uint8_t *__restrict__ tiers)
    {
      const int i = blockIdx.x * blockDim.x + threadIdx.x;
      if (i < count)
      {
        const TableEdit e = edits[i];
        addresses[e.index] = e.address;
        tiers[e.index] = static_cast<std::uint8_t>(e.tier);
      }
    }

    bool register_shape(int page_tokens, int kv_heads, int head_dim)
    {
      return page_tokens == kP && (head_dim == 64 || head_dim == 128) &&
             kv_heads * head_dim >= 128;
    }

    template <typename F>
    void with_bits(int tier, F &&f)
    {
      switch (tier)
      {
      case kINT8: f(std::integral_constant<int, 8>{}); return;
      case kINT4: f(std::integral_constant<int, 4>{}); return;
      case kINT2: f(std::integral_constant<int, 2>{}); return;
      }
      throw InvalidArgument("FP16 is not a quantised tier: a move to it is a copy");
    }

    constexpr std::size_t kMaxLds = 160 * 1024;

    void allow_lds(const void *kernel, std::size_t lds, const char *what)
    {
      if (lds > kMaxLds)
      {
        throw InvalidArgument(std::string(what) + ": a page of these positions does not fit one "
                                                  "workgroup's LDS");
      }
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(kernel, hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute page jobs LDS");
      }
    }

  } // namespace

  void launch_copy_refs(const RefPair *pairs, int count, const PageSpaces &spaces,
                        hipStream_t stream)
  {
    if (count <= 0)
    {
      return;
    }
    // Pages are tens of KiB: a few workgroups each, the batch in y.
    for (int first = 0; first < count; first += 65535)
    {
      const int n = std::min(65535, count - first);
      hipLaunchKernelGGL(copy_refs_kernel, dim3(4, n), dim3(kThreads), 0, stream, pairs + first,
                         spaces);
      hip_check(hipGetLastError(), "copy refs kernel launch");
    }
  }

  void launch_requant_refs(const RefPair *pairs, int count, int tier, const PageSpaces &spaces,
                           int page_tokens, int kv_heads, int head_dim, hipStream_t stream)
  {
    if (count <= 0)
    {
      return;
    }
    const PageLayout L = page_layout(tier, page_tokens, kv_heads, head_dim);
    with_bits(tier, [&](auto bits) {
      constexpr int B = decltype(bits)::value;
      if (register_shape(page_tokens, kv_heads, head_dim))
      {
        const long long lanes = static_cast<long long>(count) * kv_heads * head_dim;
        const int blocks = static_cast<int>((lanes + kThreads - 1) / kThreads);
        if (head_dim == 128)
        {
          hipLaunchKernelGGL((requant_refs_kernel<B, 128>), dim3(blocks), dim3(kThreads), 0,
                             stream, pairs, count, spaces, L, kv_heads);
        }
        else
        {
          hipLaunchKernelGGL((requant_refs_kernel<B, 64>), dim3(blocks), dim3(kThreads), 0,
                             stream, pairs, count, spaces, L, kv_heads);
        }
        hip_check(hipGetLastError(), "requant refs kernel launch");
        return;
      }
      const std::size_t in = fp16_page_bytes(page_tokens, static_cast<std::size_t>(kv_heads) * head_dim);
      const std::size_t lds = ((in + 15) / 16) * 16 + ((L.page_bytes + 15) / 16) * 16;
      allow_lds(reinterpret_cast<const void *>(requant_refs_lds_kernel<B>), lds, "requantise");
      hipLaunchKernelGGL(requant_refs_lds_kernel<B>, dim3(count), dim3(kThreads), lds, stream,
                         pairs, spaces, L, page_tokens, kv_heads, head_dim);
      hip_check(hipGetLastError(), "requant refs (LDS) kernel launch");
    });
  }

  bool launch_quantise_registers(const void *const *rows, void *const *pages, const void *row0,
                                 void *page0, std::ptrdiff_t values_offset, int count, int tier,
                                 int page_tokens, int kv_heads, int head_dim, hipStream_t stream)
  {
    // The register tasks load 16 bytes at a time from every row.
    const bool aligned = row0 == nullptr ||
                         ((reinterpret_cast<std::uintptr_t>(row0) | values_offset) & 15) == 0;
    if (!register_shape(page_tokens, kv_heads, head_dim) || values_offset % 16 != 0 || !aligned)
    {
      return false;
    }
    if (count <= 0)
    {
      return true;
    }
    const PageLayout L = page_layout(tier, page_tokens, kv_heads, head_dim);
    const long long lanes = static_cast<long long>(count) * kv_heads * head_dim;
    const int blocks = static_cast<int>((lanes + kThreads - 1) / kThreads);
    with_bits(tier, [&](auto bits) {
      constexpr int B = decltype(bits)::value;
      if (head_dim == 128)
      {
        hipLaunchKernelGGL((quantise_ptrs_kernel<B, 128>), dim3(blocks), dim3(kThreads), 0, stream,
                           rows, pages, row0, page0, values_offset, count, L, kv_heads);
      }
      else
      {
        hipLaunchKernelGGL((quantise_ptrs_kernel<B, 64>), dim3(blocks), dim3(kThreads), 0, stream,
                           rows, pages, row0, page0, values_offset, count, L, kv_heads);
      }
      hip_check(hipGetLastError(), "quantise (registers) kernel launch");
    });
    return true;
  }

  void launch_row_jobs(const RowJob *jobs, int count, int page_tokens, int kv_heads, int head_dim,
                       hipStream_t stream)
  {
    RowJobs batch{};
    for (int i = 0; i < count; ++i)
    {
      const int t = jobs[i].tier;
      const auto kind = static_cast<RowJobKind>(jobs[i].kind);
      if (kind != RowJobKind::kCopy && kind != RowJobKind::kFill && batch.lay[t].bits == 0)
      {
        batch.lay[t] = page_layout(t, page_tokens, kv_heads, head_dim);
      }
    }
    const bool fast = register_shape(page_tokens, kv_heads, head_dim);
    const std::size_t half = static_cast<std::size_t>(page_tokens) * kv_heads * head_dim;
    std::size_t lds = 0;
    if (!fast)
    {
      std::size_t largest = 0;
      for (const PageLayout &L : batch.lay)
      {
        largest = std::max(largest, L.page_bytes);
      }
      lds = ((4 * half + 15) / 16) * 16 + ((largest + 15) / 16) * 16;
      allow_lds(reinterpret_cast<const void *>(row_jobs_lds_kernel), lds, "store");
    }
    for (int first = 0; first < count; first += kRowJobsALaunch)
    {
      const int n = std::min(kRowJobsALaunch, count - first);
      std::copy(jobs + first, jobs + first + n, batch.job);
      if (fast)
      {
        const int blocks = static_cast<int>((static_cast<long long>(kv_heads) * head_dim + kThreads - 1) /
                                            kThreads);
        if (head_dim == 128)
        {
          hipLaunchKernelGGL(row_jobs_kernel<128>, dim3(blocks, n), dim3(kThreads), 0, stream,
                             batch, kv_heads);
        }
        else
        {
          hipLaunchKernelGGL(row_jobs_kernel<64>, dim3(blocks, n), dim3(kThreads), 0, stream,
                             batch, kv_heads);
        }
      }
      else
      {
        hipLaunchKernelGGL(row_jobs_lds_kernel, dim3(1, n), dim3(kThreads), lds, stream, batch,
                           page_tokens, kv_heads, head_dim);
      }
      hip_check(hipGetLastError(), "row jobs kernel launch");
    }
  }

  void launch_step_store(const StepStore &s, int head_dim, hipStream_t stream)
  {
    if (!register_shape(kP, s.kv_heads, head_dim))
    {
      throw InvalidArgument("a store whose position lives on the device takes head_dim 64 or 128 "
                            "and at least 128 channels a row");
    }
    StepStore args = s;
    for (int t = kINT8; t <= kINT2; ++t)
    {
      args.lay[t] = page_layout(t, kP, s.kv_heads, head_dim);
    }
    const int blocks = (s.kv_heads * head_dim + kThreads - 1) / kThreads;
    if (head_dim == 128)
    {
      hipLaunchKernelGGL(step_store_kernel<128>, dim3(blocks), dim3(kThreads), 0, stream, args);
    }
    else
    {
      hipLaunchKernelGGL(step_store_kernel<64>, dim3(blocks), dim3(kThreads), 0, stream, args);
    }
    hip_check(hipGetLastError(), "step store kernel launch");
  }

  void launch_step_rope_store(const StepRopeStore &s, int head_dim, hipStream_t stream)
  {
    const int W = s.store.kv_heads * head_dim;
    if (!register_shape(kP, s.store.kv_heads, head_dim) || W > 1024 || s.rope == nullptr ||
        s.heads <= 0)
    {
      throw InvalidArgument("the step's RoPE and store in one launch take head_dim 64 or 128, "
                            "128 to 1024 channels a row and a RoPE table");
    }
    StepRopeStore args = s;
    for (int t = kINT8; t <= kINT2; ++t)
    {
      args.store.lay[t] = page_layout(t, kP, s.store.kv_heads, head_dim);
    }
    const int threads = (W + 63) / 64 * 64;
    if (head_dim == 128)
    {
      hipLaunchKernelGGL(step_rope_store_kernel<128>, dim3(1), dim3(threads), 0, stream, args);
    }
    else
    {
      hipLaunchKernelGGL(step_rope_store_kernel<64>, dim3(1), dim3(threads), 0, stream, args);
    }
    hip_check(hipGetLastError(), "step RoPE + store kernel launch");
  }

  void launch_table_edits(const TableEdit *edits, int count, unsigned long long *addresses,
                          std::uint8_t *tiers, hipStream_t stream)
  {
    if (count <= 0)
    {
      return;
    }
    hipLaunchKernelGGL(table_edits_kernel, dim3((count + kThreads - 1) / kThreads), dim3(kThreads),
                       0, stream, edits, count, addresses, tiers);
    hip_check(hipGetLastError(), "table edits kernel launch");
  }

} // namespace mi
