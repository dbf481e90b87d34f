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
// The register quantiser's tasks (page_tasks.hpp): a 32-token page is W =
// kv_heads * head_dim tasks of 64 elements, a lane each, none staged through
// LDS. Every input byte is read once and every output byte written once; a
// page is W lanes (a workgroup of 256 covers one 1.5B page, two 0.5B pages),
// so a batch of pages fills the device with no serial walk over rows.

#include "common.hpp"
#include "kernels.hpp"
#include "page_tasks.hpp"
#include "quant_core.hpp"

#include <algorithm>

namespace mi
{
  namespace
  {
    constexpr int kThreads = 256;
    using namespace page_tasks;

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

    // ---- batches by reference ------------------------------------------------

    __device__ inline RefPair ref_at(const RefList &l, long long i)
    {
      if (l.pairs != nullptr)
      {
        return l.pairs[i];
      }
      RefPair p = l.held[0];
#pragma unroll
      for (int k = 1; k < kHeldRefs; ++k)
      {
        p = i == k ? l.held[k] : p;
      }
      return p;
    }

    // Page blockIdx.y of the batch: the blocks of x stride over its bytes.
    __global__ void __launch_bounds__(kThreads)
        copy_refs_kernel(RefList pairs, int first, PageSpaces s)
    {
      const RefPair p = ref_at(pairs, first + blockIdx.y);
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
        requant_refs_kernel(RefList pairs, int count, PageSpaces s, PageLayout L, int kv_heads)
    {
      const int W = kv_heads * HD;
      const long long lane = static_cast<long long>(blockIdx.x) * kThreads + threadIdx.x;
      const long long pair = lane / W;
      if (pair >= count)
      {
        return; // whole waves: W is a multiple of 64
      }
      const RefPair p = ref_at(pairs, pair);
      const auto *src = reinterpret_cast<const std::uint16_t *>(resolve(s, p.from));
      std::uint8_t *dst = resolve(s, p.to);
      const Rows keys{src, src, kP, W};
      const Rows values{src + static_cast<std::size_t>(kP) * W, src + static_cast<std::size_t>(kP) * W,
                        kP, W};
      page_task<Bits, HD>(static_cast<int>(lane % W), keys, values, kv_heads, dst, L, Emit::kCodes,
                          Emit::kCodes);
    }

    // A workgroup's copy of one page's bytes, 16 bytes a thread a pass and
    // any last bytes one by one. Up to kCopyBatch passes' loads are issued
    // before any of their stores, so that a page (32 KiB: 8 passes) is one
    // trip to its source, not a trip a pass: the source may be host memory
    // or the far side of the device, and a store may alias a later load
    // for all the compiler knows. A thread past the last unit copies the
    // last unit again (the same bytes to the same place), so that nothing
    // in the batch is conditional: a branch's join would wait for its load.
    constexpr int kCopyBatch = 8;
    __device__ inline void block_copy_page(std::uint8_t *dst, const std::uint8_t *src,
                                           unsigned long long bytes)
    {
      typedef unsigned copy_unit __attribute__((ext_vector_type(4)));
      const unsigned long long units = bytes / 16;
      for (unsigned long long base = 0; base < units; base += kCopyBatch * kThreads)
      {
        copy_unit v[kCopyBatch];
#pragma unroll
        for (int j = 0; j < kCopyBatch; ++j)
        {
          const unsigned long long i = base + j * kThreads + threadIdx.x;
          v[j] = reinterpret_cast<const copy_unit *>(src)[i < units ? i : units - 1];
        }
#pragma unroll
        for (int j = 0; j < kCopyBatch; ++j)
        {
          const unsigned long long i = base + j * kThreads + threadIdx.x;
          reinterpret_cast<copy_unit *>(dst)[i < units ? i : units - 1] = v[j];
        }
      }
      if (threadIdx.x < bytes % 16)
      {
        dst[16 * units + threadIdx.x] = src[16 * units + threadIdx.x];
      }
    }

    // One page's move (OneMove), a workgroup: the shadow copy, the shadow's
    // rows staged (then a barrier, so that every wave reads them whole), and
    // the page at its new tier (the register quantiser, its W tasks over the
    // workgroup's lanes; Bits 16: a copy at FP16), then, after the barrier
    // that waits for every read of the old page, the compaction copies. The
    // launch is one workgroup, so its registers are not capped for occupancy
    // (the batch quantiser's four waves a SIMD would spill its tasks here).
    template <int Bits, int HD>
    __global__ void __launch_bounds__(kThreads)
        move_one_kernel(OneMove m, PageSpaces s, PageLayout L, int kv_heads)
    {
      if (m.has_shadow)
      {
        block_copy_page(reinterpret_cast<std::uint8_t *>(m.shadow_at), resolve(s, m.shadow.from),
                        s.shadow_bytes);
      }
      if (m.has_stage)
      {
        block_copy_page(resolve(s, m.stage.to), resolve(s, m.stage.from), s.shadow_bytes);
        __syncthreads();
      }
      if constexpr (Bits == 16)
      {
        block_copy_page(resolve(s, m.page.to), resolve(s, m.page.from), s.shadow_bytes);
      }
      else
      {
        const int W = kv_heads * HD;
        const auto *src = reinterpret_cast<const std::uint16_t *>(resolve(s, m.page.from));
        std::uint8_t *dst = resolve(s, m.page.to);
        const Rows keys{src, src, kP, W};
        const Rows values{src + static_cast<std::size_t>(kP) * W,
                          src + static_cast<std::size_t>(kP) * W, kP, W};
        for (int task = threadIdx.x; task < W; task += kThreads)
        {
          page_task<Bits, HD>(task, keys, values, kv_heads, dst, L, Emit::kCodes, Emit::kCodes);
        }
      }
      __syncthreads();
      for (int k = 0; k < m.compact_count; ++k)
      {
        const RefPair p = m.compact[k];
        block_copy_page(resolve(s, p.to), resolve(s, p.from), page_size(s, p.to));
      }
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
        requant_refs_lds_kernel(RefList pairs, PageSpaces s, PageLayout L, int page_tokens,
                                int kv_heads, int head_dim)
    {
      extern __shared__ uint4 lds_raw[];
      const RefPair p = ref_at(pairs, blockIdx.x);
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

  RefList ref_list(const std::vector<RefPair> &host, std::size_t first, std::size_t count,
                   const RefPair *uploaded)
  {
    RefList l{};
    if (count > static_cast<std::size_t>(kHeldRefs))
    {
      l.pairs = uploaded + first;
      return l;
    }
    for (std::size_t i = 0; i < count; ++i)
    {
      l.held[i] = host[first + i];
    }
    return l;
  }

  void launch_copy_refs(const RefList &pairs, int count, const PageSpaces &spaces,
                        hipStream_t stream)
  {
    if (count <= 0)
    {
      return;
    }
    if (pairs.pairs == nullptr && count > kHeldRefs)
    {
      throw InvalidArgument("a copy launch holds at most " + std::to_string(kHeldRefs) +
                            " pairs in its arguments; got " + std::to_string(count));
    }
    // Pages are tens of KiB: a few workgroups each, the batch in y.
    for (int first = 0; first < count; first += 65535)
    {
      const int n = std::min(65535, count - first);
      hipLaunchKernelGGL(copy_refs_kernel, dim3(4, n), dim3(kThreads), 0, stream, pairs, first,
                         spaces);
      hip_check(hipGetLastError(), "copy refs kernel launch");
    }
  }

  bool move_one_applies(int from, int tier, int page_tokens, int kv_heads, int head_dim)
  {
    // A move from a shadow reads host memory, a page in one trip (the
    // copies issue a batch of loads before their stores).
    return from != tier && register_shape(page_tokens, kv_heads, head_dim);
  }

  bool launch_move_one(const OneMove &m, const PageSpaces &spaces, int page_tokens, int kv_heads,
                       int head_dim, hipStream_t stream)
  {
    if (m.compact_count < 0 || m.compact_count > kHeldRefs)
    {
      throw InvalidArgument("a move's launch holds at most " + std::to_string(kHeldRefs) +
                            " compaction copies; got " + std::to_string(m.compact_count));
    }
    if (!register_shape(page_tokens, kv_heads, head_dim))
    {
      return false;
    }
    if (m.tier == kFP16)
    {
      // A restore: the shadow's rows copied into the new page.
      const PageLayout none{};
      if (head_dim == 128)
      {
        hipLaunchKernelGGL((move_one_kernel<16, 128>), dim3(1), dim3(kThreads), 0, stream, m,
                           spaces, none, kv_heads);
      }
      else
      {
        hipLaunchKernelGGL((move_one_kernel<16, 64>), dim3(1), dim3(kThreads), 0, stream, m,
                           spaces, none, kv_heads);
      }
      hip_check(hipGetLastError(), "move kernel launch");
      return true;
    }
    const PageLayout L = page_layout(m.tier, page_tokens, kv_heads, head_dim);
    with_bits(m.tier, [&](auto bits) {
      constexpr int B = decltype(bits)::value;
      if (head_dim == 128)
      {
        hipLaunchKernelGGL((move_one_kernel<B, 128>), dim3(1), dim3(kThreads), 0, stream, m,
                           spaces, L, kv_heads);
      }
      else
      {
        hipLaunchKernelGGL((move_one_kernel<B, 64>), dim3(1), dim3(kThreads), 0, stream, m,
                           spaces, L, kv_heads);
      }
    });
    hip_check(hipGetLastError(), "move kernel launch");
    return true;
  }

  void launch_requant_refs(const RefList &pairs, int count, int tier, const PageSpaces &spaces,
                           int page_tokens, int kv_heads, int head_dim, hipStream_t stream)
  {
    if (count <= 0)
    {
      return;
    }
    if (pairs.pairs == nullptr && count > kHeldRefs)
    {
      throw InvalidArgument("a requantise launch holds at most " + std::to_string(kHeldRefs) +
                            " pairs in its arguments; got " + std::to_string(count));
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
