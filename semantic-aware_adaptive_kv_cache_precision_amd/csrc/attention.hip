// Attention over the KV cache for every layout and any number of queries:
// the general path, for the shapes the decode kernel (decode.hip) and the
// matrix-core chunk kernel (prefill.hip) do not take -- pages of other than
// 32 tokens, head dims other than 64 and 128, rows that are not 16-byte
// aligned, a decode's per-page mass over a contiguous cache.
//
// Semantics are the reference's attention (src/core_kernels/attention.cu):
//   - softmax(q k^T / sqrt(d)) v with the scores and the accumulation in
//     fp32, query i of seq_q at position seq_k - seq_q + i seeing the keys up
//     to its own (:449-540); query head h reads KV head h / (heads / kv_heads);
//   - a key the query may not see contributes nothing, and its bytes are not
//     read, so a NaN there cannot reach the output (:574-589); a row that
//     sees no key at all gives zeros (:597-615);
//   - a cache that seals: every page before a query's own is read at the
//     tier its table records and dequantised as dequantise_page does, an
//     unread page (tier 0xFF) not at all, and the query's own page at FP16
//     from the open page and the chunk's rows (:122-364);
//   - the key bias completes key j as k + RoPE(bias, j), from the fp32
//     {cos, sin} table (:104-116);
//   - a decode query's per-page mass, each page's share of its softmax
//     (:375-411); a contiguous cache's pages are 32 keys.
//
// Work layout (this build's own): a workgroup of 256 lanes owns one
// (query, head) and one run of keys (a split), and walks the run a tile of
// whole pages at a time. In a tile every lane scores keys (q, pre-scaled,
// from LDS against the key's row, widened and dequantised an element at a
// time), the tile's maximum and the running softmax are formed once for the
// workgroup, and then each lane owns one output channel and adds the tile's
// weighted values for it: the lanes read a value row together, coalesced.
// For the mass, each page keeps the sum of its weights and the maximum they
// are relative to. A launch of several runs writes each run's (m, l, o); the
// combine folds them and forms the masses at the folded maximum.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>

namespace mi
{
  namespace
  {
    constexpr int kThreads = 256;
    constexpr int kContiguousPage = 32; // a contiguous cache's pages, for the mass
    constexpr int kTileKeys = 256;      // keys a tile holds (whole pages; a larger page alone)
    constexpr int kMaxTile = 4096;
    constexpr int kBlocksPerCU = 8;
    constexpr int kMinSplitKeys = 256;
    constexpr int kPartialSlotsPerCU = kBlocksPerCU * 16;

    struct GeneralArgs
    {
      KVSource src;
      PageLayout lay[kTierCount];
      const std::uint16_t *q;   // (seq_q, heads, hd)
      std::uint16_t *out;       // (seq_q, heads, hd)
      const std::uint16_t *k_bias;
      const float *rope;
      int seq_q;
      int seq_k;
      int heads;
      int kv_heads;
      int hd;
      int mass_page; // keys a mass page holds
      int tile;      // keys a tile holds: whole mass pages
      int splits;
      int split_keys;
      float *partials;   // [query][head][split][2 + hd] when splits > 1
      float *page_stats; // [head][page][2]: a page's (base, sum of exp(s - base)); with mass
      float *mass;       // [head][page]; with mass
    };

    // Where key j's row is, for reading it an element at a time.
    struct Row
    {
      const std::uint16_t *k; // FP16 rows (null for a quantised page)
      const std::uint16_t *v;
      const std::uint8_t *page; // a quantised page, its tier and the key's row in it
      int tier;
      int t;
    };

    __device__ inline Row row_of(const GeneralArgs &a, int j, int own)
    {
      const KVSource &s = a.src;
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * a.hd;
      Row r{};
      r.tier = kFP16;
      if (s.layout == Layout::kContiguous)
      {
        r.k = s.k + j * W;
        r.v = s.v + j * W;
        return r;
      }
      const int P = s.page_tokens;
      const int p = j / P;
      const int t = j % P;
      if (s.layout == Layout::kPaged || p < own)
      {
        const int tier = s.layout == Layout::kPaged ? static_cast<int>(kFP16) : s.tiers[p];
        if (tier == kFP16)
        {
          const auto *h = reinterpret_cast<const std::uint16_t *>(s.pages[p]);
          r.k = h + t * W;
          r.v = h + (P + t) * W;
          return r;
        }
        r.page = reinterpret_cast<const std::uint8_t *>(s.pages[p]);
        r.tier = tier;
        r.t = t;
        return r;
      }
      // The query's own page: rows before `start` in the open page, the rest
      // the chunk's.
      if (j >= s.start)
      {
        r.k = s.chunk_k + (j - s.start) * W;
        r.v = s.chunk_v + (j - s.start) * W;
      }
      else
      {
        r.k = s.open + t * W;
        r.v = s.open + (P + t) * W;
      }
      return r;
    }

    // Whether key j is read: a page sealed before the own page may be unread.
    __device__ inline bool readable(const GeneralArgs &a, int j, int own)
    {
      if (a.src.layout != Layout::kCausal)
      {
        return true;
      }
      const int p = j / a.src.page_tokens;
      return p >= own || a.src.tiers[p] != kUnreadPage;
    }

    // code * scale + zero rounded as dequantise_page rounds it (fp32 fma,
    // then fp16).
    __device__ inline float dequantised(const std::uint8_t *page, std::size_t codes,
                                        std::size_t e, int bits, std::size_t scale,
                                        std::size_t zero, std::size_t group)
    {
      const int per_byte = 8 / bits;
      const unsigned byte = page[codes + e / per_byte];
      const unsigned code = (byte >> ((e % per_byte) * bits)) & ((1u << bits) - 1);
      const auto *s = reinterpret_cast<const std::uint16_t *>(page + scale);
      const auto *z = reinterpret_cast<const std::uint16_t *>(page + zero);
      return h2f(__half_as_ushort(
          __float2half_rn(fmaf(static_cast<float>(code), h2f(s[group]), h2f(z[group])))));
    }

    // Element `at` (of the row's kv_heads * hd) of the key, or of the value.
    __device__ inline float key_at(const GeneralArgs &a, const Row &r, std::size_t at)
    {
      if (r.page == nullptr)
      {
        return h2f(r.k[at]);
      }
      const PageLayout &L = a.lay[r.tier];
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * a.hd;
      return dequantised(r.page, L.key_codes, r.t * W + at, L.bits, L.key_scales, L.key_zeros, at);
    }

    __device__ inline float value_at(const GeneralArgs &a, const Row &r, std::size_t at)
    {
      if (r.page == nullptr)
      {
        return h2f(r.v[at]);
      }
      const PageLayout &L = a.lay[r.tier];
      const std::size_t W = static_cast<std::size_t>(a.kv_heads) * a.hd;
      const std::size_t group = static_cast<std::size_t>(r.t) * a.kv_heads + at / a.hd;
      return dequantised(r.page, L.value_codes, r.t * W + at, L.bits, L.value_scales,
                         L.value_zeros, group);
    }

    // Element c of the key bias turned to position j (rotate-half: channel
    // c pairs with c +- hd/2), from the {cos, sin} table.
    __device__ inline float bias_at(const std::uint16_t *bias, const float *rope, int j, int c,
                                    int hd)
    {
      const int half = hd / 2;
      const int i = c % half;
      const float *cs = rope + 2 * (static_cast<std::size_t>(j) * half + i);
      const float x = h2f(bias[i]);
      const float y = h2f(bias[i + half]);
      return c < half ? x * cs[0] - y * cs[1] : y * cs[0] + x * cs[1];
    }

    __global__ void __launch_bounds__(kThreads) general_attention_kernel(GeneralArgs a)
    {
      extern __shared__ float lds[];
      float *q_s = lds;              // hd: q * 1/sqrt(hd)
      float *w_s = q_s + a.hd;       // tile: the keys' scores, then their weights
      float *red = w_s + a.tile;     // a float a wave
      const int tid = threadIdx.x;
      const int query = blockIdx.x / a.heads;
      const int head = blockIdx.x % a.heads;
      const int split = blockIdx.y;
      const int kvh = head / (a.heads / a.kv_heads);
      const int position = a.seq_k - a.seq_q + query;
      const int own = a.src.layout == Layout::kContiguous ? 0 : position / a.src.page_tokens;
      const std::size_t at0 = static_cast<std::size_t>(kvh) * a.hd;
      const std::uint16_t *bias = a.k_bias != nullptr ? a.k_bias + at0 : nullptr;
      const float scale = 1.0f / sqrtf(static_cast<float>(a.hd));
      for (int c = tid; c < a.hd; c += kThreads)
      {
        q_s[c] = h2f(a.q[(static_cast<std::size_t>(query) * a.heads + head) * a.hd + c]) * scale;
      }
      const int k0 = split * a.split_keys;
      const int k1 = min(k0 + a.split_keys, position + 1);
      const bool with_mass = a.page_stats != nullptr;
      float m = -INFINITY, l = 0.0f, o = 0.0f; // o: lane tid's channel
      __syncthreads();
      for (int t0 = k0; t0 < k1; t0 += a.tile)
      {
        const int n = min(a.tile, k1 - t0);
        for (int u = tid; u < n; u += kThreads)
        {
          const int j = t0 + u;
          float score = -INFINITY;
          if (readable(a, j, own))
          {
            const Row r = row_of(a, j, own);
            float acc = 0.0f;
            for (int c = 0; c < a.hd; ++c)
            {
              float k = key_at(a, r, at0 + c);
              if (bias != nullptr)
              {
                k += bias_at(bias, a.rope, j, c, a.hd);
              }
              acc = fmaf(q_s[c], k, acc);
            }
            score = acc;
          }
          w_s[u] = score;
        }
        __syncthreads();
        float top = -INFINITY;
        for (int u = tid; u < n; u += kThreads)
        {
          top = fmaxf(top, w_s[u]);
        }
        top = block_reduce<true>(top, red);
        const float m_new = fmaxf(m, top);
        const float base = m_new == -INFINITY ? 0.0f : m_new;
        const float keep = expf(m - base); // 0 before the first visible key
        float part = 0.0f;
        for (int u = tid; u < n; u += kThreads)
        {
          const float w = expf(w_s[u] - base); // 0 for a key not seen
          w_s[u] = w;
          part += w;
        }
        part = block_reduce<false>(part, red); // its barriers publish the weights
        l = l * keep + part;
        if (with_mass && query == 0)
        {
          const int first = t0 / a.mass_page;
          const int pages = (n + a.mass_page - 1) / a.mass_page;
          for (int p = tid; p < pages; p += kThreads)
          {
            float sum = 0.0f;
            const int end = min((p + 1) * a.mass_page, n);
            for (int u = p * a.mass_page; u < end; ++u)
            {
              sum += w_s[u];
            }
            const std::size_t at = (static_cast<std::size_t>(head) *
                                        ((a.seq_k + a.mass_page - 1) / a.mass_page) +
                                    first + p) * 2;
            a.page_stats[at] = base;
            a.page_stats[at + 1] = sum;
          }
        }
        if (tid < a.hd)
        {
          float acc = 0.0f;
          for (int u = 0; u < n; ++u)
          {
            const float w = w_s[u];
            if (w != 0.0f)
            {
              acc = fmaf(w, value_at(a, row_of(a, t0 + u, own), at0 + tid), acc);
            }
          }
          o = o * keep + acc;
        }
        m = m_new;
        __syncthreads(); // the next tile's scores overwrite the weights
      }
      const std::size_t row = static_cast<std::size_t>(query) * a.heads + head;
      if (a.splits > 1)
      {
        float *slot = a.partials + (row * a.splits + split) * (2 + a.hd);
        if (tid == 0)
        {
          slot[0] = m;
          slot[1] = l;
        }
        if (tid < a.hd)
        {
          slot[2 + tid] = o;
        }
        return;
      }
      if (tid < a.hd)
      {
        a.out[row * a.hd + tid] = __half_as_ushort(__float2half(l > 0.0f ? o / l : 0.0f));
      }
      if (with_mass)
      {
        // The page statistics this workgroup wrote are visible to it after
        // the loop's last barrier.
        const int pages = (a.seq_k + a.mass_page - 1) / a.mass_page;
        for (int p = tid; p < pages; p += kThreads)
        {
          const float *st = a.page_stats + (static_cast<std::size_t>(head) * pages + p) * 2;
          a.mass[static_cast<std::size_t>(head) * pages + p] =
              l > 0.0f ? st[1] * expf(st[0] - m) / l : 0.0f;
        }
      }
    }

    // The runs of a (query, head) folded: M = max m_s, L = sum l_s e^(m_s - M),
    // out = sum o_s e^(m_s - M) / L; a decode's page masses from their page
    // statistics at M. A workgroup a (query, head), a lane a channel.
    __global__ void __launch_bounds__(kThreads) general_combine_kernel(GeneralArgs a)
    {
      __shared__ float red[kThreads / 64];
      const int tid = threadIdx.x;
      const std::size_t row = blockIdx.x;
      const int head = static_cast<int>(row % a.heads);
      const float *slots = a.partials + row * a.splits * (2 + a.hd);
      float top = -INFINITY;
      for (int s = tid; s < a.splits; s += kThreads)
      {
        top = fmaxf(top, slots[s * (2 + a.hd)]);
      }
      top = block_reduce<true>(top, red);
      const float base = top == -INFINITY ? 0.0f : top;
      float l = 0.0f, o = 0.0f;
      for (int s = 0; s < a.splits; ++s)
      {
        const float *slot = slots + s * (2 + a.hd);
        const float w = expf(slot[0] - base); // 0 for a run that saw no key
        l += slot[1] * w;
        if (tid < a.hd)
        {
          o += slot[2 + tid] * w;
        }
      }
      if (tid < a.hd)
      {
        a.out[row * a.hd + tid] = __half_as_ushort(__float2half(l > 0.0f ? o / l : 0.0f));
      }
      if (a.page_stats != nullptr && row < static_cast<std::size_t>(a.heads))
      {
        const int pages = (a.seq_k + a.mass_page - 1) / a.mass_page;
        for (int p = tid; p < pages; p += kThreads)
        {
          const float *st = a.page_stats + (static_cast<std::size_t>(head) * pages + p) * 2;
          a.mass[static_cast<std::size_t>(head) * pages + p] =
              l > 0.0f ? st[1] * expf(st[0] - top) / l : 0.0f;
        }
      }
    }

    int ceil_div(int a, int b) { return (a + b - 1) / b; }

    // Keys a tile holds: whole mass pages, about kTileKeys of them.
    int tile_for(int mass_page)
    {
      return mass_page >= kTileKeys ? mass_page : mass_page * (kTileKeys / mass_page);
    }

    int partial_slots() { return kPartialSlotsPerCU * device_multiprocessors(); }

    // Runs of whole tiles: enough workgroups to fill the device, none
    // shorter than kMinSplitKeys, every (query, head, run) a partial slot.
    Split split_for(int seq_q, int seq_k, int heads, int tile, bool may_split)
    {
      const int whole = ceil_div(std::max(seq_k, 1), tile) * tile;
      if (!may_split)
      {
        return {1, whole};
      }
      const long rows = static_cast<long>(seq_q) * heads;
      const long fill = (static_cast<long>(kBlocksPerCU) * device_multiprocessors() + rows - 1) /
                        std::max(rows, 1L);
      const long splits = std::min({fill, static_cast<long>(seq_k / kMinSplitKeys),
                                    static_cast<long>(partial_slots()) / std::max(rows, 1L)});
      if (splits <= 1)
      {
        return {1, whole};
      }
      const int keys = ceil_div(ceil_div(seq_k, static_cast<int>(splits)), tile) * tile;
      return {ceil_div(seq_k, keys), keys};
    }

    int mass_page_of(const KVSource &kv)
    {
      return kv.layout == Layout::kContiguous ? kContiguousPage : kv.page_tokens;
    }

    void check_grouping(int heads, int kv_heads)
    {
      if (heads < 0 || kv_heads < 0 || (heads == 0) != (kv_heads == 0))
      {
        throw InvalidArgument(std::to_string(heads) + " query heads and " +
                              std::to_string(kv_heads) +
                              " KV heads: either both are zero or neither is");
      }
      if (kv_heads > 0 && heads % kv_heads != 0)
      {
        throw InvalidArgument(std::to_string(heads) + " query heads and " +
                              std::to_string(kv_heads) +
                              " KV heads: the KV head count must divide the query head count");
      }
    }

  } // namespace

  int device_multiprocessors()
  {
    static const int count = [] {
      int device = 0, n = 0;
      hip_check(hipGetDevice(&device), "hipGetDevice");
      hip_check(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, device),
                "hipDeviceGetAttribute multiprocessor count");
      return n;
    }();
    return count;
  }

  std::size_t attention_partials_floats(int head_dim)
  {
    return static_cast<std::size_t>(partial_slots()) * (static_cast<std::size_t>(head_dim) + 2);
  }

  Split attention_split(int seq_q, int seq_k, int heads, int kv_heads, int page_tokens)
  {
    check_grouping(heads, kv_heads);
    const int mass_page = page_tokens > 0 ? page_tokens : kContiguousPage;
    return split_for(seq_q, seq_k, heads, tile_for(mass_page), true);
  }

  bool launch_decode_fast(const KVSource &kv, const AttentionArgs &a, hipStream_t stream);

  void launch_attention(const KVSource &kv, const AttentionArgs &a, hipStream_t stream)
  {
    check_grouping(a.heads, a.kv_heads);
    if ((a.mass != nullptr || a.scores != nullptr) && a.seq_q != 1)
    {
      throw InvalidArgument("the per-page attention mass is a decode step's, of one query; got " +
                            std::to_string(a.seq_q) + " queries");
    }
    if (a.seq_q <= 0 || a.heads == 0 || a.head_dim <= 0)
    {
      return;
    }
    if (a.head_dim % 2 != 0 || a.head_dim > kMaxHeadDim)
    {
      throw InvalidArgument("head_dim must be even and at most " + std::to_string(kMaxHeadDim) +
                            "; got " + std::to_string(a.head_dim));
    }
    if (a.k_bias != nullptr && (a.rope == nullptr || a.rope_positions < a.seq_k))
    {
      throw InvalidArgument("a key bias needs a RoPE table for head_dim " +
                            std::to_string(a.head_dim) + " covering " + std::to_string(a.seq_k) +
                            " positions");
    }
    if (launch_decode_fast(kv, a, stream))
    {
      return;
    }
    if (prefill_applies(kv, a))
    {
      launch_prefill(kv, a, stream);
      return;
    }
    GeneralArgs g{};
    g.src = kv;
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        g.lay[t] = page_layout(t, kv.page_tokens, a.kv_heads, a.head_dim);
      }
    }
    g.q = a.q;
    g.out = a.out;
    g.k_bias = a.k_bias;
    g.rope = a.k_bias != nullptr ? a.rope : nullptr;
    g.seq_q = a.seq_q;
    g.seq_k = a.seq_k;
    g.heads = a.heads;
    g.kv_heads = a.kv_heads;
    g.hd = a.head_dim;
    g.mass_page = mass_page_of(kv);
    g.tile = tile_for(g.mass_page);
    if (g.tile > kMaxTile)
    {
      throw InvalidArgument("pages of " + std::to_string(g.mass_page) +
                            " tokens are more than the general attention path takes (" +
                            std::to_string(kMaxTile) + ")");
    }
    const Split split = split_for(a.seq_q, a.seq_k, a.heads, g.tile, a.partials != nullptr);
    g.splits = split.splits;
    g.split_keys = split.split_keys;
    g.partials = a.partials;
    const bool with_mass = a.mass != nullptr || a.scores != nullptr;
    const int pages = (a.seq_k + g.mass_page - 1) / g.mass_page;
    if (with_mass)
    {
      // The page statistics, and the mass itself when the caller wants only
      // the scores, in scratch.
      const std::size_t stats = static_cast<std::size_t>(a.heads) * pages * 2;
      const std::size_t own_mass = a.mass == nullptr ? static_cast<std::size_t>(a.heads) * pages : 0;
      float *scratch = a.workspace != nullptr ? a.workspace->floats(stats + own_mass)
                                              : stream_workspace(stream, stats + own_mass);
      g.page_stats = scratch;
      g.mass = a.mass != nullptr ? a.mass : scratch + stats;
    }
    const std::size_t lds = (static_cast<std::size_t>(a.head_dim) + g.tile + kThreads / 64) *
                            sizeof(float);
    hipLaunchKernelGGL(general_attention_kernel, dim3(a.seq_q * a.heads, g.splits), dim3(kThreads),
                       lds, stream, g);
    hip_check(hipGetLastError(), "attention kernel launch");
    if (g.splits > 1)
    {
      hipLaunchKernelGGL(general_combine_kernel, dim3(a.seq_q * a.heads), dim3(kThreads), 0,
                         stream, g);
      hip_check(hipGetLastError(), "attention combine kernel launch");
    }
    if (a.scores != nullptr)
    {
      launch_fold(a.scores, g.mass, a.heads, pages, a.alpha, stream);
    }
  }

} // namespace mi
