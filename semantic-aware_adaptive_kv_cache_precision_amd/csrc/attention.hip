// Attention over the KV cache: the general kernel, for every layout and any
// number of queries, with the split-K combine.
//
// Semantics follow the reference (src/core_kernels/attention.cu):
//   - online softmax over key tiles of 32, scale folded into q in fp32
//     (:449-540), scores masked by select so a NaN in a masked key cannot
//     leak (:574-589), the -inf-row guard (:597-615);
//   - GQA rows: query head h reads KV head h / (heads / kv_heads) (:85-90);
//   - three layouts (:122-364): contiguous, an FP16 page table, and a cache
//     that seals, whose pages before a query's own are read at the tier the
//     table records and dequantised in registers exactly as dequantise_page
//     does, the own page read at FP16 from the open page and the chunk rows;
//   - key bias completed as k + RoPE(k_bias, j) from the cos/sin table (:104-116);
//   - per-page attention mass of a decode step's one query (:375-411, :697-745);
//   - split-K runs folded by the combine kernel (:754-815).
//
// Where this departs from the reference's shape (not its arithmetic): split
// runs are whole pages (a multiple of lcm(P, 32) keys), so no page's mass is
// carried across a run boundary; and each page's running (sum, max) is kept in
// global memory beside the mass output rather than in LDS, so the LDS a launch
// takes does not grow with the context.
//
// The hot decode path (one query, 32-token pages) has its own kernel in
// decode.hip; this one is the reference-exact general path and the fallback
// for every other shape.

#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <cmath>
#include <numeric>

namespace mi
{
  namespace
  {

    constexpr int kThreads = 256;
    constexpr int kTileK = 32;   // keys a tile
    constexpr int kTileQ = 16;   // queries a prefill tile
    constexpr int kSplitBlocksPerCU = 8;
    constexpr int kMinSplitKeys = 256;

    // What a device-side reader needs: the source, each quantised tier's layout.
    struct Reader
    {
      KVSource src;
      PageLayout lay[kTierCount];
      std::size_t row;          // kv_heads * head_dim
      int kv_heads;
      int head_dim;
      int own;                  // the query tile's own page (causal)

      __device__ static float h2f(std::uint16_t h) { return mi::h2f(h); }

      template <int Bits>
      __device__ static void dequant(const std::uint8_t *page, const PageLayout &L, int t,
                                     std::size_t at, std::size_t row, int kv_heads, int head_dim,
                                     float &k, float &v)
      {
        constexpr int kPerByte = 8 / Bits;
        constexpr unsigned kMask = (1u << Bits) - 1;
        const std::size_t e = static_cast<std::size_t>(t) * row + at;
        const unsigned kb = page[L.key_codes + e / kPerByte];
        const unsigned vb = page[L.value_codes + e / kPerByte];
        const int shift = static_cast<int>(e % kPerByte) * Bits;
        const auto *ks = reinterpret_cast<const std::uint16_t *>(page + L.key_scales);
        const auto *kz = reinterpret_cast<const std::uint16_t *>(page + L.key_zeros);
        const auto *vs = reinterpret_cast<const std::uint16_t *>(page + L.value_scales);
        const auto *vz = reinterpret_cast<const std::uint16_t *>(page + L.value_zeros);
        const std::size_t group = static_cast<std::size_t>(t) * kv_heads + at / head_dim;
        k = h2f(__half_as_ushort(__float2half_rn(
            fmaf(static_cast<float>((kb >> shift) & kMask), h2f(ks[at]), h2f(kz[at])))));
        v = h2f(__half_as_ushort(__float2half_rn(
            fmaf(static_cast<float>((vb >> shift) & kMask), h2f(vs[group]), h2f(vz[group])))));
      }

      // Whether key j is read at all: only a sealed page before the own page
      // can be unread.
      __device__ bool reads(int j) const
      {
        if (src.layout != Layout::kCausal)
        {
          return true;
        }
        const int p = j / src.page_tokens;
        return p >= own || src.tiers[p] != kUnreadPage;
      }

      // Element `at` of key j's row and of its value's row, widened to fp32.
      __device__ void read(int j, std::size_t at, float &k, float &v) const
      {
        switch (src.layout)
        {
        case Layout::kContiguous:
          k = h2f(src.k[static_cast<std::size_t>(j) * row + at]);
          v = h2f(src.v[static_cast<std::size_t>(j) * row + at]);
          return;
        case Layout::kPaged:
        {
          const int P = src.page_tokens;
          const auto *page = reinterpret_cast<const std::uint16_t *>(src.pages[j / P]);
          const std::size_t t = static_cast<std::size_t>(j % P);
          k = h2f(page[t * row + at]);
          v = h2f(page[(P + t) * row + at]);
          return;
        }
        case Layout::kCausal:
        {
          const int P = src.page_tokens;
          const int p = j / P;
          const int t = j % P;
          if (p < own)
          {
            const std::uint8_t tier = src.tiers[p];
            const auto *page = reinterpret_cast<const std::uint8_t *>(src.pages[p]);
            switch (tier)
            {
            case kINT8: dequant<8>(page, lay[kINT8], t, at, row, kv_heads, head_dim, k, v); return;
            case kINT4: dequant<4>(page, lay[kINT4], t, at, row, kv_heads, head_dim, k, v); return;
            case kINT2: dequant<2>(page, lay[kINT2], t, at, row, kv_heads, head_dim, k, v); return;
            case kFP16:
            {
              const auto *h = reinterpret_cast<const std::uint16_t *>(page);
              k = h2f(h[static_cast<std::size_t>(t) * row + at]);
              v = h2f(h[static_cast<std::size_t>(P + t) * row + at]);
              return;
            }
            default: // unread: its address is never touched
              k = 0.0f;
              v = 0.0f;
              return;
            }
          }
          if (j >= src.start)
          {
            k = h2f(src.chunk_k[static_cast<std::size_t>(j - src.start) * row + at]);
            v = h2f(src.chunk_v[static_cast<std::size_t>(j - src.start) * row + at]);
            return;
          }
          k = h2f(src.open[static_cast<std::size_t>(t) * row + at]);
          v = h2f(src.open[static_cast<std::size_t>(P + t) * row + at]);
          return;
        }
        }
      }
    };

    __device__ inline float rotated_bias(const std::uint16_t *bias, int position, int d,
                                         int head_dim, const float *rope)
    {
      const int half = head_dim / 2;
      const int j = d < half ? d : d - half;
      const float *cs = rope + 2 * (static_cast<std::size_t>(position) * half + j);
      const float b1 = h2f(bias[j]);
      const float b2 = h2f(bias[j + half]);
      return d < half ? b1 * cs[0] - b2 * cs[1] : b2 * cs[0] + b1 * cs[1];
    }

    struct Shape
    {
      int hpb;          // query heads a block (of one KV head)
      int qpb;          // queries a block
      int lead;         // rows before the first query, aligning tiles to pages
      int splits;
      int split_keys;
    };

    __host__ __device__ inline std::size_t slot_floats(int head_dim)
    {
      return static_cast<std::size_t>(head_dim) + 2; // m, l, then the output
    }

    // The kernel. Rows of a block: qpb queries x hpb consecutive heads, row r
    // being query r / hpb and head r % hpb. A block walks its split's keys in
    // tiles; in LDS: the rows' scaled q, output accumulators, the tile's scores,
    // keys (fp32, padded a column against bank conflicts) and values.
    template <bool kMass>
    __global__ void __launch_bounds__(kThreads)
        attention_kernel(Reader rd, AttentionArgs a, Shape s, float *page_max)
    {
      extern __shared__ float smem[];
      const int hd = a.head_dim;
      const int rows = s.hpb * s.qpb;
      const int ks = hd + 1;
      const int ss = kTileK + 1;
      float *q_s = smem;
      float *o_s = q_s + rows * hd;
      float *s_s = o_s + rows * hd;
      float *m_s = s_s + rows * ss;
      float *l_s = m_s + rows;
      float *rescale_s = l_s + rows;
      float *reads_s = rescale_s + rows;
      float *k_s = reads_s + kTileK;
      float *v_s = k_s + kTileK * ks;

      const int head_first = blockIdx.y * s.hpb;
      const int split = blockIdx.z;
      const int q_first = blockIdx.x * s.qpb - s.lead;
      const int q_last = min(q_first + s.qpb, a.seq_q) - 1;
      const int shift = a.seq_k - a.seq_q;
      const int group = a.heads / a.kv_heads;
      const std::size_t kv_off = static_cast<std::size_t>(head_first / group) * hd;
      const std::size_t token_stride = static_cast<std::size_t>(a.heads) * hd;
      if (rd.src.layout == Layout::kCausal)
      {
        rd.own = (q_first + shift) / rd.src.page_tokens;
      }
      const auto query_of = [&](int r) { return q_first + r / s.hpb; };
      const auto head_of = [&](int r) { return head_first + r % s.hpb; };
      const auto stored = [&](int r) { return query_of(r) >= 0 && query_of(r) <= q_last; };
      const float scale = 1.0f / sqrtf(static_cast<float>(hd));

      for (int i = threadIdx.x; i < rows * hd; i += blockDim.x)
      {
        const int r = i / hd;
        const int d = i % hd;
        q_s[i] = stored(r) ? h2f(a.q[query_of(r) * token_stride +
                                                    static_cast<std::size_t>(head_of(r)) * hd + d]) *
                                 scale
                           : 0.0f;
        o_s[i] = 0.0f;
      }
      for (int r = threadIdx.x; r < rows; r += blockDim.x)
      {
        m_s[r] = -INFINITY;
        l_s[r] = 0.0f;
      }

      const int key_first = split * s.split_keys;
      const int key_end = min(key_first + s.split_keys, q_last + shift + 1);
      const int P = rd.src.page_tokens;
      const int pages = kMass ? (a.seq_k + P - 1) / P : 0;
      // The page a row's thread is summing, its sum of exp(s - max), and max.
      int open = -1;
      float page_sum = 0.0f, page_top = -INFINITY;
      __syncthreads();

      for (int k_first = key_first; k_first < key_end; k_first += kTileK)
      {
        for (int i = threadIdx.x; i < kTileK * hd; i += blockDim.x)
        {
          const int c = i / hd;
          const int d = i % hd;
          const int j = k_first + c;
          const bool in_range = j < a.seq_k;
          float key = 0.0f, value = 0.0f;
          if (in_range && rd.reads(j))
          {
            rd.read(j, kv_off + d, key, value);
            if (a.k_bias != nullptr)
            {
              key += rotated_bias(a.k_bias + kv_off, j, d, hd, a.rope);
            }
          }
          k_s[c * ks + d] = key;
          v_s[c * hd + d] = value;
          if (d == 0)
          {
            reads_s[c] = !in_range || rd.reads(j) ? 1.0f : 0.0f;
          }
        }
        __syncthreads();

        for (int i = threadIdx.x; i < rows * kTileK; i += blockDim.x)
        {
          const int r = i / kTileK;
          const int c = i % kTileK;
          float dot = 0.0f;
          for (int d = 0; d < hd; ++d)
          {
            dot += q_s[r * hd + d] * k_s[c * ks + d];
          }
          const bool visible = k_first + c <= query_of(r) + shift && reads_s[c] != 0.0f;
          s_s[r * ss + c] = visible ? dot : -INFINITY;
        }
        __syncthreads();

        for (int r = threadIdx.x; r < rows; r += blockDim.x)
        {
          float *row = s_s + r * ss;
          const float m_old = m_s[r];
          float m_new = m_old;
          for (int c = 0; c < kTileK; ++c)
          {
            m_new = fmaxf(m_new, row[c]);
          }
          const float m_from = m_new == -INFINITY ? 0.0f : m_new;
          float sum = 0.0f;
          for (int c = 0; c < kTileK; ++c)
          {
            const float p = expf(row[c] - m_from);
            row[c] = p;
            sum += p;
          }
          const float rescale = expf(m_old - m_from);
          l_s[r] = l_s[r] * rescale + sum;
          m_s[r] = m_new;
          rescale_s[r] = rescale;
          if constexpr (kMass)
          {
            // One query: row r is head head_of(r). Keys past seq_k add 0.
            const std::size_t at = static_cast<std::size_t>(head_of(r)) * pages;
            for (int c = 0; c < kTileK && k_first + c < a.seq_k; ++c)
            {
              const int page = (k_first + c) / P;
              if (page != open)
              {
                if (open >= 0)
                {
                  a.mass[at + open] = page_sum;
                  page_max[at + open] = page_top;
                }
                open = page;
                page_sum = 0.0f;
                page_top = m_new;
              }
              else if (page_top < m_new)
              {
                page_sum *= expf(page_top - m_new);
                page_top = m_new;
              }
              page_sum += row[c];
            }
          }
        }
        __syncthreads();

        for (int i = threadIdx.x; i < rows * hd; i += blockDim.x)
        {
          const int r = i / hd;
          const int d = i % hd;
          const float *p = s_s + r * ss;
          float acc = o_s[i] * rescale_s[r];
          for (int c = 0; c < kTileK; ++c)
          {
            acc += p[c] * v_s[c * hd + d];
          }
          o_s[i] = acc;
        }
        __syncthreads();
      }

      const auto slot = [&](int r) {
        return a.partials + ((static_cast<std::size_t>(split) * a.seq_q + query_of(r)) * a.heads +
                             head_of(r)) * slot_floats(hd);
      };
      for (int i = threadIdx.x; i < rows * hd; i += blockDim.x)
      {
        const int r = i / hd;
        const int d = i % hd;
        if (!stored(r))
        {
          continue;
        }
        if (s.splits == 1)
        {
          a.out[query_of(r) * token_stride + static_cast<std::size_t>(head_of(r)) * hd + d] =
              __half_as_ushort(__float2half(o_s[i] / l_s[r]));
        }
        else
        {
          slot(r)[2 + d] = o_s[i];
        }
      }
      if (s.splits > 1)
      {
        for (int r = threadIdx.x; r < rows; r += blockDim.x)
        {
          if (stored(r))
          {
            slot(r)[0] = m_s[r];
            slot(r)[1] = l_s[r];
          }
        }
      }
      if constexpr (kMass)
      {
        for (int r = threadIdx.x; r < rows; r += blockDim.x)
        {
          if (open >= 0)
          {
            const std::size_t at = static_cast<std::size_t>(head_of(r)) * pages;
            a.mass[at + open] = page_sum;
            page_max[at + open] = page_top;
          }
        }
        __syncthreads();
        // This run's pages: whole pages, since runs are.
        const int first = key_first / P;
        const int last = (min(key_first + s.split_keys, a.seq_k) - 1) / P;
        const int local = last - first + 1;
        for (int i = threadIdx.x; i < rows * local; i += blockDim.x)
        {
          const int r = i / local;
          const int page = first + i % local;
          const std::size_t at = static_cast<std::size_t>(head_of(r)) * pages + page;
          const float m = m_s[r];
          const float sum = a.mass[at];
          const float top = page_max[at];
          if (s.splits == 1)
          {
            a.mass[at] = sum * expf(top - m) / l_s[r];
          }
          else
          {
            // Relative to this run's m; the combine brings it to the whole's.
            a.mass[at] = m == -INFINITY ? 0.0f : sum * expf(top - m);
          }
        }
      }
    }

    // Folds the runs: M = max m_s, w_s = exp(m_s - M), out = sum(w o) / sum(w l);
    // a page's mass, relative to its run's m, is weighed by its run's w and
    // divided by the same sum (reference: attention.cu:754-815; no carry, as
    // runs are whole pages here). One block a (query, head); a thread a run,
    // the sums over runs taken through LDS, never by one thread alone.
    constexpr int kCombineThreads = 256;
    constexpr int kCombineDims = 32;

    __global__ void __launch_bounds__(kCombineThreads)
        combine_kernel(const float *__restrict__ partials, std::uint16_t *__restrict__ out,
                       int seq_q, int heads, int head_dim, int splits, int split_keys,
                       float *__restrict__ mass, int page_tokens, int seq_k)
    {
      extern __shared__ float s_w[]; // a weight per run
      __shared__ float s_red[kCombineThreads / 64];
      __shared__ float s_acc[kCombineThreads][kCombineDims + 1];
      const int query = blockIdx.x / heads;
      const int head = blockIdx.x % heads;
      const int t = threadIdx.x;
      const std::size_t sf = slot_floats(head_dim);
      const auto slot = [&](int s) {
        return partials + ((static_cast<std::size_t>(s) * seq_q + query) * heads + head) * sf;
      };
      float top = -INFINITY;
      for (int s = t; s < splits; s += kCombineThreads)
      {
        top = fmaxf(top, slot(s)[0]);
      }
      top = block_reduce<true>(top, s_red);
      float l = 0.0f;
      for (int s = t; s < splits; s += kCombineThreads)
      {
        // A run none of whose keys this row reads weighs exactly 0.
        const float w = expf(slot(s)[0] - top);
        s_w[s] = w;
        l += slot(s)[1] * w;
      }
      l = block_reduce<false>(l, s_red);
      for (int d0 = 0; d0 < head_dim; d0 += kCombineDims)
      {
        const int n = min(kCombineDims, head_dim - d0);
        float acc[kCombineDims];
        for (int d = 0; d < kCombineDims; ++d)
        {
          acc[d] = 0.0f;
        }
        for (int s = t; s < splits; s += kCombineThreads)
        {
          const float *p = slot(s) + 2 + d0;
          for (int d = 0; d < n; ++d)
          {
            acc[d] += p[d] * s_w[s];
          }
        }
        __syncthreads();
        for (int d = 0; d < kCombineDims; ++d)
        {
          s_acc[t][d] = acc[d];
        }
        __syncthreads();
        if (t < n)
        {
          float sum = 0.0f;
          for (int u = 0; u < kCombineThreads; ++u)
          {
            sum += s_acc[u][t];
          }
          out[(static_cast<std::size_t>(query) * heads + head) * head_dim + d0 + t] =
              __half_as_ushort(__float2half(sum / l));
        }
      }
      if (mass == nullptr)
      {
        return;
      }
      __syncthreads();
      const int pages = (seq_k + page_tokens - 1) / page_tokens;
      float *head_mass = mass + static_cast<std::size_t>(head) * pages;
      for (int page = t; page < pages; page += kCombineThreads)
      {
        const int s = page * page_tokens / split_keys;
        head_mass[page] = head_mass[page] * s_w[s] / l;
      }
    }

    std::size_t shared_floats(int head_dim, int rows)
    {
      return 2 * static_cast<std::size_t>(rows) * head_dim + rows * (kTileK + 1) + 3 * rows +
             kTileK + static_cast<std::size_t>(kTileK) * (head_dim + 1) +
             static_cast<std::size_t>(kTileK) * head_dim;
    }

    int ceil_div(int a, int b) { return (a + b - 1) / b; }
    int round_up(int a, int b) { return ceil_div(a, b) * b; }

    Shape shape_for(int seq_q, int seq_k, int heads, int kv_heads, bool aligned, int page_tokens,
                    bool may_split)
    {
      Shape p{1, kTileQ, 0, 1, round_up(std::max(seq_k, 1), kTileK)};
      if (seq_q == 1)
      {
        const int group = heads / kv_heads;
        p.qpb = 1;
        for (int h = std::min(group, kTileQ); h >= 1; --h)
        {
          if (group % h == 0)
          {
            p.hpb = h;
            break;
          }
        }
      }
      p.lead = aligned ? (seq_k - seq_q) % p.qpb : 0;
      if (!may_split)
      {
        return p;
      }
      const long blocks = static_cast<long>(ceil_div(p.lead + seq_q, p.qpb)) * (heads / p.hpb);
      const long target = static_cast<long>(kSplitBlocksPerCU) * device_multiprocessors();
      const int splits = static_cast<int>(std::min<long>(target / blocks, seq_k / kMinSplitKeys));
      if (splits <= 1)
      {
        return p;
      }
      // Runs are whole tiles and whole pages.
      const int unit = page_tokens > 0 ? std::lcm(page_tokens, kTileK) : kTileK;
      p.split_keys = round_up(ceil_div(seq_k, splits), unit);
      p.splits = ceil_div(seq_k, p.split_keys);
      if (p.splits == 1)
      {
        p.split_keys = round_up(seq_k, kTileK);
      }
      return p;
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

    // The per-page running maxima a mass launch keeps beside its output: a
    // library-owned device buffer, grown on demand and kept.
    float *page_max_buffer(std::size_t floats)
    {
      static float *buffer = nullptr;
      static std::size_t held = 0;
      if (floats > held)
      {
        if (buffer != nullptr)
        {
          hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before growing scratch");
          hip_check(hipFree(buffer), "hipFree attention scratch");
          buffer = nullptr;
          held = 0;
        }
        const std::size_t grown = std::max<std::size_t>(floats, 1 << 16);
        hip_check(hipMalloc(reinterpret_cast<void **>(&buffer), grown * sizeof(float)),
                  "hipMalloc attention scratch");
        held = grown;
      }
      return buffer;
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
    return static_cast<std::size_t>(kSplitBlocksPerCU) * device_multiprocessors() * kTileQ *
           slot_floats(head_dim);
  }

  Split attention_split(int seq_q, int seq_k, int heads, int kv_heads, int page_tokens)
  {
    check_grouping(heads, kv_heads);
    const Shape p = shape_for(seq_q, seq_k, heads, kv_heads, page_tokens > 0, page_tokens, true);
    return {p.splits, p.split_keys};
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
    const bool aligned = kv.layout == Layout::kCausal;
    const int P = kv.layout == Layout::kContiguous ? 0 : kv.page_tokens;
    Shape s = shape_for(a.seq_q, a.seq_k, a.heads, a.kv_heads, aligned, P, a.partials != nullptr);

    Reader rd{};
    rd.src = kv;
    rd.row = static_cast<std::size_t>(a.kv_heads) * a.head_dim;
    rd.kv_heads = a.kv_heads;
    rd.head_dim = a.head_dim;
    rd.own = 0;
    for (int t = kINT8; t <= kINT2; ++t)
    {
      if (kv.layout == Layout::kCausal && kv.may_be_at[t])
      {
        rd.lay[t] = page_layout(t, kv.page_tokens, a.kv_heads, a.head_dim);
      }
    }
    // A mass over a contiguous layout has no pages: it is over pages of the
    // kernel's tile size.
    if (kv.layout == Layout::kContiguous)
    {
      rd.src.page_tokens = kTileK;
    }

    float *mass = a.mass;
    AttentionArgs args = a;
    float *page_max = nullptr;
    const int mass_pages = (a.seq_k + rd.src.page_tokens - 1) / rd.src.page_tokens;
    const std::size_t mass_floats = static_cast<std::size_t>(a.heads) * mass_pages;
    float *own_mass = nullptr;
    if (a.scores != nullptr && mass == nullptr)
    {
      // Scores need the mass: kept in scratch after the page maxima.
      float *scratch = page_max_buffer(2 * mass_floats);
      own_mass = scratch + mass_floats;
      mass = own_mass;
    }
    args.mass = mass;
    if (mass != nullptr)
    {
      page_max = page_max_buffer(own_mass ? 2 * mass_floats : mass_floats);
    }

    const int rows = s.hpb * s.qpb;
    const std::size_t lds = shared_floats(a.head_dim, rows) * sizeof(float);
    const dim3 grid(ceil_div(s.lead + a.seq_q, s.qpb), a.heads / s.hpb, s.splits);
    const auto run = [&](auto kernel) {
      if (lds > 64 * 1024)
      {
        hip_check(hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(lds)),
                  "hipFuncSetAttribute attention LDS");
      }
      hipLaunchKernelGGL(kernel, grid, dim3(kThreads), lds, stream, rd, args, s, page_max);
    };
    if (mass != nullptr)
    {
      run(attention_kernel<true>);
    }
    else
    {
      run(attention_kernel<false>);
    }
    hip_check(hipGetLastError(), "attention kernel launch");
    if (s.splits > 1)
    {
      hipLaunchKernelGGL(combine_kernel, dim3(a.seq_q * a.heads), dim3(kCombineThreads),
                         s.splits * sizeof(float), stream, a.partials, a.out, a.seq_q,
                         a.heads, a.head_dim, s.splits, s.split_keys, mass, rd.src.page_tokens,
                         a.seq_k);
      hip_check(hipGetLastError(), "attention combine kernel launch");
    }
    if (a.scores != nullptr)
    {
      launch_fold(a.scores, mass, a.heads, mass_pages, a.alpha, stream);
    }
  }

} // namespace mi
