// The C ABI (include/microinfer_hip.h): every entry point catches what the
// runtime throws and returns a status, with the message kept per thread.

#include "../../include/microinfer_hip.h"

#include "decode_step.hpp"
#include "kernels.hpp"
#include "runtime.hpp"

#include <algorithm>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>
#include <string>

// A KVPages keeps its allocator alive (the reference's binding does the
// same, bindings_device.cpp:701-718): the allocator goes when its own handle
// and every cache on it are gone, whatever order the caller drops them in
// (a garbage collector's order is arbitrary).
struct mi_cache
{
  std::shared_ptr<mi::PagedKVCache> owner;
  mi::PagedKVCache &impl;
  template <typename... A>
  explicit mi_cache(A &&...a)
      : owner(std::make_shared<mi::PagedKVCache>(std::forward<A>(a)...)), impl(*owner)
  {
  }
};
struct mi_kv_pages
{
  std::shared_ptr<mi::PagedKVCache> allocator; // declared first: destroyed last
  mi::KVPages impl;
  template <typename... A>
  mi_kv_pages(std::shared_ptr<mi::PagedKVCache> a, A &&...rest)
      : allocator(std::move(a)), impl(*allocator, std::forward<A>(rest)...)
  {
  }
};
struct mi_scores
{
  mi::ImportanceScores impl;
  template <typename... A> explicit mi_scores(A &&...a) : impl(std::forward<A>(a)...) {}
};
struct mi_shadows
{
  mi::ShadowStore impl;
  explicit mi_shadows(std::size_t b) : impl(b) {}
};
struct mi_decode_step
{
  mi::DecodeStep impl;
  template <typename... A> explicit mi_decode_step(A &&...a) : impl(std::forward<A>(a)...) {}
};
struct mi_rope_table
{
  mi::RopeTable impl;
  mi_rope_table(int hd, double theta) : impl(hd, theta) {}
};

namespace
{
  thread_local std::string g_error;

  int fail(int status, const char *what)
  {
    g_error = what;
    return status;
  }

  template <typename F> int guarded(F &&f)
  {
    try
    {
      g_error.clear();
      f();
      return MI_OK;
    }
    catch (const mi::InvalidArgument &e) { return fail(MI_ERR_INVALID, e.what()); }
    catch (const mi::OutOfRange &e) { return fail(MI_ERR_RANGE, e.what()); }
    catch (const mi::PageNotFound &e) { return fail(MI_ERR_NOT_FOUND, e.what()); }
    catch (const mi::OpenPageError &e) { return fail(MI_ERR_OPEN_PAGE, e.what()); }
    catch (const mi::OutOfMemory &e) { return fail(MI_ERR_OUT_OF_MEMORY, e.what()); }
    catch (const mi::LogicError &e) { return fail(MI_ERR_LOGIC, e.what()); }
    catch (const mi::Full &e) { return fail(MI_ERR_FULL, e.what()); }
    catch (const mi::DeviceError &e) { return fail(MI_ERR_DEVICE, e.what()); }
    catch (const std::bad_alloc &) { return fail(MI_ERR_OUT_OF_MEMORY, "host allocation failed"); }
    catch (const std::out_of_range &e) { return fail(MI_ERR_RANGE, e.what()); }
    catch (const std::exception &e) { return fail(MI_ERR_LOGIC, e.what()); }
    catch (...) { return fail(MI_ERR_LOGIC, "unknown error"); }
  }

  // A null stream argument is the runtime's current stream (the null stream
  // unless mi_set_stream named another), so every launch follows it.
  hipStream_t as_stream(void *s)
  {
    return s != nullptr ? static_cast<hipStream_t>(s) : mi::runtime_stream();
  }

  // ---- the allocation-free decode's scratch -------------------------------
  // A static device array: each GPU the library runs on holds its own copy,
  // at its own address, until the process ends. Host code never passes the
  // array's name to a kernel (on the host it is a stand-in, not a device
  // address): it looks up, once per device with that device current, the
  // address hipGetSymbolAddress gives, and passes that.
  constexpr std::size_t kNoAllocScratchBytes = std::size_t{8} << 20;
  constexpr std::size_t kNoAllocScratchFloats = kNoAllocScratchBytes / sizeof(float);
  constexpr int kMaxDevices = 64;
  static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

  float *scratch_on_current_device()
  {
    static std::once_flag once[kMaxDevices];
    static float *address[kMaxDevices] = {};
    int device = 0;
    mi::hip_check(hipGetDevice(&device), "hipGetDevice");
    if (device < 0 || device >= kMaxDevices)
    {
      throw mi::InvalidArgument("device " + std::to_string(device) + " is beyond the " +
                                std::to_string(kMaxDevices) + " the scratch table holds");
    }
    std::call_once(once[device], [device] {
      void *p = nullptr;
      mi::hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)),
                    "hipGetSymbolAddress of the decode scratch");
      address[device] = static_cast<float *>(p);
    });
    if (address[device] == nullptr)
    {
      throw mi::DeviceError("the decode scratch has no address on device " +
                            std::to_string(device));
    }
    return address[device];
  }

  // Hands the launch the static scratch, and refuses a need beyond it.
  struct StaticScratch final : mi::WorkspaceSource
  {
    float *base;
    float *floats(std::size_t count) override
    {
      if (count > kNoAllocScratchFloats)
      {
        throw mi::InvalidArgument(
            "this decode needs " + std::to_string(count * sizeof(float)) +
            " bytes of scratch; the allocation-free entry point holds " +
            std::to_string(kNoAllocScratchBytes) + " (fewer pages or heads fit)");
      }
      return base;
    }
  };

  void need(const void *p, const char *what)
  {
    if (p == nullptr)
    {
      throw mi::InvalidArgument(std::string(what) + " must not be null");
    }
  }

  mi::TierMap tier_map_of(const int *flat, const int *lengths, int rows)
  {
    mi::TierMap map;
    if (flat == nullptr || rows <= 0)
    {
      return map;
    }
    std::size_t at = 0;
    for (int r = 0; r < rows; ++r)
    {
      if (lengths[r] < 0)
      {
        throw mi::InvalidArgument("a tier map row has a negative length");
      }
      map.emplace_back(flat + at, flat + at + lengths[r]);
      at += static_cast<std::size_t>(lengths[r]);
    }
    return map;
  }

  void check_filled(int filled, int page_tokens)
  {
    if (filled < page_tokens)
    {
      throw mi::OpenPageError(
          "the page holds " + std::to_string(filled) + " of " + std::to_string(page_tokens) +
          " positions and is still being filled: a key channel's scale spans the whole page, so "
          "the open page stays at FP16");
    }
    if (filled > page_tokens)
    {
      throw mi::InvalidArgument(std::to_string(filled) + " positions do not fit a page of " +
                                std::to_string(page_tokens));
    }
  }

  void fill_args(mi::AttentionArgs &a, const void *q, const void *k_bias, const float *rope,
                 int rope_positions, void *out, int seq_q, int seq_k, int heads, int kv_heads,
                 int head_dim, float *mass, float *scores, float alpha, float *partials)
  {
    need(q, "q");
    need(out, "out");
    a.q = static_cast<const std::uint16_t *>(q);
    a.out = static_cast<std::uint16_t *>(out);
    a.k_bias = static_cast<const std::uint16_t *>(k_bias);
    a.rope = rope;
    a.rope_positions = rope_positions;
    a.seq_q = seq_q;
    a.seq_k = seq_k;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.mass = mass;
    a.scores = scores;
    a.alpha = alpha;
    a.partials = partials;
    // The header's contract: a partials buffer holds
    // mi_attention_partials_floats(head_dim) floats.
    a.partials_floats = partials != nullptr && head_dim > 0 ? mi::attention_partials_floats(head_dim)
                                                            : 0;
    if (seq_q < 0 || seq_k < 0 || seq_q > seq_k)
    {
      throw mi::InvalidArgument("seq_q " + std::to_string(seq_q) + " exceeds seq_k " +
                                std::to_string(seq_k));
    }
  }
} // namespace

extern "C" {

const char *mi_last_error(void) { return g_error.c_str(); }

const char *mi_build_info(void)
{
  static const std::string info = "microinfer_hip: gfx950, HIP " +
                                  std::to_string(HIP_VERSION_MAJOR) + "." +
                                  std::to_string(HIP_VERSION_MINOR) +
                                  ", -O3 -ffp-contract=off, no packed fp32";
  return info.c_str();
}

int mi_device_count(int *count)
{
  return guarded([&] { mi::hip_check(hipGetDeviceCount(count), "hipGetDeviceCount"); });
}

int mi_device_name(char *out, size_t capacity)
{
  return guarded([&] {
    int device = 0;
    mi::hip_check(hipGetDevice(&device), "hipGetDevice");
    hipDeviceProp_t prop{};
    mi::hip_check(hipGetDeviceProperties(&prop, device), "hipGetDeviceProperties");
    // Some runtimes leave the marketing name empty: the architecture then
    // names the device.
    const std::string arch = prop.gcnArchName;
    const std::string base = prop.name[0] != '\0' ? std::string(prop.name)
                                                  : "AMD GPU " + arch.substr(0, arch.find(':'));
    const std::string name = base + " (" + arch + ")";
    std::strncpy(out, name.c_str(), capacity);
    if (capacity > 0)
    {
      out[capacity - 1] = '\0';
    }
  });
}

int mi_host_alloc(void **host, void **device, size_t bytes)
{
  return guarded([&] {
    need(host, "host");
    need(device, "device");
    *host = nullptr;
    *device = nullptr;
    mi::hip_check(hipHostMalloc(host, bytes, hipHostMallocMapped), "hipHostMalloc");
    const hipError_t mapped = hipHostGetDevicePointer(device, *host, 0);
    if (mapped != hipSuccess)
    {
      (void)hipHostFree(*host);
      *host = nullptr;
      mi::hip_check(mapped, "hipHostGetDevicePointer");
    }
  });
}

int mi_host_free(void *host)
{
  return guarded([&] {
    if (host != nullptr)
    {
      mi::hip_check(hipHostFree(host), "hipHostFree");
    }
  });
}

int mi_device_pci_bus_id(char *out, size_t capacity)
{
  return guarded([&] {
    int device = 0;
    mi::hip_check(hipGetDevice(&device), "hipGetDevice");
    mi::hip_check(hipDeviceGetPCIBusId(out, static_cast<int>(capacity), device),
                  "hipDeviceGetPCIBusId");
  });
}

int mi_runtime_version(int *version)
{
  return guarded([&] { mi::hip_check(hipRuntimeGetVersion(version), "hipRuntimeGetVersion"); });
}

int mi_driver_version(int *version)
{
  return guarded([&] { mi::hip_check(hipDriverGetVersion(version), "hipDriverGetVersion"); });
}

int mi_memory_info(size_t *free_bytes, size_t *total_bytes)
{
  return guarded([&] { mi::hip_check(hipMemGetInfo(free_bytes, total_bytes), "hipMemGetInfo"); });
}

int mi_granule_bytes(size_t *out)
{
  return guarded([&] { *out = mi::granule_bytes(); });
}

int mi_malloc(void **out, size_t bytes)
{
  return guarded([&] {
    *out = nullptr;
    if (bytes > 0)
    {
      mi::hip_check(hipMalloc(out, bytes), "hipMalloc");
    }
  });
}

int mi_free(void *ptr)
{
  return guarded([&] {
    if (ptr != nullptr)
    {
      mi::hip_check(hipFree(ptr), "hipFree");
    }
  });
}

int mi_memcpy(void *dst, const void *src, size_t bytes, int kind)
{
  return guarded([&] {
    if (bytes == 0)
    {
      return;
    }
    const hipMemcpyKind k = kind == 0   ? hipMemcpyHostToDevice
                            : kind == 1 ? hipMemcpyDeviceToHost
                                        : hipMemcpyDeviceToDevice;
    mi::hip_check(hipMemcpy(dst, src, bytes, k), "hipMemcpy");
  });
}

int mi_memset(void *dst, int value, size_t bytes)
{
  return guarded([&] {
    if (bytes > 0)
    {
      mi::hip_check(hipMemset(dst, value, bytes), "hipMemset");
    }
  });
}

int mi_synchronize(void)
{
  return guarded([&] { mi::hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize"); });
}

int mi_event_create(void **event)
{
  return guarded([&] {
    hipEvent_t e;
    mi::hip_check(hipEventCreate(&e), "hipEventCreate");
    *event = e;
  });
}

int mi_event_destroy(void *event)
{
  return guarded([&] { mi::hip_check(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy"); });
}

int mi_event_record(void *event, void *stream)
{
  return guarded([&] {
    mi::hip_check(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)),
                  "hipEventRecord");
  });
}

int mi_event_elapsed_ms(void *start, void *end, float *ms)
{
  return guarded([&] {
    mi::hip_check(hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize");
    mi::hip_check(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start),
                                      static_cast<hipEvent_t>(end)),
                  "hipEventElapsedTime");
  });
}

int mi_stream_create(void **stream)
{
  return guarded([&] {
    hipStream_t s;
    mi::hip_check(hipStreamCreate(&s), "hipStreamCreate");
    *stream = s;
  });
}

int mi_stream_destroy(void *stream)
{
  return guarded([&] { mi::hip_check(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy"); });
}

int mi_stream_synchronize(void *stream)
{
  return guarded(
      [&] { mi::hip_check(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize"); });
}

int mi_set_stream(void *stream)
{
  // NULL names the null stream itself (not "the current one", as a null
  // stream argument of a launcher does).
  return guarded([&] { mi::set_runtime_stream(static_cast<hipStream_t>(stream)); });
}

int mi_graph_begin(void *stream)
{
  return guarded([&] {
    if (stream == nullptr)
    {
      throw mi::InvalidArgument("the null stream cannot be captured; create a stream");
    }
    mi::hip_check(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal),
                  "hipStreamBeginCapture");
  });
}

int mi_graph_end(void *stream, void **exec)
{
  return guarded([&] {
    hipGraph_t graph = nullptr;
    mi::hip_check(hipStreamEndCapture(as_stream(stream), &graph), "hipStreamEndCapture");
    hipGraphExec_t e = nullptr;
    const hipError_t made = hipGraphInstantiate(&e, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    mi::hip_check(made, "hipGraphInstantiate");
    *exec = e;
  });
}

int mi_graph_launch(void *exec, void *stream)
{
  return guarded([&] {
    mi::hip_check(hipGraphLaunch(static_cast<hipGraphExec_t>(exec), as_stream(stream)),
                  "hipGraphLaunch");
  });
}

int mi_graph_destroy(void *exec)
{
  return guarded([&] {
    mi::hip_check(hipGraphExecDestroy(static_cast<hipGraphExec_t>(exec)), "hipGraphExecDestroy");
  });
}

uint16_t mi_half_bits_from_double(double x) { return mi::half_bits_from_double(x); }

uint16_t mi_scale_bits_of(float lo, float hi, int bits) { return mi::scale_bits_of(lo, hi, bits); }

int mi_quantised_page_layout(int tier, int page_tokens, int kv_heads, int head_dim,
                             mi_page_layout *out)
{
  return guarded([&] {
    const mi::PageLayout l = mi::page_layout(tier, page_tokens, kv_heads, head_dim);
    out->bits = l.bits;
    out->key_codes = l.key_codes;
    out->value_codes = l.value_codes;
    out->key_scales = l.key_scales;
    out->key_zeros = l.key_zeros;
    out->value_scales = l.value_scales;
    out->value_zeros = l.value_zeros;
    out->metadata_bytes = l.metadata_bytes;
    out->page_bytes = l.page_bytes;
    out->effective_bits = l.effective_bits;
  });
}

size_t mi_fp16_page_bytes(int page_tokens, size_t kv_width)
{
  return mi::fp16_page_bytes(page_tokens, kv_width);
}

int mi_quantise_page(const void *keys, const void *values, void *page, int tier, int page_tokens,
                     int filled, int kv_heads, int head_dim, void *stream)
{
  return guarded([&] {
    mi::page_layout(tier, page_tokens, kv_heads, head_dim);
    check_filled(filled, page_tokens);
    need(keys, "keys");
    need(values, "values");
    need(page, "page");
    mi::launch_quantise_pages(nullptr, nullptr, keys, page,
                              static_cast<const char *>(values) - static_cast<const char *>(keys), 1,
                              tier, page_tokens, kv_heads, head_dim, as_stream(stream));
  });
}

int mi_quantise_pages(const void *const *rows, void *const *pages, int count, int tier,
                      int page_tokens, int kv_heads, int head_dim, void *stream)
{
  return guarded([&] {
    mi::page_layout(tier, page_tokens, kv_heads, head_dim);
    if (count <= 0)
    {
      return;
    }
    need(rows, "rows");
    need(pages, "pages");
    const std::ptrdiff_t half =
        static_cast<std::ptrdiff_t>(page_tokens) * kv_heads * head_dim * 2;
    mi::launch_quantise_pages(rows, pages, nullptr, nullptr, half, count, tier, page_tokens,
                              kv_heads, head_dim, as_stream(stream));
  });
}

int mi_dequantise_page(const void *page, void *keys, void *values, int tier, int page_tokens,
                       int kv_heads, int head_dim, void *stream)
{
  return guarded([&] {
    need(page, "page");
    need(keys, "keys");
    need(values, "values");
    mi::launch_dequantise_page(page, keys, values, tier, page_tokens, kv_heads, head_dim,
                               as_stream(stream));
  });
}

size_t mi_attention_partials_floats(int head_dim)
{
  try
  {
    return mi::attention_partials_floats(head_dim);
  }
  catch (...)
  {
    return 0;
  }
}

int mi_attention_split(int seq_q, int seq_k, int heads, int kv_heads, int page_tokens,
                       int *splits, int *split_keys)
{
  return guarded([&] {
    const mi::Split s = mi::attention_split(seq_q, seq_k, heads, kv_heads, page_tokens);
    *splits = s.splits;
    *split_keys = s.split_keys;
  });
}

int mi_attention(const void *q, const void *k, const void *v, const void *k_bias,
                 const float *rope, int rope_positions, void *out, int seq_q, int seq_k, int heads,
                 int kv_heads, int head_dim, float *partials, void *stream)
{
  return guarded([&] {
    mi::AttentionArgs a{};
    fill_args(a, q, k_bias, rope, rope_positions, out, seq_q, seq_k, heads, kv_heads, head_dim,
              nullptr, nullptr, 0.0f, partials);
    mi::KVSource kv{};
    kv.layout = mi::Layout::kContiguous;
    kv.k = static_cast<const std::uint16_t *>(k);
    kv.v = static_cast<const std::uint16_t *>(v);
    kv.may_be_at[mi::kFP16] = true;
    if (seq_k > 0)
    {
      need(k, "k");
      need(v, "v");
    }
    mi::launch_attention(kv, a, as_stream(stream));
  });
}

int mi_attention_paged(const void *q, const unsigned long long *pages, int page_tokens,
                       const void *k_bias, const float *rope, int rope_positions, void *out,
                       int seq_q, int seq_k, int heads, int kv_heads, int head_dim, float *mass,
                       float *partials, void *stream)
{
  return guarded([&] {
    if (page_tokens <= 0)
    {
      throw mi::InvalidArgument("page_tokens must be positive, got " + std::to_string(page_tokens));
    }
    mi::AttentionArgs a{};
    fill_args(a, q, k_bias, rope, rope_positions, out, seq_q, seq_k, heads, kv_heads, head_dim,
              mass, nullptr, 0.0f, partials);
    mi::KVSource kv{};
    kv.layout = mi::Layout::kPaged;
    kv.pages = pages;
    kv.page_tokens = page_tokens;
    kv.may_be_at[mi::kFP16] = true;
    mi::launch_attention(kv, a, as_stream(stream));
  });
}

int mi_attention_paged_causal(const void *q, const unsigned long long *sealed,
                              const uint8_t *tiers, int may_be_at_mask, const void *open,
                              const void *chunk_k, const void *chunk_v, int page_tokens,
                              const void *k_bias, const float *rope, int rope_positions, void *out,
                              int seq_q, int seq_k, int heads, int kv_heads, int head_dim,
                              float *mass, float *scores, float alpha, float *partials,
                              void *stream)
{
  return guarded([&] {
    if (page_tokens <= 0 || page_tokens % 16 != 0)
    {
      throw mi::InvalidArgument(
          "causal paged attention aligns query tiles of 16 to pages, so page_tokens must be a "
          "positive multiple of it; got " +
          std::to_string(page_tokens));
    }
    mi::AttentionArgs a{};
    fill_args(a, q, k_bias, rope, rope_positions, out, seq_q, seq_k, heads, kv_heads, head_dim,
              mass, scores, alpha, partials);
    mi::KVSource kv{};
    kv.layout = mi::Layout::kCausal;
    kv.pages = sealed;
    kv.tiers = tiers;
    kv.open = static_cast<const std::uint16_t *>(open);
    kv.chunk_k = static_cast<const std::uint16_t *>(chunk_k);
    kv.chunk_v = static_cast<const std::uint16_t *>(chunk_v);
    kv.page_tokens = page_tokens;
    kv.start = seq_k - seq_q;
    for (int t = 0; t < mi::kTierCount; ++t)
    {
      kv.may_be_at[t] = (may_be_at_mask >> t) & 1;
      if (kv.may_be_at[t] && t != mi::kFP16)
      {
        mi::page_layout(t, page_tokens, kv_heads, head_dim);
      }
    }
    mi::launch_attention(kv, a, as_stream(stream));
  });
}

int mi_attention_paged_causal_noalloc(const void *q, const unsigned long long *sealed,
                                      const uint8_t *tiers, int may_be_at_mask, const void *open,
                                      const void *chunk_k, const void *chunk_v, int page_tokens,
                                      void *out, int seq_k, int heads, int kv_heads, int head_dim,
                                      float *mass, float *scores, float alpha, void *stream)
{
  return guarded([&] {
    mi::AttentionArgs a{};
    fill_args(a, q, nullptr, nullptr, 0, out, 1, seq_k, heads, kv_heads, head_dim, mass, scores,
              alpha, nullptr);
    mi::KVSource kv{};
    kv.layout = mi::Layout::kCausal;
    kv.pages = sealed;
    kv.tiers = tiers;
    kv.open = static_cast<const std::uint16_t *>(open);
    kv.chunk_k = static_cast<const std::uint16_t *>(chunk_k);
    kv.chunk_v = static_cast<const std::uint16_t *>(chunk_v);
    kv.page_tokens = page_tokens;
    kv.start = seq_k - 1;
    for (int t = 0; t < mi::kTierCount; ++t)
    {
      kv.may_be_at[t] = (may_be_at_mask >> t) & 1;
    }
    if (!mi::decode_fast_applies(kv, a))
    {
      throw mi::InvalidArgument(
          "the allocation-free decode takes one query over 32-token pages at head_dim 64 or 128, "
          "at most 16 query heads a KV head, with 16-byte aligned q, open page and rows");
    }
    StaticScratch ws;
    ws.base = scratch_on_current_device();
    a.workspace = &ws;
    mi::DecodeLayers one{};
    one.split = true;
    one.layers = 1;
    mi::launch_decode_layers(kv, a, one, as_stream(stream));
  });
}

int mi_copy_pages(const void *const *from, void *const *to, size_t bytes, int count, void *stream)
{
  return guarded([&] { mi::launch_copy_pages(from, to, bytes, count, as_stream(stream)); });
}

int mi_store_pages(const void *keys, const void *values, const unsigned long long *pages,
                   int page_tokens, size_t row, int start, int n, void *stream)
{
  return guarded([&] {
    mi::launch_store_pages(keys, values, pages, page_tokens, row, start, n, as_stream(stream));
  });
}

int mi_fill_f32(float *out, size_t count, float value, void *stream)
{
  return guarded([&] { mi::launch_fill(out, count, value, as_stream(stream)); });
}

int mi_fold_scores(float *scores, const float *mass, int heads, int pages, float alpha,
                   void *stream)
{
  return guarded([&] { mi::launch_fold(scores, mass, heads, pages, alpha, as_stream(stream)); });
}

int mi_rope(const void *x, const int32_t *positions, void *out, int seq, int heads, int head_dim,
            double theta, void *stream)
{
  return guarded([&] {
    if (head_dim % 2 != 0)
    {
      throw mi::InvalidArgument("head_dim must be even for rotate-half RoPE, got " +
                                std::to_string(head_dim));
    }
    if (!(theta > 0.0))
    {
      throw mi::InvalidArgument("theta must be positive, got " + std::to_string(theta));
    }
    if (x == out && seq > 0)
    {
      throw mi::InvalidArgument("rope cannot write over its input");
    }
    mi::launch_rope(x, positions, out, seq, heads, head_dim, theta, as_stream(stream));
  });
}

int mi_rope_from_table(const void *x, const int32_t *positions, const float *table,
                       int table_positions, void *out, int seq, int heads, int head_dim,
                       void *stream)
{
  return guarded([&] {
    if (x == out && seq > 0)
    {
      throw mi::InvalidArgument("RoPE from a table writes a separate output; x == out");
    }
    mi::RopeRows r{};
    r.x[0] = x;
    r.out[0] = out;
    r.heads[0] = heads;
    r.positions = positions;
    r.table = table;
    r.table_positions = table_positions;
    r.seq = seq;
    r.head_dim = head_dim;
    mi::launch_rope_rows(r, as_stream(stream));
  });
}

int mi_rope_table_fill(float *table, int positions, int head_dim, double theta, void *stream)
{
  return guarded(
      [&] { mi::launch_rope_table(table, positions, head_dim, theta, as_stream(stream)); });
}

int mi_rmsnorm(const void *x, int x_is_f32, const void *weight, void *out, int rows, int hidden,
               float eps, void *stream)
{
  return guarded([&] {
    mi::launch_rmsnorm(x, x_is_f32 != 0, weight, out, rows, hidden, eps, as_stream(stream));
  });
}

int mi_swiglu(const void *gate, const void *up, void *out, size_t count, void *stream)
{
  return guarded([&] {
    if (count > 0 && (out == gate || out == up))
    {
      throw mi::InvalidArgument("swiglu cannot write over its input");
    }
    mi::launch_swiglu(gate, up, out, count, as_stream(stream));
  });
}

int mi_add(const void *a, const void *b, void *out, size_t count, void *stream)
{
  return guarded([&] { mi::launch_add(a, b, out, count, as_stream(stream)); });
}

// ---- dense projections, embedding, logits ----------------------------------------

namespace
{
  std::size_t scratch_elements_of(int rows, int vocab)
  {
    if (rows < 0 || vocab < 0)
    {
      throw mi::InvalidArgument("scratch is sized for rows >= 0 and vocab >= 0");
    }
    const std::size_t bytes = static_cast<std::size_t>(rows) * vocab * sizeof(float) +
                              static_cast<std::size_t>(rows) * sizeof(std::int32_t);
    return (bytes + 1) / 2;
  }

  // Rows [first_row, first_row + rows) of x through the (vocab, hidden) head,
  // fp32 logits into the scratch.
  float *logits_into(const void *x, const void *head, void *scratch, size_t scratch_elements,
                     int first_row, int rows, int hidden, int vocab, hipStream_t stream)
  {
    if (first_row < 0 || rows < 0)
    {
      throw mi::InvalidArgument("first_row and rows are >= 0; got " + std::to_string(first_row) +
                                " and " + std::to_string(rows));
    }
    if (scratch_elements < scratch_elements_of(rows, vocab))
    {
      throw mi::InvalidArgument("scratch holds " + std::to_string(scratch_elements) +
                                ", and the logits of " + std::to_string(rows) + " rows need " +
                                std::to_string(scratch_elements_of(rows, vocab)));
    }
    need(x, "x");
    need(head, "head");
    need(scratch, "scratch");
    auto *out = static_cast<float *>(scratch);
    const auto *rows_x =
        static_cast<const std::uint16_t *>(x) + static_cast<std::size_t>(first_row) * hidden;
    mi::linear_float(rows_x, head, out, false, rows, hidden, vocab, stream);
    return out;
  }
}

int mi_linear(const void *x, const void *weight, const void *bias, void *out, int rows,
              int in_features, int out_features, void *stream)
{
  return guarded([&] {
    mi::linear_half(x, weight, bias, out, rows, in_features, out_features, as_stream(stream));
  });
}

int mi_linear_f32(const void *x, const void *weight, float *out, int accumulate, int rows,
                  int in_features, int out_features, void *stream)
{
  return guarded([&] {
    mi::linear_float(x, weight, out, accumulate != 0, rows, in_features, out_features,
                     as_stream(stream));
  });
}

int mi_embed(const int32_t *ids, int count, const void *table, void *out, int out_is_f32,
             int hidden, int vocab, void *stream)
{
  return guarded([&] {
    mi::launch_embed(ids, count, table, out, out_is_f32 != 0, hidden, vocab, as_stream(stream));
  });
}

int mi_argmax_rows(const float *x, int rows, int cols, int32_t *out, void *stream)
{
  return guarded([&] { mi::launch_argmax_rows(x, rows, cols, out, as_stream(stream)); });
}

int mi_scratch_elements(int rows, int vocab, size_t *out)
{
  return guarded([&] { *out = scratch_elements_of(rows, vocab); });
}

int mi_logits(const void *x, const void *head, void *scratch, size_t scratch_elements,
              int first_row, int rows, int hidden, int vocab, float *host_out)
{
  return guarded([&] {
    const hipStream_t stream = mi::runtime_stream();
    const float *dev = logits_into(x, head, scratch, scratch_elements, first_row, rows, hidden,
                                   vocab, stream);
    const std::size_t bytes = static_cast<std::size_t>(rows) * vocab * sizeof(float);
    if (bytes > 0)
    {
      mi::hip_check(hipMemcpyAsync(host_out, dev, bytes, hipMemcpyDeviceToHost, stream),
                    "hipMemcpyAsync logits device-to-host");
      mi::hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize logits");
    }
  });
}

int mi_greedy(const void *x, const void *head, void *scratch, size_t scratch_elements,
              int first_row, int rows, int hidden, int vocab, int32_t *host_ids)
{
  return guarded([&] {
    const hipStream_t stream = mi::runtime_stream();
    const float *dev = logits_into(x, head, scratch, scratch_elements, first_row, rows, hidden,
                                   vocab, stream);
    if (rows == 0)
    {
      return;
    }
    auto *ids = reinterpret_cast<std::int32_t *>(static_cast<char *>(scratch) +
                                                 static_cast<std::size_t>(rows) * vocab *
                                                     sizeof(float));
    mi::launch_argmax_rows(dev, rows, vocab, ids, stream);
    mi::hip_check(hipMemcpyAsync(host_ids, ids, static_cast<std::size_t>(rows) * sizeof(int32_t),
                                 hipMemcpyDeviceToHost, stream),
                  "hipMemcpyAsync ids device-to-host");
    mi::hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize greedy");
    for (int r = 0; r < rows; ++r)
    {
      if (host_ids[r] >= vocab)
      {
        throw mi::LogicError("row " + std::to_string(first_row + r) +
                             " has no finite logit, so there is no greedy choice; the forward "
                             "pass produced NaN or -inf throughout");
      }
    }
  });
}

// ---- PagedKVCache ------------------------------------------------------------

int mi_cache_create(const size_t page_bytes[4], const size_t capacity_pages[4], mi_cache **out)
{
  return guarded([&] {
    std::array<std::size_t, 4> pb{}, cp{};
    for (int t = 0; t < 4; ++t)
    {
      pb[t] = page_bytes[t];
      cp[t] = capacity_pages[t];
    }
    *out = new mi_cache(pb, cp);
  });
}

void mi_cache_destroy(mi_cache *cache) { delete cache; }

int mi_cache_allocate(mi_cache *c, int layer, int page, int tier)
{
  return guarded([&] { c->impl.allocate({layer, page}, tier); });
}

int mi_cache_free(mi_cache *c, int layer, int page)
{
  return guarded([&] { c->impl.free({layer, page}); });
}

int mi_cache_free_pages(mi_cache *c, const int *keys, size_t n)
{
  return guarded([&] {
    std::vector<mi::PageKey> v;
    for (size_t i = 0; i < n; ++i)
    {
      v.push_back({keys[2 * i], keys[2 * i + 1]});
    }
    c->impl.free_pages(v);
  });
}

int mi_cache_replace(mi_cache *c, int layer, int page, int staged_layer, int staged_page)
{
  return guarded([&] { c->impl.replace({layer, page}, {staged_layer, staged_page}); });
}

int mi_cache_replace_pages(mi_cache *c, const int *quads, size_t n)
{
  return guarded([&] {
    std::vector<std::pair<mi::PageKey, mi::PageKey>> v;
    for (size_t i = 0; i < n; ++i)
    {
      v.push_back({{quads[4 * i], quads[4 * i + 1]}, {quads[4 * i + 2], quads[4 * i + 3]}});
    }
    c->impl.replace_pages(v);
  });
}

int mi_cache_write(mi_cache *c, int layer, int page, const void *host, size_t bytes)
{
  return guarded([&] { c->impl.write({layer, page}, host, bytes); });
}

int mi_cache_read(mi_cache *c, int layer, int page, void *host, size_t bytes)
{
  return guarded([&] { c->impl.read({layer, page}, host, bytes); });
}

int mi_cache_locate(mi_cache *c, int layer, int page, int *tier, size_t *slot)
{
  return guarded([&] {
    const mi::PageLocation l = c->impl.locate({layer, page});
    *tier = l.tier;
    *slot = l.slot;
  });
}

int mi_cache_contains(mi_cache *c, int layer, int page, int *out)
{
  return guarded([&] { *out = c->impl.contains({layer, page}) ? 1 : 0; });
}

int mi_cache_pages(mi_cache *c, int tier, int *keys, size_t capacity, size_t *count)
{
  return guarded([&] {
    if (tier < 0 || tier >= mi::kTierCount)
    {
      throw mi::InvalidArgument("tier " + std::to_string(tier) + " is not one of the four");
    }
    const auto &slots = c->impl.pages(tier);
    *count = slots.size();
    for (size_t i = 0; i < slots.size() && i < capacity; ++i)
    {
      keys[2 * i] = slots[i].layer;
      keys[2 * i + 1] = slots[i].page;
    }
  });
}

#define MI_TIER_GETTER(name, expr)                                                            \
  int name(mi_cache *c, int tier, size_t *out)                                                \
  {                                                                                           \
    return guarded([&] {                                                                      \
      if (tier < 0 || tier >= mi::kTierCount)                                                 \
      {                                                                                       \
        throw mi::InvalidArgument("tier " + std::to_string(tier) + " is not one of the four"); \
      }                                                                                       \
      *out = c->impl.expr(tier);                                                              \
    });                                                                                       \
  }
MI_TIER_GETTER(mi_cache_page_bytes, page_bytes)
MI_TIER_GETTER(mi_cache_reserved_bytes, reserved_bytes)
MI_TIER_GETTER(mi_cache_mapped_bytes, mapped_bytes)
MI_TIER_GETTER(mi_cache_spare_granules, spare_granules)
#undef MI_TIER_GETTER

int mi_cache_keep_spare_granules(mi_cache *c, int tier, size_t granules)
{
  return guarded([&] { c->impl.keep_spare_granules(tier, granules); });
}

int mi_cache_granule_bytes(mi_cache *c, size_t *out)
{
  return guarded([&] { *out = c->impl.granule(); });
}

int mi_cache_drain_releases(mi_cache *c)
{
  return guarded([&] { c->impl.drain_releases(); });
}

int mi_debug_fail_next_granules(int n)
{
  return guarded([&] { mi::fail_next_granules(n); });
}

// ---- ShadowStore ----------------------------------------------------------------

int mi_shadows_create(size_t page_bytes, mi_shadows **out)
{
  return guarded([&] { *out = new mi_shadows(page_bytes); });
}

void mi_shadows_destroy(mi_shadows *s) { delete s; }

int mi_shadows_take(mi_shadows *s, int layer, int page, const void *device_page)
{
  return guarded([&] { s->impl.take({layer, page}, device_page, mi::runtime_stream()); });
}

int mi_shadows_contains(mi_shadows *s, int layer, int page, int *out)
{
  return guarded([&] { *out = s->impl.contains({layer, page}) ? 1 : 0; });
}

int mi_shadows_read(mi_shadows *s, int layer, int page, void *host, size_t bytes)
{
  return guarded([&] {
    if (bytes != s->impl.page_bytes())
    {
      throw mi::InvalidArgument("a shadow holds " + std::to_string(s->impl.page_bytes()) +
                                " bytes, not " + std::to_string(bytes));
    }
    std::memcpy(host, s->impl.shadow({layer, page}), bytes);
  });
}

int mi_shadows_count(mi_shadows *s, size_t *out)
{
  return guarded([&] { *out = s->impl.count(); });
}

int mi_shadows_bytes(mi_shadows *s, size_t *out)
{
  return guarded([&] { *out = s->impl.bytes(); });
}

// ---- ImportanceScores ---------------------------------------------------------------

int mi_scores_create(int layers, int max_pages, float alpha, mi_scores **out)
{
  return guarded([&] { *out = new mi_scores(layers, max_pages, alpha); });
}

void mi_scores_destroy(mi_scores *s) { delete s; }

int mi_scores_fold(mi_scores *s, int layer, const float *mass, int heads, int pages)
{
  return guarded([&] { s->impl.fold(layer, mass, heads, pages, mi::runtime_stream()); });
}

int mi_scores_download(mi_scores *s, float *host, size_t count)
{
  return guarded([&] {
    const std::vector<float> v = s->impl.download();
    if (count < v.size())
    {
      throw mi::InvalidArgument("the scores need " + std::to_string(v.size()) + " floats");
    }
    std::memcpy(host, v.data(), v.size() * sizeof(float));
  });
}

int mi_scores_upload(mi_scores *s, const float *host, int layers, int max_pages)
{
  return guarded([&] { s->impl.upload(host, layers, max_pages); });
}

int mi_scores_layer_row(mi_scores *s, int layer, float **row)
{
  return guarded([&] { *row = s->impl.layer_scores(layer); });
}

int mi_scores_info(mi_scores *s, int *layers, int *max_pages, float *alpha, size_t *downloads)
{
  return guarded([&] {
    *layers = s->impl.layers();
    *max_pages = s->impl.max_pages();
    *alpha = s->impl.alpha();
    *downloads = s->impl.downloads();
  });
}

// ---- RopeTable ------------------------------------------------------------------------

int mi_rope_table_create(int head_dim, double theta, mi_rope_table **out)
{
  return guarded([&] { *out = new mi_rope_table(head_dim, theta); });
}

void mi_rope_table_destroy(mi_rope_table *t) { delete t; }

int mi_rope_table_cover(mi_rope_table *t, int positions)
{
  return guarded([&] { t->impl.cover(positions); });
}

int mi_rope_table_info(mi_rope_table *t, int *positions, const float **data)
{
  return guarded([&] {
    *positions = t->impl.positions();
    *data = t->impl.data();
  });
}

// ---- KVPages ----------------------------------------------------------------------------

int mi_kv_create(mi_cache *allocator, int layers, int page_tokens, int kv_heads, int head_dim,
                 int tier, int halves, const int *tier_map, const int *row_lengths, int map_rows,
                 int always_seal, mi_kv_pages **out)
{
  return guarded([&] {
    need(allocator, "allocator");
    if (halves < 0 || halves > 2)
    {
      throw mi::InvalidArgument("halves is 0 (Both), 1 (Keys) or 2 (Values)");
    }
    *out = new mi_kv_pages(allocator->owner, layers, page_tokens, kv_heads, head_dim, tier,
                           static_cast<mi::Halves>(halves),
                           tier_map_of(tier_map, row_lengths, map_rows), always_seal != 0);
  });
}

void mi_kv_destroy(mi_kv_pages *kv) { delete kv; }

int mi_kv_seals_for(int tier, const int *tier_map, const int *row_lengths, int map_rows,
                    int always_seal, int *out)
{
  return guarded([&] {
    *out = mi::KVPages::seals_for(tier, tier_map_of(tier_map, row_lengths, map_rows),
                                  always_seal != 0)
               ? 1
               : 0;
  });
}

int mi_kv_reserve(mi_kv_pages *kv, int tokens)
{
  return guarded([&] { kv->impl.reserve(tokens); });
}

int mi_kv_store(mi_kv_pages *kv, int layer, const void *keys, const void *values, int start, int n)
{
  return guarded([&] {
    if (n > 0)
    {
      need(keys, "keys");
      need(values, "values");
    }
    kv->impl.store(layer, keys, values, start, n);
  });
}

int mi_kv_attention(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                    mi_rope_table *rope, void *out, int seq_q, int seq_k, int heads, int kv_heads,
                    int head_dim, const void *keys, const void *values, float *mass, float *scores,
                    float alpha, float *partials)
{
  return guarded([&] {
    if (seq_q > seq_k)
    {
      throw mi::InvalidArgument("seq_q " + std::to_string(seq_q) + " exceeds seq_k " +
                                std::to_string(seq_k));
    }
    if (seq_q < 0)
    {
      throw mi::InvalidArgument("seq_q must not be negative, got " + std::to_string(seq_q));
    }
    const mi::RopeTable *table = rope != nullptr ? &rope->impl : nullptr;
    if (k_bias != nullptr && (table == nullptr || table->positions() < seq_k))
    {
      throw mi::InvalidArgument("a key bias needs a RoPE table for head_dim " +
                                std::to_string(head_dim) + " covering " + std::to_string(seq_k) +
                                " positions");
    }
    kv->impl.attention(layer, q, k_bias, table, out, seq_q, seq_k, heads, kv_heads, head_dim, keys,
                       values, mass, scores, alpha, partials);
  });
}

int mi_kv_attention_layers(mi_kv_pages *kv, int first_layer, int layers, const void *q,
                           long long q_stride, void *out, long long out_stride, int seq_k,
                           int heads, int kv_heads, int head_dim, const void *keys,
                           const void *values, long long kv_stride, float *mass,
                           long long mass_stride, float *scores, long long scores_stride,
                           float alpha)
{
  return guarded([&] {
    if (q == nullptr || out == nullptr)
    {
      throw mi::InvalidArgument("q and out must be device pointers, got null");
    }
    kv->impl.attention_layers(first_layer, layers, q, q_stride, out, out_stride, seq_k, heads,
                              kv_heads, head_dim, keys, values, kv_stride, mass, mass_stride,
                              scores, scores_stride, alpha);
  });
}

int mi_kv_attention_kept(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                         mi_rope_table *rope, void *out, int seq_k, int heads, int kv_heads,
                         int head_dim, const void *keys, const void *values)
{
  return guarded([&] {
    need(q, "q");
    need(out, "out");
    const mi::RopeTable *table = rope != nullptr ? &rope->impl : nullptr;
    if (k_bias != nullptr && (table == nullptr || table->positions() < seq_k))
    {
      throw mi::InvalidArgument("a key bias needs a RoPE table for head_dim " +
                                std::to_string(head_dim) + " covering " + std::to_string(seq_k) +
                                " positions");
    }
    kv->impl.attention_kept(layer, q, k_bias, table, out, seq_k, heads, kv_heads, head_dim, keys,
                            values);
  });
}

int mi_kv_fold_kept(mi_kv_pages *kv, float *mass, long long mass_stride, float *scores,
                    long long scores_stride, float alpha)
{
  return guarded([&] { kv->impl.fold_kept(mass, mass_stride, scores, scores_stride, alpha); });
}

int mi_kv_store_at(mi_kv_pages *kv, int layer, const void *keys, const void *values,
                   const int *position)
{
  return guarded([&] {
    need(kv, "kv");
    need(keys, "keys");
    need(values, "values");
    need(position, "position");
    kv->impl.store_step(layer, keys, values, position);
  });
}

int mi_kv_attention_at(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                       mi_rope_table *rope, void *out, const int *seq_k, int max_seq_k,
                       int heads, int kv_heads, int head_dim, const void *keys,
                       const void *values)
{
  return guarded([&] {
    need(kv, "kv");
    need(q, "q");
    need(out, "out");
    need(seq_k, "seq_k");
    need(keys, "keys");
    need(values, "values");
    kv->impl.attention_step(layer, q, k_bias, rope != nullptr ? &rope->impl : nullptr, out, seq_k,
                            max_seq_k, heads, kv_heads, head_dim, keys, values, nullptr);
  });
}

int mi_kv_rope_store(mi_kv_pages *kv, int layer, const void *qk, void *qk_out, int q_heads,
                     const int32_t *position, mi_rope_table *rope, const void *values,
                     const float *x, const void *norm_weight, void *normed, int hidden, float eps)
{
  return guarded([&] {
    need(kv, "kv");
    need(position, "position");
    need(rope, "rope");
    if (qk == qk_out)
    {
      throw mi::InvalidArgument("rope cannot write over its input");
    }
    kv->impl.rope_store(layer, qk, qk_out, q_heads, position, rope->impl, values, x, norm_weight,
                        normed, hidden, eps);
  });
}

int mi_kv_attend_row(mi_kv_pages *kv, int layer, const void *qk, void *qk_out, int q_heads,
                     int seq_k, mi_rope_table *rope, const void *values, void *out,
                     const float *x, const void *norm_weight, void *normed, int hidden, float eps)
{
  return guarded([&] {
    need(kv, "kv");
    need(rope, "rope");
    if (qk_out != nullptr && qk == qk_out)
    {
      throw mi::InvalidArgument("rope cannot write over its input");
    }
    kv->impl.attend_row(layer, qk, qk_out, q_heads, seq_k, rope->impl, values, out, x,
                        norm_weight, normed, hidden, eps);
  });
}

int mi_kv_stored_on_device(mi_kv_pages *kv, int end)
{
  return guarded([&] {
    need(kv, "kv");
    kv->impl.stored_on_device(end);
  });
}

int mi_decode_step_create(mi_decode_step **out, mi_kv_pages *kv, const mi_model_shape *shape,
                          const void *embed, const void *final_norm, const void *head,
                          const mi_layer_weights *layers, mi_scores *scores, int score_every)
{
  return guarded([&] {
    need(out, "out");
    need(kv, "kv");
    need(shape, "shape");
    need(layers, "layers");
    *out = nullptr;
    const mi::ModelShape sh{shape->layers,   shape->hidden,   shape->intermediate,
                            shape->heads,    shape->kv_heads, shape->head_dim,
                            shape->vocab,    shape->rms_eps,  shape->rope_theta};
    if (sh.layers <= 0)
    {
      throw mi::InvalidArgument("a model has at least one layer");
    }
    const auto half = [](const void *p) { return static_cast<const std::uint16_t *>(p); };
    mi::ModelWeights w{half(embed), half(final_norm), half(head), {}};
    for (int l = 0; l < sh.layers; ++l)
    {
      const mi_layer_weights &x = layers[l];
      w.layers.push_back({half(x.input_norm), half(x.q_w), half(x.q_b), half(x.k_w), half(x.k_b),
                          half(x.v_w), half(x.v_b), half(x.o_w), half(x.post_norm),
                          half(x.gate_w), half(x.up_w), half(x.down_w)});
    }
    *out = new mi_decode_step(kv->impl, sh, std::move(w),
                              scores != nullptr ? &scores->impl : nullptr, score_every);
  });
}

int mi_decode_step_destroy(mi_decode_step *step)
{
  return guarded([&] { delete step; });
}

int mi_decode_step_run(mi_decode_step *step, int token, int position, int steps,
                       int32_t *tokens, double *device_ms)
{
  return guarded([&] {
    need(step, "step");
    const double ms = step->impl.run(token, position, steps, tokens);
    if (device_ms != nullptr)
    {
      *device_ms = ms;
    }
  });
}

int mi_decode_step_run_eager(mi_decode_step *step, int token, int position, int steps,
                             int32_t *tokens, double *device_ms)
{
  return guarded([&] {
    need(step, "step");
    const double ms = step->impl.run(token, position, steps, tokens, false);
    if (device_ms != nullptr)
    {
      *device_ms = ms;
    }
  });
}

int mi_decode_step_prefill(mi_decode_step *step, const int32_t *tokens, int n, int position,
                           int chunk, int32_t *first, double *device_ms)
{
  return guarded([&] {
    need(step, "step");
    const double ms = step->impl.prefill(tokens, n, position, chunk, first);
    if (device_ms != nullptr)
    {
      *device_ms = ms;
    }
  });
}

int mi_decode_step_logits(mi_decode_step *step, float *out, size_t count)
{
  return guarded([&] {
    need(step, "step");
    need(out, "out");
    step->impl.logits(out, count);
  });
}

int mi_decode_step_launches(mi_decode_step *step, int *out)
{
  return guarded([&] {
    need(step, "step");
    need(out, "out");
    *out = step->impl.launches();
  });
}

int mi_decode_step_plans(mi_decode_step *step, int *out, size_t capacity, size_t *count)
{
  return guarded([&] {
    need(step, "step");
    need(count, "count");
    const std::vector<int> &plans = step->impl.plans();
    *count = plans.size();
    if (out != nullptr)
    {
      std::copy(plans.begin(), plans.begin() + std::min(capacity, plans.size()), out);
    }
  });
}

int mi_random_half(void *out, size_t count, unsigned long long seed, float scale)
{
  return guarded([&] {
    need(out, "out");
    mi::launch_random_half(out, count, seed, scale, mi::runtime_stream());
  });
}

int mi_kv_downgrade(mi_kv_pages *kv, int layer, int page, int target)
{
  return guarded([&] { kv->impl.downgrade(layer, page, target); });
}

int mi_kv_upgrade(mi_kv_pages *kv, int layer, int page, int target)
{
  return guarded([&] { kv->impl.upgrade(layer, page, target); });
}

int mi_kv_move_pages(mi_kv_pages *kv, const int *triples, size_t n)
{
  return guarded([&] {
    std::vector<mi::PageMove> moves;
    moves.reserve(n);
    for (size_t i = 0; i < n; ++i)
    {
      moves.push_back({{triples[3 * i], triples[3 * i + 1]}, triples[3 * i + 2]});
    }
    kv->impl.move_pages(moves);
  });
}

int mi_kv_pin_shadows(mi_kv_pages *kv, size_t pages)
{
  return guarded([&] { kv->impl.pin_shadows(pages); });
}

int mi_kv_evict(mi_kv_pages *kv, int layer, int page)
{
  return guarded([&] { kv->impl.evict(layer, page); });
}

int mi_kv_mask(mi_kv_pages *kv, int layer, int page)
{
  return guarded([&] { kv->impl.mask(layer, page); });
}

int mi_kv_page_tier(mi_kv_pages *kv, int layer, int page, int *tier)
{
  return guarded([&] { *tier = kv->impl.page_tier({layer, page}); });
}

int mi_kv_has_shadow(mi_kv_pages *kv, int layer, int page, int *out)
{
  return guarded([&] { *out = kv->impl.shadows().contains({layer, page}) ? 1 : 0; });
}

int mi_kv_shadow(mi_kv_pages *kv, int layer, int page, void *host, size_t bytes)
{
  return guarded([&] {
    const mi::ShadowStore &s = kv->impl.shadows();
    if (bytes != s.page_bytes())
    {
      throw mi::InvalidArgument("a shadow holds " + std::to_string(s.page_bytes()) + " bytes");
    }
    std::memcpy(host, s.shadow({layer, page}), bytes);
  });
}

int mi_kv_page_tiers(mi_kv_pages *kv, int8_t *out, size_t capacity)
{
  return guarded([&] {
    const int layers = kv->impl.layers();
    const int pages = kv->impl.pages_per_layer();
    if (capacity < static_cast<size_t>(layers) * pages)
    {
      throw mi::InvalidArgument("page_tiers needs layers * pages_per_layer entries");
    }
    for (int l = 0; l < layers; ++l)
    {
      for (int p = 0; p < pages; ++p)
      {
        out[static_cast<size_t>(l) * pages + p] = static_cast<int8_t>(
            kv->impl.evicted({l, p}) ? mi::kTierCount : kv->impl.page_tier({l, p}));
      }
    }
  });
}

int mi_kv_flags(mi_kv_pages *kv, int which, uint8_t *out, size_t capacity)
{
  return guarded([&] {
    const int layers = kv->impl.layers();
    const int pages = kv->impl.pages_per_layer();
    if (capacity < static_cast<size_t>(layers) * pages)
    {
      throw mi::InvalidArgument("flags need layers * pages_per_layer entries");
    }
    for (int l = 0; l < layers; ++l)
    {
      for (int p = 0; p < pages; ++p)
      {
        const mi::PageKey key{l, p};
        bool v = false;
        if (which == 0)
        {
          v = kv->impl.shadows().contains(key) && !kv->impl.evicted(key);
        }
        else if (which == 1)
        {
          v = kv->impl.evicted(key);
        }
        else
        {
          v = kv->impl.masked(key);
        }
        out[static_cast<size_t>(l) * pages + p] = v ? 1 : 0;
      }
    }
  });
}

int mi_kv_info_get(mi_kv_pages *kv, mi_kv_info *out)
{
  return guarded([&] {
    const mi::KVPages &k = kv->impl;
    out->layers = k.layers();
    out->page_tokens = k.page_tokens();
    out->kv_heads = k.kv_heads();
    out->head_dim = k.head_dim();
    out->pages_per_layer = k.pages_per_layer();
    out->capacity_tokens = k.capacity_tokens();
    out->tier = k.tier();
    out->halves = static_cast<int>(k.halves());
    out->storage_tier = k.storage_tier();
    out->seals = k.seals() ? 1 : 0;
    out->born_at_one_tier = k.born_at_one_tier() ? 1 : 0;
    out->page_bytes = k.page_bytes();
    out->kv_width = k.kv_width();
    out->shadow_count = k.shadows().count();
    out->shadow_bytes = k.shadows().bytes();
  });
}

int mi_kv_birth_tier(mi_kv_pages *kv, int layer, int page, int *tier)
{
  return guarded([&] { *tier = kv->impl.birth_tier(layer, page); });
}

int mi_kv_last_move(mi_kv_pages *kv, int *has, int *ints4, size_t *bytes2, double *seconds2)
{
  return guarded([&] {
    const auto &m = kv->impl.last_move();
    *has = m ? 1 : 0;
    if (m)
    {
      ints4[0] = m->key.layer;
      ints4[1] = m->key.page;
      ints4[2] = m->from_tier;
      ints4[3] = m->to_tier;
      bytes2[0] = m->from_bytes;
      bytes2[1] = m->to_bytes;
      seconds2[0] = m->seconds;
      seconds2[1] = m->shadow_seconds;
    }
  });
}

int mi_kv_last_batch(mi_kv_pages *kv, int *has, size_t *moves, size_t *shadows_taken,
                     double *seconds)
{
  return guarded([&] {
    const auto &b = kv->impl.last_batch();
    *has = b ? 1 : 0;
    if (b)
    {
      *moves = b->moves;
      *shadows_taken = b->shadows_taken;
      *seconds = b->seconds;
    }
  });
}

int mi_kv_last_batch_phases(mi_kv_pages *kv, double *phases)
{
  return guarded([&] {
    need(kv, "kv");
    need(phases, "phases");
    const auto &b = kv->impl.last_batch();
    phases[0] = b ? b->prepare_seconds : 0.0;
    phases[1] = b ? b->allocate_seconds : 0.0;
    phases[2] = b ? b->finish_seconds : 0.0;
  });
}

} // extern "C"
