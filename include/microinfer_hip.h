/*
 * microinfer_hip.h — the C ABI of the MI355X-native paged mixed-precision
 * KV-cache library (libmicroinfer_hip.so).
 *
 * This is the drop-in boundary for the reference's one native module,
 * `_microinfer` and its submodule `_microinfer.device`
 * (lecuong1502/Semantic-Aware_Adaptive_KV_Cache_Precision:
 * src/core_kernels/bindings.cpp:427-669, bindings_device.cpp:251-993).
 * Every entry point is `extern "C"` with plain pointers and sizes; the
 * Python shim `microinfer._microinfer` re-presents the reference's surface on
 * top of it through ctypes. Each declaration cites the reference interface it
 * replaces.
 *
 * Conventions.
 *   - Every function returns an mi_status; 0 is success. On failure
 *     mi_last_error() gives the message of the calling thread's last failure.
 *     The status picks the exception class the shim raises, as the
 *     reference's bindings map C++ exceptions (bindings.cpp:546-554).
 *   - "device" pointers are device-visible addresses (hipMalloc'd memory, or
 *     pinned host memory mapped for the device); "host" pointers are host
 *     memory. fp16 data is passed as raw 16-bit storage.
 *   - `stream` is a hipStream_t; 0 = the runtime's current stream, which
 *     every object of the runtime uses (the null stream unless
 *     mi_set_stream names another). Launchers enqueue and return without synchronising;
 *     execution errors surface at the next synchronising call
 *     (reference: device_ops.h:20-28).
 *   - Tiers: 0 FP16, 1 INT8, 2 INT4, 3 INT2 (reference: paged_kv_cache.h:16-25).
 *     A page-table tier of 0xFF is a page no query reads (device_ops.h:91-96).
 */
#ifndef MICROINFER_HIP_H
#define MICROINFER_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum mi_status {
  MI_OK = 0,
  MI_ERR_INVALID = 1,       /* std::invalid_argument -> ValueError            */
  MI_ERR_RANGE = 2,         /* std::out_of_range -> IndexError                */
  MI_ERR_NOT_FOUND = 3,     /* PageNotFound -> KeyError subclass              */
  MI_ERR_OPEN_PAGE = 4,     /* OpenPage -> ValueError subclass                */
  MI_ERR_OUT_OF_MEMORY = 5, /* OutOfMemory -> MemoryError subclass            */
  MI_ERR_LOGIC = 6,         /* std::logic_error -> RuntimeError               */
  MI_ERR_FULL = 7,          /* std::length_error "... is full" -> ValueError  */
  MI_ERR_DEVICE = 8         /* a HIP runtime error -> RuntimeError            */
} mi_status;

typedef struct mi_cache mi_cache;           /* PagedKVCache   */
typedef struct mi_kv_pages mi_kv_pages;     /* device.KVPages */
typedef struct mi_scores mi_scores;         /* device.ImportanceScores */
typedef struct mi_shadows mi_shadows;       /* device.ShadowStore */
typedef struct mi_rope_table mi_rope_table; /* device.RopeTable */

/* The calling thread's last error message ("" if none). */
const char *mi_last_error(void);
/* The library's build string: arch and flags. */
const char *mi_build_info(void);

/* ---- device and memory --------------------------------------------------
 * reference: device.cu:14-34 (device_name, device_memory_info),
 * device_tensor.cu:14-152 (DeviceTensor/DeviceFloats RAII storage),
 * paged_kv_cache.cu:46-60 (allocation_granularity). */
int mi_device_count(int *count);
int mi_device_name(char *out, size_t capacity);
/* The current device's PCI bus id ("dddd:bb:dd.f"), by which a management
 * library (amdsmi) finds the same GPU. No counterpart in the reference, whose
 * NVML reader takes device 0 (nvml.py:80-84). */
int mi_device_pci_bus_id(char *out, size_t capacity);
int mi_runtime_version(int *version);
/* reference: device.cu:10-17 cuda_driver_version (renamed: the HIP driver's). */
int mi_driver_version(int *version);
int mi_memory_info(size_t *free_bytes, size_t *total_bytes);
int mi_granule_bytes(size_t *out);
int mi_malloc(void **out, size_t bytes);
/* Pinned host memory mapped for the device (the memory FP16 shadows live
 * in): *host its host address, *device the address kernels use. For
 * measuring the host link a batch of moves crosses. No counterpart in the
 * reference. */
int mi_host_alloc(void **host, void **device, size_t bytes);
int mi_host_free(void *host);
int mi_free(void *ptr);
/* kind: 0 host-to-device, 1 device-to-host, 2 device-to-device. Synchronous. */
int mi_memcpy(void *dst, const void *src, size_t bytes, int kind);
int mi_memset(void *dst, int value, size_t bytes);
int mi_synchronize(void);
/* Timing on the stream a kernel runs on (hipEvent). */
int mi_event_create(void **event);
int mi_event_destroy(void *event);
int mi_event_record(void *event, void *stream);
int mi_event_elapsed_ms(void *start, void *end, float *ms);
/* Streams and graphs. A created stream has the default priority and orders
 * with the null stream. mi_set_stream picks the stream the runtime objects
 * (KVPages, PagedKVCache, ImportanceScores, RopeTable) launch on from the
 * calling thread; NULL is the null stream. A graph captures the launches made
 * on a stream between begin and end (hipStreamBeginCapture, thread-local
 * mode), to replay a launch-bound sequence, such as a decode step's attention
 * over every layer, with one launch. No counterpart in the reference, which
 * launches everything on the legacy default stream (device_ops.h:20-28). */
int mi_stream_create(void **stream);
int mi_stream_destroy(void *stream);
int mi_stream_synchronize(void *stream);
int mi_set_stream(void *stream);
int mi_graph_begin(void *stream);
int mi_graph_end(void *stream, void **exec);
int mi_graph_launch(void *exec, void *stream);
int mi_graph_destroy(void *exec);
/* Host conversions of the library's own rounding, for tests:
 * fp64 -> nearest fp16 bits in one rounding, and a group's stored scale
 * (reference: quant.cu:44-56 scale_of). Need no device. */
uint16_t mi_half_bits_from_double(double x);
uint16_t mi_scale_bits_of(float lo, float hi, int bits);

/* ---- quantised pages ----------------------------------------------------
 * reference: quant.h:45-59 QuantisedPageLayout, quant.cu:358-392. */
typedef struct mi_page_layout {
  int bits;
  size_t key_codes, value_codes, key_scales, key_zeros, value_scales, value_zeros;
  size_t metadata_bytes, page_bytes;
  double effective_bits;
} mi_page_layout;
int mi_quantised_page_layout(int tier, int page_tokens, int kv_heads, int head_dim,
                             mi_page_layout *out);
/* An FP16 page's bytes (reference: kv_pages.cu:62-66 page_bytes_for). */
size_t mi_fp16_page_bytes(int page_tokens, size_t kv_width);
/* One page (reference: quant.cu:403-417 device::quantise_page): keys and
 * values (page_tokens, kv_heads, head_dim) fp16 on the device, `filled`
 * positions of them; fewer than page_tokens is MI_ERR_OPEN_PAGE. */
int mi_quantise_page(const void *keys, const void *values, void *page, int tier,
                     int page_tokens, int filled, int kv_heads, int head_dim, void *stream);
/* A batch (reference: quant.cu:419-436 device::quantise_pages): page i from
 * rows[i] (an FP16 page, keys then values) into pages[i]; both tables in
 * device-visible memory; a row may be mapped pinned host memory. */
int mi_quantise_pages(const void *const *rows, void *const *pages, int count, int tier,
                      int page_tokens, int kv_heads, int head_dim, void *stream);
/* reference: quant.cu:438-450 device::dequantise_page. */
int mi_dequantise_page(const void *page, void *keys, void *values, int tier, int page_tokens,
                       int kv_heads, int head_dim, void *stream);

/* ---- attention ----------------------------------------------------------
 * reference: device_ops.h:61-147; attention.cu:1047-1142. Layout of q and
 * out (seq_q, heads, head_dim) fp16; k_bias (kv_heads, head_dim) fp16 or
 * NULL; rope a RopeTable's fp32 {cos, sin} (positions, head_dim/2, 2), read
 * only with k_bias. `partials` (mi_attention_partials_floats floats) lets a
 * long launch split its keys; NULL splits nothing. */
size_t mi_attention_partials_floats(int head_dim);
int mi_attention_split(int seq_q, int seq_k, int heads, int kv_heads, int page_tokens,
                       int *splits, int *split_keys);
/* Contiguous k, v (seq_k, kv_heads, head_dim) (reference: device::attention). */
int mi_attention(const void *q, const void *k, const void *v, const void *k_bias,
                 const float *rope, int rope_positions, void *out, int seq_q, int seq_k, int heads,
                 int kv_heads, int head_dim, float *partials, void *stream);
/* Through an FP16 page table of `pages` addresses (reference:
 * device::attention_paged). `mass` (heads, pages) fp32 or NULL. */
int mi_attention_paged(const void *q, const unsigned long long *pages, int page_tokens,
                       const void *k_bias, const float *rope, int rope_positions, void *out,
                       int seq_q, int seq_k, int heads, int kv_heads, int head_dim, float *mass,
                       float *partials, void *stream);
/* A cache that seals, read causally (reference: device::attention_paged_causal,
 * attention.cu:1091-1142): `sealed` and `tiers` the layer's table;
 * may_be_at_mask bit t set if a page may be at tier t; `open` the FP16 page
 * holding the own page's rows before seq_k - seq_q; chunk_k/chunk_v the
 * seq_q rows the queries brought. `scores`, if given, is the layer's row of
 * importance scores, into which the step's mass is folded with `alpha`
 * (reference: importance_scores.cu:74-98) in the same pass. */
int mi_attention_paged_causal(const void *q, const unsigned long long *sealed,
                              const uint8_t *tiers, int may_be_at_mask, const void *open,
                              const void *chunk_k, const void *chunk_v, int page_tokens,
                              const void *k_bias, const float *rope, int rope_positions, void *out,
                              int seq_q, int seq_k, int heads, int kv_heads, int head_dim,
                              float *mass, float *scores, float alpha, float *partials,
                              void *stream);

/* No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc). mi_attention_paged_causal's one-query decode (seq_q 1, no key
 * bias, split across pages) that allocates nothing: its scratch (split
 * partials and page statistics) is a static device array of 8 MiB that each
 * GPU holds until the process ends, instead of library memory. The caller
 * passes every input and output. Only what the decode fast path takes is
 * accepted (32-token pages, head_dim 64 or 128, at most 16 query heads a KV
 * head, 16-byte aligned q, open page and rows); anything else, or a decode
 * whose scratch would exceed 8 MiB (about 290K positions at Qwen2.5-1.5B's
 * shape), fails with MI_ERR_INVALID. Nothing in the scratch needs clearing:
 * every split and page writes its slot before the combine reads it. Every
 * call on one GPU shares that GPU's array, so calls that overlap on one GPU
 * (different streams, or threads) race; calls on one stream are ordered. */
int mi_attention_paged_causal_noalloc(const void *q, const unsigned long long *sealed,
                                      const uint8_t *tiers, int may_be_at_mask, const void *open,
                                      const void *chunk_k, const void *chunk_v, int page_tokens,
                                      void *out, int seq_k, int heads, int kv_heads, int head_dim,
                                      float *mass, float *scores, float alpha, void *stream);

/* ---- pages, rows and scores ----------------------------------------------
 * reference: page_copy.cu:41-70, kv_pages.cu:47-60, importance_scores.cu:18-50. */
int mi_copy_pages(const void *const *from, void *const *to, size_t bytes, int count, void *stream);
int mi_store_pages(const void *keys, const void *values, const unsigned long long *pages,
                   int page_tokens, size_t row, int start, int n, void *stream);
int mi_fill_f32(float *out, size_t count, float value, void *stream);
int mi_fold_scores(float *scores, const float *mass, int heads, int pages, float alpha,
                   void *stream);

/* ---- RoPE, RMSNorm, SwiGLU ------------------------------------------------
 * reference: rope.cu:57-68, rope_table.cu:18-68, rmsnorm.cu:87-109,
 * swiglu.cu:41-52, residual.cu (add). */
int mi_rope(const void *x, const int32_t *positions, void *out, int seq, int heads, int head_dim,
            double theta, void *stream);
int mi_rope_table_fill(float *table, int positions, int head_dim, double theta, void *stream);
int mi_rmsnorm(const void *x, int x_is_f32, const void *weight, void *out, int rows, int hidden,
               float eps, void *stream);
int mi_swiglu(const void *gate, const void *up, void *out, size_t count, void *stream);
int mi_add(const void *a, const void *b, void *out, size_t count, void *stream);

/* ---- Dense projections, embedding, logits ---------------------------------
 * fp16 operands, fp32 accumulation through hipBLASLt; W is (out, in) as the
 * checkpoint stores it, and y = x W^T.
 * mi_linear replaces device::linear (linear.cu:99-114; bindings_device.cpp:
 * 411-428, and the NumPy `linear`, bindings.cpp:513-517): y (rows, out) fp16,
 * the bias (out) fp16 or null added in fp32 before the one rounding.
 * mi_linear_f32 replaces device::linear_fp32_out (linear.cu:116-125) and,
 * with accumulate != 0, linear_accumulate (:127-138; bindings_device.cpp:
 * 351-365): out (rows, out) fp32 = or += x W^T. */
int mi_linear(const void *x, const void *weight, const void *bias, void *out, int rows,
              int in_features, int out_features, void *stream);
int mi_linear_f32(const void *x, const void *weight, float *out, int accumulate, int rows,
                  int in_features, int out_features, void *stream);
/* reference: embed.cu:60-76, bindings_device.cpp:321-334 (embed_f32) and
 * :383-396 (embed): out (count, hidden) = table rows ids[i], fp16 or widened
 * to fp32 (out_is_f32); an id outside [0, vocab) gives a zero row. */
int mi_embed(const int32_t *ids, int count, const void *table, void *out, int out_is_f32,
             int hidden, int vocab, void *stream);
/* reference: argmax.cu:71-81. out[r] = the index of row r's largest value,
 * the lowest on a tie; cols for a row with no value >= -FLT_MAX. */
int mi_argmax_rows(const float *x, int rows, int cols, int32_t *out, void *stream);
/* reference: bindings_device.cpp:109-195. scratch_elements: fp16 elements of
 * scratch that logits or greedy need for `rows` rows (fp32 logits, then the
 * int32 ids). mi_logits: fp32 logits of x's rows [first_row, first_row +
 * rows) through the (vocab, hidden) head, copied to host_out (rows, vocab),
 * synchronously. mi_greedy: each row's argmax id to host_ids; a row with no
 * finite logit fails with MI_ERR_LOGIC ("no finite logit"). Both run on the
 * runtime's current stream. */
int mi_scratch_elements(int rows, int vocab, size_t *out);
int mi_logits(const void *x, const void *head, void *scratch, size_t scratch_elements,
              int first_row, int rows, int hidden, int vocab, float *host_out);
int mi_greedy(const void *x, const void *head, void *scratch, size_t scratch_elements,
              int first_row, int rows, int hidden, int vocab, int32_t *host_ids);

/* ---- PagedKVCache: the per-tier VMM allocator ------------------------------
 * reference: paged_kv_cache.h:112-227, bindings.cpp:579-668. Keys are
 * (layer, page_index) int pairs. */
int mi_cache_create(const size_t page_bytes[4], const size_t capacity_pages[4], mi_cache **out);
void mi_cache_destroy(mi_cache *cache);
int mi_cache_allocate(mi_cache *cache, int layer, int page, int tier);
int mi_cache_free(mi_cache *cache, int layer, int page);
/* keys: n (layer, page) pairs, 2n ints. */
int mi_cache_free_pages(mi_cache *cache, const int *keys, size_t n);
int mi_cache_replace(mi_cache *cache, int layer, int page, int staged_layer, int staged_page);
/* quads: n (layer, page, staged_layer, staged_page), 4n ints. */
int mi_cache_replace_pages(mi_cache *cache, const int *quads, size_t n);
int mi_cache_write(mi_cache *cache, int layer, int page, const void *host, size_t bytes);
int mi_cache_read(mi_cache *cache, int layer, int page, void *host, size_t bytes);
int mi_cache_locate(mi_cache *cache, int layer, int page, int *tier, size_t *slot);
int mi_cache_contains(mi_cache *cache, int layer, int page, int *out);
/* The tier's keys in slot order: up to `capacity` pairs into keys (2 ints
 * each); *count receives the number held. */
int mi_cache_pages(mi_cache *cache, int tier, int *keys, size_t capacity, size_t *count);
int mi_cache_page_bytes(mi_cache *cache, int tier, size_t *out);
int mi_cache_reserved_bytes(mi_cache *cache, int tier, size_t *out);
int mi_cache_mapped_bytes(mi_cache *cache, int tier, size_t *out);
int mi_cache_keep_spare_granules(mi_cache *cache, int tier, size_t granules);
int mi_cache_spare_granules(mi_cache *cache, int tier, size_t *out);
int mi_cache_granule_bytes(mi_cache *cache, size_t *out);
/* Granules a range gives up are unmapped and released by a thread of the
 * cache's own, after the call that gave them up has returned (the reference
 * releases them inside that call, paged_kv_cache.cu). This waits until every
 * one is back with the driver. No counterpart in the reference. */
int mi_cache_drain_releases(mi_cache *cache);
/* Test hook (no counterpart in the reference; the reference forces the
 * same paths by exhausting VRAM): the next n granule maps fail as out of
 * memory. */
int mi_debug_fail_next_granules(int n);

/* ---- ShadowStore ------------------------------------------------------------
 * reference: shadow_store.h:23-85, bindings_device.cpp:652-686. */
int mi_shadows_create(size_t page_bytes, mi_shadows **out);
void mi_shadows_destroy(mi_shadows *s);
int mi_shadows_take(mi_shadows *s, int layer, int page, const void *device_page);
int mi_shadows_contains(mi_shadows *s, int layer, int page, int *out);
int mi_shadows_read(mi_shadows *s, int layer, int page, void *host, size_t bytes);
int mi_shadows_count(mi_shadows *s, size_t *out);
int mi_shadows_bytes(mi_shadows *s, size_t *out);

/* ---- ImportanceScores --------------------------------------------------------
 * reference: importance_scores.h:27-66, bindings_device.cpp:601-650. */
int mi_scores_create(int layers, int max_pages, float alpha, mi_scores **out);
void mi_scores_destroy(mi_scores *s);
int mi_scores_fold(mi_scores *s, int layer, const float *mass, int heads, int pages);
int mi_scores_download(mi_scores *s, float *host, size_t count);
int mi_scores_upload(mi_scores *s, const float *host, int layers, int max_pages);
int mi_scores_layer_row(mi_scores *s, int layer, float **row);
int mi_scores_info(mi_scores *s, int *layers, int *max_pages, float *alpha, size_t *downloads);

/* ---- RopeTable ----------------------------------------------------------------
 * reference: rope_table.h:25-44, bindings_device.cpp:529-566. */
int mi_rope_table_create(int head_dim, double theta, mi_rope_table **out);
void mi_rope_table_destroy(mi_rope_table *t);
int mi_rope_table_cover(mi_rope_table *t, int positions);
int mi_rope_table_info(mi_rope_table *t, int *positions, const float **data);
/* Beyond the reference (whose rope kernel forms every angle, rope.cu:57-68):
 * mi_rope's rotation of x (seq, heads, head_dim) fp16 at positions[token],
 * the angles read from a table that mi_rope_table_cover filled for
 * `table_positions` positions (every position must be below it); the rows are
 * mi_rope's to the bit. x == out is refused. */
int mi_rope_from_table(const void *x, const int32_t *positions, const float *table,
                       int table_positions, void *out, int seq, int heads, int head_dim,
                       void *stream);

/* ---- KVPages: the cache manager ---------------------------------------------------
 * reference: kv_pages.h:105-412, bindings_device.cpp:688-978. tier_map: a
 * flat array of `map_rows` rows, row l holding row_lengths[l] tiers; NULL for
 * none. halves: 0 Both, 1 Keys, 2 Values. The allocator must outlive it. */
int mi_kv_create(mi_cache *allocator, int layers, int page_tokens, int kv_heads, int head_dim,
                 int tier, int halves, const int *tier_map, const int *row_lengths, int map_rows,
                 int always_seal, mi_kv_pages **out);
void mi_kv_destroy(mi_kv_pages *kv);
int mi_kv_seals_for(int tier, const int *tier_map, const int *row_lengths, int map_rows,
                    int always_seal, int *out);
int mi_kv_reserve(mi_kv_pages *kv, int tokens);
/* keys, values: (n, kv_width) fp16 on the device. */
int mi_kv_store(mi_kv_pages *kv, int layer, const void *keys, const void *values, int start, int n);
/* reference: KVPages::attention (kv_pages.cu:901-947) with, beyond it,
 * `scores`/`alpha`: the step's mass folded into the layer's importance
 * scores in the same launch sequence. */
int mi_kv_attention(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                    mi_rope_table *rope, void *out, int seq_q, int seq_k, int heads, int kv_heads,
                    int head_dim, const void *keys, const void *values, float *mass, float *scores,
                    float alpha, float *partials);
/* Beyond the reference (which attends one layer a call, kv_pages.cu:901-947):
 * one decode query per head for `layers` consecutive layers in one launch,
 * for callers holding several layers' queries at once. Layer first_layer + i
 * reads q + i*q_stride, its own rows at keys/values + i*kv_stride, and writes
 * out + i*out_stride, mass + i*mass_stride, scores + i*scores_stride
 * (strides in elements; mass and scores may be NULL). Results are
 * mi_kv_attention's for each layer (seq_q 1, no key bias) within the
 * attention tolerance: the pages are split among waves differently. */
int mi_kv_attention_layers(mi_kv_pages *kv, int first_layer, int layers, const void *q,
                           long long q_stride, void *out, long long out_stride, int seq_k,
                           int heads, int kv_heads, int head_dim, const void *keys,
                           const void *values, long long kv_stride, float *mass,
                           long long mass_stride, float *scores, long long scores_stride,
                           float alpha);
/* Beyond the reference (which folds a layer's mass as it attends it,
 * model.py:280-286 with importance_scores.cu:74-98): a decode step whose
 * per-page mass is formed and folded once for every layer. Each layer's
 * mi_kv_attention_kept (one query a head, as mi_kv_attention with seq_q 1
 * and no mass) keeps its page statistics; mi_kv_fold_kept then writes every
 * layer's masses (mass + layer * mass_stride, if mass is given) and folds
 * them into the scores (scores + layer * scores_stride, if given) with
 * `alpha`, in one launch, to the bits mi_kv_attention gives with mass and
 * scores. Every layer must be attended, at one seq_k, between two folds. */
int mi_kv_attention_kept(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                         mi_rope_table *rope, void *out, int seq_k, int heads, int kv_heads,
                         int head_dim, const void *keys, const void *values);
int mi_kv_fold_kept(mi_kv_pages *kv, float *mass, long long mass_stride, float *scores,
                    long long scores_stride, float alpha);
/* Beyond the reference: the store and the decode of a step whose position
 * lives in device memory, what mi_decode_step's graph launches, for callers
 * that capture graphs of their own (the reference's KVPages.store and
 * attention take it from the host: kv_pages.h:161-195). mi_kv_store_at
 * stores one row (keys, values: kv_width fp16 each) at *position, read when
 * the kernel runs, sealing the page that row completes, as mi_kv_store does
 * for one row. mi_kv_attention_at decodes one layer (one query a head) at
 * seq_k = *seq_k, read when the kernels run, the launch sized for max_seq_k:
 * to the bit mi_kv_attention's with partials at that seq_k. Positions up to
 * max_seq_k must be reserved and no page may move while they run; the cache
 * must seal. mi_kv_stored_on_device records afterwards that every position
 * before `end` was stored. */
int mi_kv_store_at(mi_kv_pages *kv, int layer, const void *keys, const void *values,
                   const int *position);
int mi_kv_attention_at(mi_kv_pages *kv, int layer, const void *q, const void *k_bias,
                       mi_rope_table *rope, void *out, const int *seq_k, int max_seq_k,
                       int heads, int kv_heads, int head_dim, const void *keys,
                       const void *values);
int mi_kv_stored_on_device(mi_kv_pages *kv, int end);
/* Beyond the reference: a decode row's RoPE and store as one launch, for a
 * cache that does not seal (FP16 pages), where the reference makes three
 * calls (rmsnorm.cu:87-109, rope.cu:57-68 and KVPages.store,
 * kv_pages.h:161-180). qk holds q_heads then kv_heads rows of head_dim fp16;
 * they are rotated into qk_out at *position with rope's angles, and the
 * rotated k rows and `values` (kv_heads * head_dim fp16) are stored at that
 * position of `layer`. When x is not NULL, the RMSNorm of that fp32 row of
 * `hidden` values (weight norm_weight, eps) is written to `normed` in the
 * same launch. The bits are those of mi_rmsnorm, mi_rope_from_table and
 * mi_kv_store. The position must be reserved and below rope's positions
 * (read when the kernel runs: outside the reserved positions nothing is
 * stored). qk == qk_out is refused. */
int mi_kv_rope_store(mi_kv_pages *kv, int layer, const void *qk, void *qk_out, int q_heads,
                     const int32_t *position, mi_rope_table *rope, const void *values,
                     const float *x, const void *norm_weight, void *normed, int hidden, float eps);
/* Beyond the reference: mi_kv_rope_store at position seq_k - 1 and
 * mi_kv_attention's one-query split decode over the positions before seq_k
 * (kv_pages.h:163-179 KVPages.attention with partials) as two launches, the
 * pages launch and its combine, for a cache that does not seal. The pages
 * launch turns q and the row's k by RoPE in the waves that read them, stores
 * the turned k rows and `values` at seq_k - 1 by the wave that reads that
 * page, forms the RMSNorm of x (when not NULL) in one more workgroup, and
 * writes the turned rows to qk_out when it is not NULL. The bits of
 * mi_kv_rope_store then mi_kv_attention with partials. q_heads a whole
 * number of heads a KV head (at most 16); head_dim 64 or 128; 32-token pages;
 * rope covers seq_k positions; rows 16-byte aligned. */
int mi_kv_attend_row(mi_kv_pages *kv, int layer, const void *qk, void *qk_out, int q_heads,
                     int seq_k, mi_rope_table *rope, const void *values, void *out,
                     const float *x, const void *norm_weight, void *normed, int hidden, float eps);

/* ---- a whole decode step as one HIP graph (beyond the reference) ---------
 * The reference sequences a decode step from the host, a device call at a
 * time (src/microinfer/model.py:332-403 Model.run; the greedy loop of
 * engine.py:1180-1206). mi_decode_step captures every launch of a step --
 * embedding, per layer RMSNorm, the q/k/v projections, RoPE, the store, the
 * paged decode, the output projection into the fp32 residual, RMSNorm, gate
 * and up with SwiGLU, the down projection; then the final RMSNorm, the
 * head's logits and the greedy token -- as one graph whose kernels read the
 * step's token, position and seq_k from device memory, so one graph serves
 * every step of a run. Weights are fp16 device pointers, [out][in]; biases
 * may be NULL; a key bias (on every layer or on none) is added by attention,
 * rotated, as the reference does (ADR-0009). The cache must seal its pages
 * and outlive the step; `scores` (may be NULL) takes each step's masses at
 * seq_k a multiple of score_every. */
typedef struct mi_decode_step mi_decode_step;
typedef struct mi_model_shape {
  int layers;
  int hidden;
  int intermediate;
  int heads;
  int kv_heads;
  int head_dim;
  int vocab;
  float rms_eps;
  double rope_theta;
} mi_model_shape;
typedef struct mi_layer_weights {
  const void *input_norm;
  const void *q_w;
  const void *q_b;
  const void *k_w;
  const void *k_b;
  const void *v_w;
  const void *v_b;
  const void *o_w;
  const void *post_norm;
  const void *gate_w;
  const void *up_w;
  const void *down_w;
} mi_layer_weights;
int mi_decode_step_create(mi_decode_step **out, mi_kv_pages *kv, const mi_model_shape *shape,
                          const void *embed, const void *final_norm, const void *head,
                          const mi_layer_weights *layers, mi_scores *scores, int score_every);
int mi_decode_step_destroy(mi_decode_step *step);
/* `steps` greedy steps, the first feeding `token` at `position` (the cache
 * holds every position before it); the chosen tokens to `tokens` (host,
 * `steps` of them); *device_ms (may be NULL) the replays' device time. The
 * run reserves its pages first and records its stores after. */
int mi_decode_step_run(mi_decode_step *step, int token, int position, int steps,
                       int32_t *tokens, double *device_ms);
/* The same run with each step's launches made from the host in turn (no
 * graph), as the reference sequences a step: bit-identical to
 * mi_decode_step_run, for tools that follow individual launches. */
int mi_decode_step_run_eager(mi_decode_step *step, int token, int position, int steps,
                             int32_t *tokens, double *device_ms);
/* The prompt (n tokens from host memory) at positions [position,
 * position + n) in chunks of `chunk` rows, a layer at a time as the
 * reference's Model.run (model.py:332-403) takes a chunk: RMSNorm, q/k/v
 * projections, RoPE, store, the chunk's attention, output projection, MLP;
 * then the greedy token after the last row, to *first (feed it to
 * mi_decode_step_run at position + n). *device_ms (may be NULL) the
 * prefill's device time. */
int mi_decode_step_prefill(mi_decode_step *step, const int32_t *tokens, int n, int position,
                           int chunk, int32_t *first, double *device_ms);
/* The last step's logits, fp32, to host memory (count <= vocab). */
int mi_decode_step_logits(mi_decode_step *step, float *out, size_t count);
int mi_decode_step_launches(mi_decode_step *step, int *out);
/* No counterpart in the reference (its projections are cuBLAS calls,
 * linear.cu:85-142): the plans the last step's GEMVs ran as, seven ints
 * each -- which one (0 layer 0's output projection, 1 its gate/up, 2 its
 * down projection, 3 the head), rows, input length, the waves a row is
 * split over, 1 if the grid was the device's resident one with several rows
 * a wave, waves a workgroup, workgroups. *count the ints there are; up to
 * `capacity` of them to `out` (may be NULL). */
int mi_decode_step_plans(mi_decode_step *step, int *out, size_t capacity, size_t *count);
/* Synthetic fp16 weights made on the device: uniform in [-scale, scale)
 * from `seed`. */
int mi_random_half(void *out, size_t count, unsigned long long seed, float scale);
int mi_kv_downgrade(mi_kv_pages *kv, int layer, int page, int target);
int mi_kv_upgrade(mi_kv_pages *kv, int layer, int page, int target);
/* triples: n (layer, page, target tier), 3n ints. */
int mi_kv_move_pages(mi_kv_pages *kv, const int *triples, size_t n);
/* Pins host memory for `pages` more FP16 shadows now, so that first
 * downgrades later pin nothing on their own path. No counterpart in the
 * reference, whose shadows are pinned as they are taken; its ADR-0015
 * (:202-208) names pinning ahead of need as the remedy for a first
 * downgrade's cost. shadow_bytes counts what is pinned. */
int mi_kv_pin_shadows(mi_kv_pages *kv, size_t pages);
int mi_kv_evict(mi_kv_pages *kv, int layer, int page);
int mi_kv_mask(mi_kv_pages *kv, int layer, int page);
int mi_kv_page_tier(mi_kv_pages *kv, int layer, int page, int *tier);
int mi_kv_has_shadow(mi_kv_pages *kv, int layer, int page, int *out);
int mi_kv_shadow(mi_kv_pages *kv, int layer, int page, void *host, size_t bytes);
/* Per-page arrays (layers, pages_per_layer): tiers as page_tiers gives them
 * (evicted = 4), and shadowed / evicted flags. */
int mi_kv_page_tiers(mi_kv_pages *kv, int8_t *out, size_t capacity);
int mi_kv_flags(mi_kv_pages *kv, int which, uint8_t *out, size_t capacity);
typedef struct mi_kv_info {
  int layers, page_tokens, kv_heads, head_dim, pages_per_layer, capacity_tokens;
  int tier, halves, storage_tier, seals, born_at_one_tier;
  size_t page_bytes, kv_width, shadow_count, shadow_bytes;
} mi_kv_info;
int mi_kv_info_get(mi_kv_pages *kv, mi_kv_info *out);
int mi_kv_birth_tier(mi_kv_pages *kv, int layer, int page, int *tier);
/* last_move: has, layer, page, from, to; bytes; seconds. */
int mi_kv_last_move(mi_kv_pages *kv, int *has, int *ints4, size_t *bytes2, double *seconds2);
int mi_kv_last_batch(mi_kv_pages *kv, int *has, size_t *moves, size_t *shadows_taken,
                     double *seconds);
/* Where the last batch's seconds went (no counterpart in the reference):
 * phases[0] the host's work before the first launch, [1] the new pages'
 * allocation, [2] the page table's switch, the old pages' release and the
 * wait for the device. */
int mi_kv_last_batch_phases(mi_kv_pages *kv, double *phases);

#ifdef __cplusplus
}
#endif

#endif /* MICROINFER_HIP_H */
