// Launchers of the library's HIP kernels. Each enqueues on `stream` and
// returns without synchronising; launch errors throw at once, execution
// errors surface at the next synchronising call.
#pragma once

#include "common.hpp"

namespace mi
{

  // ---- requantisation (quant.hip) ------------------------------------------------
  // Quantises `count` FP16 pages at `tier`: page i's keys from rows[i] and its
  // values from rows[i] + values_offset bytes, into pages[i]. `rows` and
  // `pages` are device-visible tables (pinned host memory mapped for the
  // device is a valid row). With null tables, one page: row0 -> page0.
  void launch_quantise_pages(const void *const *rows, void *const *pages, const void *row0,
                             void *page0, std::ptrdiff_t values_offset, int count, int tier,
                             int page_tokens, int kv_heads, int head_dim, hipStream_t stream);
  void launch_dequantise_page(const void *page, void *keys, void *values, int tier,
                              int page_tokens, int kv_heads, int head_dim, hipStream_t stream);

  // ---- page jobs by reference (page_jobs.hip) -----------------------------------
  // A page's place as 32 bits: the space that holds it (bits 29-31) and its
  // index there. Spaces 0-3 are the allocator's four tier ranges (the index
  // a slot), space 4 the FP16 shadows in pinned host memory (the index a
  // shadow number), space 5 FP16 pages staged in device memory. Kernels turn a reference into an address themselves, so
  // a batch sends 8 bytes a page pair to the device, not two addresses.
  constexpr int kShadowSpace = 4;
  constexpr int kStagingSpace = 5; // FP16 pages staged in device memory, by index
  constexpr unsigned kRefIndexBits = 29;
  constexpr std::uint32_t kRefIndexMask = (1u << kRefIndexBits) - 1;
  __host__ __device__ constexpr std::uint32_t page_ref(int space, std::uint32_t index)
  {
    return (static_cast<std::uint32_t>(space) << kRefIndexBits) | index;
  }

  // Where the spaces are: each tier range's base and page size (fixed for an
  // allocator's life), and the device table of the shadows' mapped addresses.
  struct PageSpaces
  {
    unsigned long long base[kTierCount];
    unsigned long long bytes[kTierCount];
    const unsigned long long *shadows; // shadow number -> device address
    unsigned long long shadow_bytes;   // an FP16 page
    unsigned long long staging;        // base of the staged FP16 pages, shadow_bytes apart
  };

  struct RefPair
  {
    std::uint32_t from;
    std::uint32_t to;
  };

  // A launch's page pairs: in device memory (`pairs`), or, for a few, held
  // in the launch's own arguments (`pairs` null), so that a small batch
  // (a single move, a free's one tail move) uploads nothing first.
  constexpr int kHeldRefs = 4;
  struct RefList
  {
    const RefPair *pairs;
    RefPair held[kHeldRefs];
  };
  // Pairs [first, first + count) of `host` as a RefList: held when count is
  // at most kHeldRefs, else `uploaded` (where `host` was uploaded whole) +
  // first.
  RefList ref_list(const std::vector<RefPair> &host, std::size_t first, std::size_t count,
                   const RefPair *uploaded);

  // Copies pair i's page from `from` to `to`: the destination space's page
  // size (an FP16 page when either side is a shadow). No copy may read
  // what another writes.
  void launch_copy_refs(const RefList &pairs, int count, const PageSpaces &spaces,
                        hipStream_t stream);
  // Quantises pair i's FP16 page (a slot of the FP16 range, or a shadow) to
  // `tier` into its destination slot. head_dim 64 or 128, 32-token pages and
  // kv_heads * head_dim >= 128 take the register quantiser (a lane a task of
  // 64 elements, nothing staged); any other shape the LDS one.
  // One page's move as one launch (one workgroup): the page's FP16 bytes to
  // its shadow (shadow.from -> shadow_at, the new shadow's mapped address,
  // so that the launch needs no upload of the shadow table) when has_shadow;
  // the shadow's rows
  // into device staging (stage.from -> stage.to) when has_stage, then a
  // barrier; the page at its new tier (page.from, FP16 rows, -> page.to: the
  // register quantiser at `tier`, or a copy at FP16); then, after a barrier,
  // the compaction copies of the tier the page left, which may overwrite
  // what came before them. It applies at a shape the register quantiser
  // takes (move_one_applies): a move from FP16 (its rows the page), and a
  // move of a page that has a shadow (its rows the shadow: copied at FP16,
  // staged first for a quantised tier, whose quantiser reads its rows
  // twice); anything else takes the separate launches.
  struct OneMove
  {
    RefPair shadow;
    RefPair page;
    RefPair compact[kHeldRefs];
    int has_shadow;
    int tier;
    int compact_count;
    RefPair stage;
    int has_stage;
    unsigned long long shadow_at;
  };
  bool launch_move_one(const OneMove &m, const PageSpaces &spaces, int page_tokens, int kv_heads,
                       int head_dim, hipStream_t stream);
  bool move_one_applies(int from, int tier, int page_tokens, int kv_heads, int head_dim);
  void launch_requant_refs(const RefList &pairs, int count, int tier, const PageSpaces &spaces,
                           int page_tokens, int kv_heads, int head_dim, hipStream_t stream);
  // The register quantiser over pages named by address (launch_quantise_pages'
  // arguments): false, launching nothing, for a shape it does not take
  // (not 32-token pages at head_dim 64/128, or rows not 16-byte aligned).
  bool launch_quantise_registers(const void *const *rows, void *const *pages, const void *row0,
                                 void *page0, std::ptrdiff_t values_offset, int count, int tier,
                                 int page_tokens, int kv_heads, int head_dim, hipStream_t stream);

  // A job on one page's rows, as a cache's store makes them. A page's keys
  // are rows of kv_heads * head_dim fp16; rows [0, split) come from k_lo /
  // v_lo (an open page's), rows [split, P) from k_hi / v_hi (the rows the
  // store brought), row t at k_hi + (t - split) * width.
  enum class RowJobKind : int
  {
    kQuantise = 0,  // seal at `tier` into the page at dst
    kCopy = 1,      // seal at FP16: the rows as they are
    kRoundKeys = 2, // the diagnostic Halves: keys through `tier` and back, values as they are
    kRoundValues = 3,
    kFill = 4,      // rows [0, rows) of k_hi / v_hi to rows [dst_row, dst_row + rows) of an
                    // open page at dst
  };
  struct RowJob
  {
    const std::uint16_t *k_lo;
    const std::uint16_t *v_lo;
    const std::uint16_t *k_hi;
    const std::uint16_t *v_hi;
    std::uint8_t *dst;
    int split;
    int kind;
    int tier;
    int rows;
    int dst_row;
    int pad;
  };
  constexpr int kRowJobsALaunch = 24;
  // The jobs of one store, every kind in one launch (in launches of
  // kRowJobsALaunch, passed by value: a decode step's store sends nothing
  // ahead of its launch).
  void launch_row_jobs(const RowJob *jobs, int count, int page_tokens, int kv_heads, int head_dim,
                       hipStream_t stream);

  // Page table edits: entry `index` of the address and tier arrays set.
  struct TableEdit
  {
    unsigned long long address;
    std::uint32_t index;
    std::uint32_t tier;
  };
  void launch_table_edits(const TableEdit *edits, int count, unsigned long long *addresses,
                          std::uint8_t *tiers, hipStream_t stream);

  // ---- pages and scores (pages.hip) ----------------------------------------------
  // from[i] -> to[i], `bytes` each, `count` pages, one launch; tables on the
  // device. No copy may read what another writes.
  void launch_copy_pages(const void *const *from, void *const *to, std::size_t bytes, int count,
                         hipStream_t stream);
  // Rows of n tokens, (n, row) fp16 keys and values, to positions
  // [start, start + n) of an FP16 page table (P rows of keys then P of values).
  void launch_store_pages(const void *keys, const void *values, const unsigned long long *pages,
                          int page_tokens, std::size_t row, int start, int n, hipStream_t stream);
  void launch_fill(float *out, std::size_t count, float value, hipStream_t stream);
  // scores[p] = isnan(old) ? obs : alpha*obs + (1-alpha)*old with obs the
  // head-order sum of mass[h][p] over `heads` divided by heads, every
  // operation rounded once (reference: importance_scores.cu:31-50).
  void launch_fold(float *scores, const float *mass, int heads, int pages, float alpha,
                   hipStream_t stream);

  // ---- pointwise (pointwise.hip) --------------------------------------------------
  void launch_rope(const void *x, const std::int32_t *positions, void *out, int seq, int heads,
                   int head_dim, double theta, hipStream_t stream);
  // fp16 high and low parts of a RoPE table's cos (channels < head_dim/2)
  // and sin (the rest) per position: [position][hi | lo][head_dim].
  void launch_rope_angles(const float *table, std::uint16_t *angles, int positions, int head_dim,
                          hipStream_t stream);
  void launch_rope_table(float *table, int positions, int head_dim, double theta,
                         hipStream_t stream);
  // RoPE of up to two sets of rows ((seq, heads[i], head_dim) fp16 each;
  // heads[1] 0 for one set) at positions[token], the angles from a table
  // launch_rope_table filled for table_positions positions: launch_rope's
  // rows to the bit, without forming an angle a pair.
  struct RopeRows
  {
    const void *x[2];
    void *out[2];
    int heads[2];
    const std::int32_t *positions;
    const float *table;
    int table_positions;
    int seq;
    int head_dim;
  };
  void launch_rope_rows(const RopeRows &r, hipStream_t stream);
  // One decode row's RMSNorm (x: one fp32 row, optional), the RoPE of its q
  // and k heads (qk: q_heads then kv_heads rows of head_dim fp16) at
  // *position with the table's angles, and the rotated k and the values
  // stored in the layer's FP16 page at that position (pages: the layer's
  // page addresses; positions outside [0, positions) store nothing).
  struct RowPrep
  {
    const float *x;
    const std::uint16_t *norm_weight;
    std::uint16_t *normed;
    int hidden;
    float eps;
    const std::uint16_t *qk;
    std::uint16_t *qk_out;
    int q_heads;
    int kv_heads;
    int head_dim;
    const std::int32_t *position;
    const float *table;
    int table_positions;
    const std::uint16_t *values;
    const unsigned long long *pages;
    int page_tokens;
    int positions;
  };
  void launch_row_prep(const RowPrep &r, hipStream_t stream);
  void launch_rmsnorm(const void *x, bool x_is_f32, const void *weight, void *out, int rows,
                      int hidden, float eps, hipStream_t stream);
  void launch_swiglu(const void *gate, const void *up, void *out, std::size_t count,
                     hipStream_t stream);
  void launch_add(const void *a, const void *b, void *out, std::size_t count, hipStream_t stream);

  // ---- dense projections and their neighbours (linear.cpp, dense.hip) ------------------
  // y = x W^T (+ bias): x (rows, in) fp16, W (out, in) fp16, y (rows, out)
  // fp16, fp32 accumulation and one rounding; bias (out) fp16 or null.
  void linear_half(const void *x, const void *weight, const void *bias, void *out, int rows,
                   int in_features, int out_features, hipStream_t stream);
  // y = x W^T in fp32, or y += x W^T when `accumulate`.
  void linear_float(const void *x, const void *weight, float *out, bool accumulate, int rows,
                    int in_features, int out_features, hipStream_t stream);
  // out row t = table row ids[t] (fp16, or widened to fp32); an id outside
  // [0, vocab) gives a zero row.
  void launch_embed(const std::int32_t *ids, int count, const void *table, void *out,
                    bool out_is_f32, int hidden, int vocab, hipStream_t stream);
  // out[r] = the index of row r's largest value, the lowest on a tie; cols
  // for a row with no value >= -FLT_MAX.
  void launch_argmax_rows(const float *x, int rows, int cols, std::int32_t *out,
                          hipStream_t stream);
  // Every row of out (rows, cols) fp16 = row (cols), or zero when row is null.
  void launch_broadcast_rows(const void *row, void *out, int rows, int cols, hipStream_t stream);

  // ---- attention (attention.hip, decode.hip) -------------------------------------------
  // Where keys and values are read from. Contiguous: k and v (seq_k, kv, hd).
  // Paged: an FP16 page table, `pages`, P rows of keys then values. Causal:
  // a cache that seals: sealed pages at the tier `tiers` records, the
  // query's own page from `open` (FP16 page) before `start` and from
  // chunk_k/chunk_v (the rows the queries brought) from `start` on.
  enum class Layout : int
  {
    kContiguous = 0,
    kPaged = 1,
    kCausal = 2,
  };

  struct KVSource
  {
    Layout layout;
    // Contiguous.
    const std::uint16_t *k;
    const std::uint16_t *v;
    // Paged and causal.
    const unsigned long long *pages;
    const std::uint8_t *tiers;
    const std::uint16_t *open;
    const std::uint16_t *chunk_k;
    const std::uint16_t *chunk_v;
    int page_tokens;
    int start;
    // Which tiers a page may be at: a layout is formed for each.
    bool may_be_at[kTierCount];
    // Decode of one layer: the next layer's page table (its first warm_count
    // entries), which the launch reads ahead once its own work is done, so
    // that the next layer's first trip to memory finds it in cache. Null:
    // none.
    const unsigned long long *warm_pages;
    const std::uint8_t *warm_tiers;
    int warm_count;
  };

  // Device scratch a launch needs beside its inputs and outputs (the decode
  // path's split partials and page statistics): `count` floats on the
  // stream the launch goes on, valid until the next request of the same
  // source. An owner (a KVPages, the allocation-free entry point's static
  // array) gives its own; a launch without one takes the caller's partials
  // buffer when it is large enough, else a library buffer of the stream's.
  struct WorkspaceSource
  {
    virtual float *floats(std::size_t count) = 0;

  protected:
    ~WorkspaceSource() = default;
  };
  // The library's scratch for launches on `stream`: one buffer a stream,
  // grown on demand and never freed before the process ends (an address a
  // captured graph holds stays valid). Launches on different streams never
  // share one; launches on one stream are ordered by it.
  float *stream_workspace(hipStream_t stream, std::size_t count);

  struct AttentionArgs
  {
    const std::uint16_t *q;   // (seq_q, heads, hd) fp16
    std::uint16_t *out;       // (seq_q, heads, hd) fp16
    const std::uint16_t *k_bias; // (kv_heads, hd) fp16 or null
    const float *rope;        // {cos, sin} per (position, j < hd/2), fp32; with k_bias
    int rope_positions;
    // The first 32 positions' angles as fp16 high and low parts
    // ([position][hi | lo][hd]), when the caller has them (a RopeTable's):
    // the decode fast path takes the key bias only with these.
    const std::uint16_t *rope_angles;
    int seq_q;
    int seq_k;
    int heads;
    int kv_heads;
    int head_dim;
    float *mass;              // (heads, pages) fp32 or null; decode only
    float *scores;            // this layer's importance scores or null; decode only
    float alpha;
    float *partials;          // attention_partials_floats(hd) or null: no split
    std::size_t partials_floats; // its size, when the caller knows it (0: unknown)
    WorkspaceSource *workspace;  // the decode path's scratch, or null (see above)
  };

  // How a launch given partials splits its keys: runs and keys a run.
  struct Split
  {
    int splits;
    int split_keys;
  };
  Split attention_split(int seq_q, int seq_k, int heads, int kv_heads, int page_tokens);
  std::size_t attention_partials_floats(int head_dim);
  int device_multiprocessors();

  void launch_attention(const KVSource &kv, const AttentionArgs &a, hipStream_t stream);

  // The matrix-core chunk path (prefill.hip): any number of queries, no mass,
  // head_dim 64 or 128, 32-key pages (or a contiguous cache), 16-byte aligned
  // rows. launch_attention takes it when it applies and the decode fast path
  // does not.
  bool prefill_applies(const KVSource &kv, const AttentionArgs &a);
  void launch_prefill(const KVSource &kv, const AttentionArgs &a, hipStream_t stream);

  // The decode fast path (decode.hip) over `layers` consecutive layers of one
  // cache in one launch. Layer first_layer + i reads its page addresses and
  // tiers at kv.pages / kv.tiers + (first_layer + i) * table_stride, its open
  // page at open_table[first_layer + i] (kv.open when open_table is null),
  // and its q, chunk rows, output, mass and scores at i times the strides
  // (in elements) from the AttentionArgs / KVSource bases. AttentionArgs'
  // partials are not read: the fast path keeps its own workspace.
  struct StepStore;

  struct DecodeLayers
  {
    bool split; // a wave a page and a combine; else a workgroup a KV head
    int first_layer;
    int layers;
    long long table_stride;
    const unsigned long long *open_table;
    long long q_stride;
    long long chunk_stride;
    long long out_stride;
    long long mass_stride;
    long long scores_stride;
    // A decode whose page statistics are kept for a later fold (one layer,
    // split, no mass or scores of its own): its split maxima and sums and
    // its page statistics go here, in a DecodeFold's layout for its layer.
    float *keep_ml;
    float *keep_stats;
    // A decode whose position lives on the device (one layer, split, not
    // several layers at once): seq_k is read from *live_seq_k when the
    // kernels run, and AttentionArgs::seq_k is the most it may be, which
    // sizes the launch and the strides.
    const int *live_seq_k;
    // With a live position: the step's page seal, done by one more
    // workgroup of the combine when *seal->position is its page's last row
    // (the page quantised, or copied at FP16, from the open page's rows and
    // the step's k and v rows into its slot). Null: no seal.
    const StepStore *seal;
    // The row launch's work done by the pages launch (one split layer of
    // FP16 pages of a cache that does not seal, no key bias): RMSNorm of
    // row->x by one more workgroup, q and the current row's k (position
    // AttentionArgs::seq_k - 1, which row->table covers) turned by RoPE in
    // the waves that read them, and that row's k and values stored into its
    // page (row->pages) by the wave that reads the page. AttentionArgs::q is
    // row->qk's raw q rows; row->qk_out (optional) receives the turned rows.
    // Null: none.
    const RowPrep *row;
  };
  // Whether the fast path takes this decode: one query, no key bias, 32-token
  // pages, head_dim 64 or 128, a group of at most 16 heads, 16-byte aligned
  // rows and page regions.
  bool decode_fast_applies(const KVSource &kv, const AttentionArgs &a);
  void launch_decode_layers(const KVSource &kv, const AttentionArgs &a, const DecodeLayers &ls,
                            hipStream_t stream);

  // The fold of decodes that kept their statistics: every layer's page
  // masses (into mass + layer * mass_stride, if given) and its importance
  // scores (scores + layer * scores_stride, if given) in one launch, to the
  // same bits the fused form gives. `kept` holds, for `layers` layers of one
  // step (the same seq_k), first every layer's split maxima and sums
  // [layer][heads][splits][2], then every layer's page statistics
  // [layer][kv_heads][pages][group][2]; decode_kept_floats is one layer's share.
  struct DecodeFold
  {
    int layers;
    int heads;
    int kv_heads;
    int head_dim;
    int seq_k;
    float *kept;
    float *mass;
    long long mass_stride;
    float *scores;
    long long scores_stride;
    float alpha;
    // With the position on the device: seq_k read from *live_seq_k, `seq_k`
    // above the most it may be (the kept layout's size); the fold runs only
    // where that seq_k is a multiple of score_every.
    const int *live_seq_k;
    int score_every;
  };
  std::size_t decode_kept_floats(int heads, int kv_heads, int seq_k);
  void launch_decode_fold(const DecodeFold &f, hipStream_t stream);

  // ---- a decode step's dense half (step.hip) ---------------------------------------------
  // One token's projections against fp16 weights [rows][in]: q, k and v in
  // one launch (up to three matrices), gate and up with the SwiGLU, the
  // fp32 residual accumulated, the head's logits with each block's best.
  enum class ProjectMode : int
  {
    kHalf,       // out fp16 = acc + bias (fp32, one rounding)
    kAccumulate, // out fp32 += acc
    kSwiglu,     // seg[0] gate, seg[1] up: seg[0].out fp16 = silu(g) u
    kLogits,     // out fp32 = acc, and each block's best (value, index)
  };
  constexpr int kProjectSegments = 3;
  struct ProjectSegment
  {
    const std::uint16_t *w;
    const std::uint16_t *bias; // kHalf only; may be null
    void *out;
    int rows;
  };
  struct ProjectArgs
  {
    ProjectSegment seg[kProjectSegments];
    int segments;
    int in;
    const std::uint16_t *x;
    ProjectMode mode;
    float *best_value; // kLogits: [project_blocks]
    int *best_index;
    int best_count; // kLogits: the entries best_value and best_index hold
    // With norm_weight: x is RMSNorm of the fp32 `residual` row (in values),
    // formed in the launch as the RMSNorm kernel forms it, to the bit.
    const float *residual;
    const std::uint16_t *norm_weight;
    float eps;
  };
  // The workgroups launch_project makes for `p` (its mode, segments' rows
  // and input length): the entries a kLogits call's best arrays need.
  int project_blocks(const ProjectArgs &p);
  // The variant a projection ran as: the waves a row is split over, whether
  // the grid is the device's resident one with several rows a wave, the
  // waves a workgroup and the workgroups launched.
  struct ProjectPlanInfo
  {
    int split;
    int pipelined;
    int waves;
    int blocks;
  };
  ProjectPlanInfo launch_project(const ProjectArgs &p, hipStream_t stream);
  // A step's state in device memory, four ints.
  constexpr int kStepToken = 0;    // the token the step feeds
  constexpr int kStepPosition = 1; // its position
  constexpr int kStepSeqK = 2;     // positions attended: position + 1
  constexpr int kStepIndex = 3;    // steps taken in the run
  // The greedy token from the head's block bests, written to tokens[step]
  // (while step < max_tokens) and as the next step's token; the state moved on.
  void launch_advance(const float *best_value, const int *best_index, int blocks, int vocab,
                      int *state, std::int32_t *tokens, int max_tokens, hipStream_t stream);
  // Synthetic fp16 weights: uniform in [-scale, scale), from a seed.
  void launch_random_half(void *out, std::size_t count, unsigned long long seed, float scale,
                          hipStream_t stream);

  // A decode step's store with its position on the device (page_jobs.hip):
  // the rows go to row position % 32 of the layer's open page, and the row
  // that completes a page seals it, at its tier in the table, from the open
  // page and the rows (store_sealed's jobs for one row, chosen on the device).
  struct StepStore
  {
    const std::uint16_t *keys;
    const std::uint16_t *values;
    const int *position;
    std::uint16_t *open;
    const unsigned long long *addresses; // the layer's row of the page table
    const std::uint8_t *tiers;
    int kv_heads;
    PageLayout lay[kTierCount];
  };
  void launch_step_store(const StepStore &s, int head_dim, hipStream_t stream);

  // One decode step's q, k and v of a layer in one launch: the projections
  // of RMSNorm(residual) (formed in the launch, to the RMSNorm kernel's
  // bits), a wave the two rows of one rotation pair (channels j and
  // j + head_dim/2 of a head), each row's bias added before its one rounding
  // to fp16 (the projection's arithmetic); q and k then rotated at
  // *position (the RoPE kernel's arithmetic) into qk = [q | k], v into v;
  // k's and v's rows also written into the open page at row *position % 32
  // unless that is the page's last row, whose seal reads them from qk and v
  // (DecodeLayers::seal). Bit-identical to the projection, RoPE and store
  // launched apart.
  struct QkvStep
  {
    const std::uint16_t *w[3]; // q, k, v weights, [rows][in]
    const std::uint16_t *b[3]; // their biases, or null
    int in;
    const float *residual;
    const std::uint16_t *norm_weight;
    float eps;
    int heads;
    int kv_heads;
    int head_dim;
    const float *rope; // {cos, sin} per (position, j < head_dim / 2)
    const int *position;
    std::uint16_t *qk; // heads * head_dim of q, then kv_heads * head_dim of k
    std::uint16_t *v;
    std::uint16_t *open; // the layer's open page: P rows of keys, then P of values
  };
  void launch_qkv_step(const QkvStep &s, hipStream_t stream);

} // namespace mi
