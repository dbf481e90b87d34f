// The cache runtime on the host: the per-tier page allocator, the pinned
// FP16 shadow store, the importance scores, the RoPE table, and KVPages, the
// cache manager that stores, seals, attends and moves pages between tiers.
//
// The classes keep the reference's names and observable behaviour
// (src/core_kernels/paged_kv_cache.h, shadow_store.h, importance_scores.h,
// rope_table.h, kv_pages.h): slot order, error classes and messages, what a
// page holds after every operation. How they drive the device is this
// build's own: page tables kept current by edits the allocator reports as
// pages move, batches named by 32-bit page references that the kernels turn
// into addresses, granules released off the caller's path once the device
// has passed their last use, and one launch for all of a store's seals.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

#include <array>
#include <condition_variable>
#include <deque>
#include <memory>
#include <mutex>
#include <optional>
#include <thread>
#include <unordered_map>
#include <utility>
#include <vector>

namespace mi
{

  struct PageKey
  {
    int layer;
    int page;
    bool operator<(const PageKey &o) const
    {
      return layer != o.layer ? layer < o.layer : page < o.page;
    }
    bool operator==(const PageKey &o) const { return layer == o.layer && page == o.page; }
  };

  // A key as one 64-bit word, for hashing and packed arrays.
  inline std::uint64_t pack(PageKey k)
  {
    return (static_cast<std::uint64_t>(static_cast<std::uint32_t>(k.layer)) << 32) |
           static_cast<std::uint32_t>(k.page);
  }
  inline PageKey unpack(std::uint64_t w)
  {
    return {static_cast<int>(static_cast<std::uint32_t>(w >> 32)),
            static_cast<int>(static_cast<std::uint32_t>(w))};
  }

  std::string describe(PageKey key);

  // Device memory owned by the library: RAII over hipMalloc.
  class DeviceBuffer
  {
  public:
    explicit DeviceBuffer(std::size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    void *raw() const { return ptr_; }
    template <typename T> T *as() const { return static_cast<T *>(ptr_); }
    std::size_t bytes() const { return bytes_; }

  private:
    void *ptr_ = nullptr;
    std::size_t bytes_ = 0;
  };

  // Host data sent to a device buffer on a stream, the buffer grown as
  // needed (a grown buffer's old one is freed after the device is idle).
  class UploadBuffer
  {
  public:
    template <typename T> const T *send(const std::vector<T> &host, hipStream_t stream)
    {
      return static_cast<const T *>(send_bytes(host.data(), host.size() * sizeof(T), stream));
    }
    const void *send_bytes(const void *host, std::size_t bytes, hipStream_t stream);

  private:
    std::unique_ptr<DeviceBuffer> buffer_;
  };

  // Page pairs sent to the device in pieces while the launches of earlier
  // pieces run: a pinned host area and a device area of one capacity, grown
  // only while the stream is idle (a batch's start), each piece written at
  // its own offset, so that no copy waits for the stream and none overwrites
  // what a queued copy still reads.
  class StagedPairs
  {
  public:
    StagedPairs() = default;
    StagedPairs(const StagedPairs &) = delete;
    StagedPairs &operator=(const StagedPairs &) = delete;
    ~StagedPairs();
    void reserve(std::size_t count);
    RefPair *host() const { return host_; }
    // Pairs [first, first + count) of host() to the device; their device copy.
    const RefPair *send(std::size_t first, std::size_t count, hipStream_t stream);

  private:
    RefPair *host_ = nullptr;
    std::unique_ptr<DeviceBuffer> device_;
    std::size_t capacity_ = 0;
  };

  // A workspace of one owner's: a device buffer grown on demand. A buffer it
  // outgrows is kept until the owner goes, so that an address a captured
  // graph holds stays valid as long as the owner does.
  class OwnedWorkspace final : public WorkspaceSource
  {
  public:
    float *floats(std::size_t count) override
    {
      if (current_ == nullptr || current_->bytes() < count * sizeof(float))
      {
        if (current_ != nullptr)
        {
          outgrown_.push_back(std::move(current_));
        }
        current_ = std::make_unique<DeviceBuffer>(std::max<std::size_t>(count, 1 << 16) *
                                                  sizeof(float));
      }
      return current_->as<float>();
    }

  private:
    std::unique_ptr<DeviceBuffer> current_;
    std::vector<std::unique_ptr<DeviceBuffer>> outgrown_;
  };

  // Test hook: the next `n` granule maps fail as if the device were out of
  // memory, so rollback paths are exercised without exhausting real VRAM.
  void fail_next_granules(int n);

  // The granule the allocator maps and releases tier ranges in, on the
  // current device: the driver's recommended granularity, at least 2 MiB.
  std::size_t granule_bytes();

  struct PageLocation
  {
    int tier;
    std::size_t slot;
  };

  // Told of every page whose place changes: a KVPages keeps its device page
  // tables current from these, instead of rebuilding them.
  class PlacementObserver
  {
  public:
    virtual void placed(PageKey key, int tier, std::size_t slot) = 0;
    virtual void removed(PageKey key) = 0;

  protected:
    ~PlacementObserver() = default;
  };

  class GranuleReleaser;

  // The longest run of granules one physical allocation backs (128 MiB at
  // 2 MiB granules): bounds the bytes a split copies, and sets how many
  // unmap calls (~0.2 ms each, whatever a run's length) a shrinking range
  // makes: a 704 MB tail is six.
  constexpr std::size_t kMaxRunGranules = 64;

  // ADR-0007's allocator (reference: paged_kv_cache.h:88-227): one reserved
  // virtual range per tier, pages packed from slot 0 with no holes, physical
  // granules mapped only as far as the packed pages reach and given back as
  // the tail retracts. A free moves the tier's tail page into the hole; a
  // batched free fills the holes below the kept count with the pages above
  // it, in slot order. A page's address is never handed out.
  class PagedKVCache
  {
  public:
    PagedKVCache(const std::array<std::size_t, kTierCount> &page_bytes,
                 const std::array<std::size_t, kTierCount> &capacity_pages);
    ~PagedKVCache();
    PagedKVCache(const PagedKVCache &) = delete;
    PagedKVCache &operator=(const PagedKVCache &) = delete;

    void allocate(PageKey key, int tier);
    // Every key at `tier`, in order, mapping the granules they need once;
    // all or none. Spare granules are taken first; with top_up_spares the
    // spares are mapped again afterwards, as a single allocation does.
    void allocate_run(const std::vector<PageKey> &keys, int tier, bool top_up_spares = true);
    void free(PageKey key);
    void free_pages(const std::vector<PageKey> &keys);
    void replace(PageKey key, PageKey staged);
    void replace_pages(const std::vector<std::pair<PageKey, PageKey>> &pairs);
    // While a sink is set, the compaction copies of frees and replaces are
    // appended to it instead of launched, and the runs a range gives up are
    // held back: the caller launches the copies itself (after the work that
    // reads the freed pages) and then calls finish_deferred, which queues
    // the held runs for release behind what the stream has been given.
    void defer_copies(std::vector<RefPair> *sink) { deferred_copies_ = sink; }
    void finish_deferred();
    void write(PageKey key, const void *host, std::size_t bytes);
    void read(PageKey key, void *host, std::size_t bytes) const;
    PageLocation locate(PageKey key) const;
    bool contains(PageKey key) const { return where_.count(pack(key)) != 0; }
    std::vector<PageKey> pages(int tier) const;
    std::size_t page_bytes(int tier) const { return ranges_.at(tier).page_bytes; }
    // Pages a tier holds: the slot the next allocation there takes.
    std::size_t held(int tier) const { return ranges_.at(tier).owners.size(); }
    std::size_t reserved_bytes(int tier) const { return ranges_.at(tier).reserved; }
    std::size_t mapped_bytes(int tier) const { return ranges_.at(tier).mapped * granule_; }
    void keep_spare_granules(int tier, std::size_t granules);
    std::size_t spare_granules(int tier) const { return ranges_.at(tier).spare; }
    std::size_t granule() const { return granule_; }
    std::uint64_t generation() const { return generation_; }
    // Waits until every granule given up so far is back with the driver
    // (a run the tail cut is settled here).
    void drain_releases();
    // Valid until the next allocator operation: for the cache's own launches.
    char *address(PageKey key, std::size_t bytes) const;
    char *address_of(PageLocation at) const
    {
      const Range &r = ranges_[at.tier];
      return r.base + at.slot * r.page_bytes;
    }
    // The kernels' view of the four ranges (bases and page sizes), and a
    // page's 32-bit reference.
    PageSpaces spaces() const;
    std::uint32_t ref_of(PageKey key) const;
    void watch(PlacementObserver *o) { observers_.push_back(o); }
    void unwatch(PlacementObserver *o);

  private:
    // Granules [first, first + count) of a range backed by one physical
    // allocation, mapped by one call: the driver's unmap costs the same for
    // a run of any length, so a range given back in runs costs a call a run,
    // not a call a granule.
    struct Run
    {
      std::size_t first;
      std::size_t count;
      hipMemGenericAllocationHandle_t handle;
    };
    struct Range
    {
      char *reservation = nullptr; // a guard granule, never mapped, then the range
      char *base = nullptr;
      std::size_t reserved = 0;
      std::size_t page_bytes = 0;
      std::size_t capacity = 0;
      std::vector<std::uint64_t> owners; // slot -> packed key
      std::vector<Run> runs;             // in address order, from granule 0
      // Granules the range counts as mapped. The last run may reach past
      // them: a run the tail cut, whose granules past `mapped` are given
      // back when the cut is settled (or counted back by the next growth).
      std::size_t mapped = 0;
      std::size_t spare = 0;
      std::size_t runs_end() const { return runs.empty() ? 0 : runs.back().first + runs.back().count; }
    };
    static void check_tier(int tier);
    // The location word kept per key: tier in the top byte, slot below.
    static std::uint64_t loc_word(int tier, std::size_t slot)
    {
      return (static_cast<std::uint64_t>(tier) << 56) | slot;
    }
    static PageLocation loc_of(std::uint64_t w)
    {
      return {static_cast<int>(w >> 56), static_cast<std::size_t>(w & ((1ull << 56) - 1))};
    }
    void release_keys(const std::vector<PageKey> &keys);
    void fit(Range &r, bool map_spares);
    // Maps granules at the range's end until it has `count`, in runs of at
    // most kMaxRunGranules; all or none.
    void map_to(Range &r, std::size_t count);
    // Gives back the granules from `keep` on: whole runs to the releaser; a
    // run that `keep` cuts stays whole until the cut is settled, its
    // granules past `keep` no longer counted.
    void retract(Range &r, std::size_t keep);
    // Settles every range's cut: the run is replaced by a shorter one
    // holding the same bytes (copied out to a device buffer and back), so
    // that exactly the counted granules stay mapped. Synchronises the
    // device first; a range whose shorter run cannot be made stays cut.
    void settle_cuts();
    void split_run(Range &r, std::size_t keep);
    hipMemGenericAllocationHandle_t create_physical(std::size_t granules);
    // Grants read and write over the range's first `granules` granules, and
    // checks that granules [from, granules) have it.
    void grant_access(Range &r, std::size_t from, std::size_t granules);
    std::unique_ptr<DeviceBuffer> split_buffer_; // a run's kept bytes during a split
    void tell_placed(std::uint64_t key, int tier, std::size_t slot);
    void tell_removed(std::uint64_t key);

    std::uint64_t generation_ = 0;
    int device_ = 0;
    hipMemAllocationProp prop_{};
    std::size_t granule_ = 0;
    std::array<Range, kTierCount> ranges_;
    std::unordered_map<std::uint64_t, std::uint64_t> where_; // packed key -> loc word
    std::vector<PlacementObserver *> observers_;
    std::unique_ptr<GranuleReleaser> releaser_;
    UploadBuffer moves_upload_;
    std::vector<RefPair> *deferred_copies_ = nullptr;
    struct HeldRun
    {
      char *at;
      std::size_t bytes;
      hipMemGenericAllocationHandle_t handle;
    };
    std::vector<HeldRun> deferred_runs_;
  };

  // FP16 shadows of downgraded pages in pinned host memory mapped for the
  // device (reference: shadow_store.h:11-86): packed into pinned blocks of
  // about 2 MiB, or of any size pinned ahead (reserve), numbered in the
  // order they are taken. A device table gives each number's mapped address,
  // so kernels read and write shadows by number. Only ever added; freed with
  // the store.
  class ShadowStore
  {
  public:
    static constexpr std::size_t kAllocationBytes = std::size_t{2} << 20;
    explicit ShadowStore(std::size_t page_bytes);
    ~ShadowStore();
    ShadowStore(const ShadowStore &) = delete;
    ShadowStore &operator=(const ShadowStore &) = delete;

    // One device page copied into a new shadow (synchronously).
    void take(PageKey key, const void *device_page, hipStream_t stream);
    // Pinned room for `count` more shadows, made now.
    void reserve(std::size_t count);
    // A new shadow's number, its room pinned already or now.
    std::uint32_t add(PageKey key);
    // Forgets the shadows numbered `count` and above (the last added), as
    // if they had not been: a batch that fails after taking them.
    void truncate(std::size_t count);
    bool contains(PageKey key) const { return number_.count(pack(key)) != 0; }
    std::uint32_t number(PageKey key) const;
    // Shadow `number`'s mapped address (what the device table holds for it).
    unsigned long long device_address(std::uint32_t number) const { return device_[number]; }
    const std::uint8_t *shadow(PageKey key) const;
    std::size_t page_bytes() const { return page_bytes_; }
    std::size_t count() const { return host_.size(); }
    std::size_t bytes() const { return pinned_pages_ * page_bytes_; }
    // The device table of every shadow's mapped address, current on `stream`.
    const unsigned long long *device_table(hipStream_t stream);

  private:
    struct Block
    {
      std::uint8_t *host;
      std::uint8_t *device;
      std::size_t pages;
      std::size_t used;
    };
    std::size_t page_bytes_;
    std::vector<Block> blocks_;
    std::size_t pinned_pages_ = 0;
    std::size_t cursor_ = 0; // the first block with room
    std::unordered_map<std::uint64_t, std::uint32_t> number_;
    std::vector<std::uint8_t *> host_;       // by number
    std::vector<unsigned long long> device_; // by number
    std::vector<std::uint64_t> keys_;        // by number
    std::vector<std::size_t> block_of_;      // by number
    std::size_t sent_ = 0;                   // entries already in the device table
    std::unique_ptr<DeviceBuffer> table_;
    std::vector<std::unique_ptr<DeviceBuffer>> outgrown_;
  };

  // The per-(layer, page) EWMA of attention mass (reference:
  // importance_scores.h:11-66), on the device, NaN where never observed.
  class ImportanceScores
  {
  public:
    static constexpr float kDefaultAlpha = 0.2f;
    ImportanceScores(int layers, int max_pages, float alpha);
    void fold(int layer, const float *mass, int heads, int pages, hipStream_t stream);
    std::vector<float> download();
    void upload(const float *host, int layers, int max_pages);
    float *layer_scores(int layer) const;
    int layers() const { return layers_; }
    int max_pages() const { return max_pages_; }
    float alpha() const { return alpha_; }
    std::size_t downloads() const { return downloads_; }
    std::size_t nbytes() const { return static_cast<std::size_t>(layers_) * max_pages_ * 4; }

  private:
    int layers_;
    int max_pages_;
    float alpha_;
    std::unique_ptr<DeviceBuffer> scores_;
    std::size_t downloads_ = 0;
  };

  // {cos, sin} of every RoPE angle per position, fp32, formed in fp64
  // (reference: rope_table.h:11-44); grows by doubling.
  class RopeTable
  {
  public:
    RopeTable(int head_dim, double theta);
    void cover(int count);
    const float *data() const { return table_ ? table_->as<const float>() : nullptr; }
    // The angles of the first kAngleRows positions (a decode page's rows)
    // as fp16 high and low parts, for the decode kernel's key bias:
    // [position][hi | lo][head_dim], cos then sin. The table always covers
    // that many positions.
    static constexpr int kAngleRows = 32;
    const std::uint16_t *angles() const
    {
      return angles_ ? angles_->as<const std::uint16_t>() : nullptr;
    }
    int positions() const { return positions_; }
    int head_dim() const { return head_dim_; }
    double theta() const { return theta_; }
    std::size_t nbytes() const { return static_cast<std::size_t>(positions_) * head_dim_ * 4; }

  private:
    int head_dim_;
    double theta_;
    int positions_ = 0;
    std::unique_ptr<DeviceBuffer> table_;
    std::unique_ptr<DeviceBuffer> angles_;
  };

  // The page_index of a layer's two open pages, of a move's staging page, of
  // the shadow upload page, and the base of a batch's staging pages
  // (reference: kv_pages.h:32-48).
  constexpr int kOpenPages[2] = {-1, -2};
  constexpr int kStagingPage = -3;
  constexpr int kShadowUploadPage = -4;
  constexpr int kBatchStagingPage = -16;

  enum class Halves : int
  {
    kBoth = 0,
    kKeys = 1,
    kValues = 2,
  };

  using TierMap = std::vector<std::vector<int>>;

  struct PageMove
  {
    PageKey key;
    int target;
  };

  struct MoveRecord
  {
    PageKey key;
    int from_tier;
    int to_tier;
    std::size_t from_bytes;
    std::size_t to_bytes;
    double seconds;
    double shadow_seconds;
  };

  struct BatchRecord
  {
    std::size_t moves;
    std::size_t shadows_taken;
    double seconds;
    // Where the seconds went: the host's work before the first launch; the
    // new pages' allocation (while the shadows travel); the page table's
    // switch to the new pages, the old ones' release and the wait for the
    // device.
    double prepare_seconds;
    double allocate_seconds;
    double finish_seconds;
  };

  // Every layer's page addresses and tiers on the device, [layer][stride]
  // each, with a host copy. Entries change one at a time as the allocator
  // reports pages moving; commit() sends the changed entries (or the whole
  // table, if that is less) before the next launch that reads it.
  class PageTable
  {
  public:
    explicit PageTable(int layers) : layers_(layers) {}
    int stride() const { return stride_; }
    // Room for `pages` a layer; a new stride starts every entry unread.
    void ensure(int pages);
    void set(int layer, int page, unsigned long long address, std::uint8_t tier);
    void commit(hipStream_t stream);
    const unsigned long long *addresses() const
    {
      return device_ ? device_->as<const unsigned long long>() : nullptr;
    }
    const std::uint8_t *tiers() const
    {
      return device_ ? reinterpret_cast<const std::uint8_t *>(
                           device_->as<const unsigned long long>() + entries())
                     : nullptr;
    }

  private:
    std::size_t entries() const { return static_cast<std::size_t>(layers_) * stride_; }
    int layers_;
    int stride_ = 0;
    std::vector<unsigned long long> address_;
    std::vector<std::uint8_t> tier_;
    std::vector<std::uint8_t> dirty_;    // an entry changed since the last commit
    std::vector<std::uint32_t> marked_;  // those entries, once each
    bool whole_ = false;
    std::unique_ptr<DeviceBuffer> device_;
    UploadBuffer edit_upload_;
  };

  // The engine's KV cache on pages (reference: kv_pages.h:66-412).
  class KVPages final : private PlacementObserver
  {
  public:
    static bool seals_for(int tier, const TierMap &tier_map, bool always_seal);

    KVPages(PagedKVCache &allocator, int layers, int page_tokens, int kv_heads, int head_dim,
            int tier, Halves halves, TierMap tier_map, bool always_seal);
    ~KVPages();
    KVPages(const KVPages &) = delete;
    KVPages &operator=(const KVPages &) = delete;

    void reserve(int tokens);
    void store(int layer, const void *keys, const void *values, int start, int n);
    void attention(int layer, const void *q, const void *k_bias, const RopeTable *rope, void *out,
                   int seq_q, int seq_k, int heads, int kv_heads, int head_dim, const void *keys,
                   const void *values, float *mass, float *scores, float alpha, float *partials);
    // One decode step of `layers` consecutive layers in one launch: layer
    // first_layer + i reads its q, chunk rows and writes its output, mass and
    // scores at i times the strides (elements) from the bases; always split.
    void attention_layers(int first_layer, int layers, const void *q, long long q_stride,
                          void *out, long long out_stride, int seq_k, int heads, int kv_heads,
                          int head_dim, const void *keys, const void *values,
                          long long kv_stride, float *mass, long long mass_stride,
                          float *scores, long long scores_stride, float alpha);
    // Beyond the reference: a decode step whose per-page mass is folded once
    // for every layer instead of once a layer. attention_kept is one layer's
    // decode (one query a head) keeping its page statistics; fold_kept then
    // forms every layer's page masses and folds them into the scores in one
    // launch, to the bits attention(..., mass, scores) gives a layer at a
    // time. Every layer is attended, at one seq_k, between two folds.
    void attention_kept(int layer, const void *q, const void *k_bias, const RopeTable *rope,
                        void *out, int seq_k, int heads, int kv_heads, int head_dim,
                        const void *keys, const void *values);
    void fold_kept(float *mass, long long mass_stride, float *scores, long long scores_stride,
                   float alpha);
    // Beyond the reference: the pieces of a decode step whose position lives
    // on the device, so that one captured graph serves every step of a run.
    // store_step stores one row at *position (sealing the page it
    // completes); attention_step decodes one layer at seq_k = *live_seq_k,
    // its launch sized for max_seq_k, keeping its statistics in `keep` (a
    // DecodeFold's layout for every layer at max_seq_k) when keep is not
    // null; fold_step folds the kept statistics into the scores where seq_k
    // is a multiple of score_every. prepare_step readies the tables and
    // scratch for max_seq_k beforehand, so that the launches allocate and
    // upload nothing; the pages up to max_seq_k must be reserved, and no
    // page may move, while they run. stored_on_device(end) then records that
    // the positions before `end` were stored.
    void prepare_step(int max_seq_k, int heads, int head_dim);
    void store_step(int layer, const void *keys, const void *values, const int *position);
    // For a cache that does not seal (FP16 pages throughout): one decode
    // row's RoPE (qk: q_heads then kv_heads rows of head_dim fp16, rotated
    // into qk_out at *position with `rope`'s angles) and its store at that
    // position (the rotated k heads and `values`), with the RMSNorm of an
    // independent fp32 row (x, when not null) in the same launch: the bits
    // of launch_rmsnorm, launch_rope_rows and store for that row. The
    // position must be reserved and covered by the table.
    void rope_store(int layer, const void *qk, void *qk_out, int q_heads, const int *position,
                    const RopeTable &rope, const void *values, const float *x,
                    const void *norm_weight, void *normed, int hidden, float eps);
    // For a cache that does not seal: rope_store at position seq_k - 1 and
    // attention's one-query decode over the positions before seq_k, as the
    // pages launch and its combine (the pages launch turns q and the row's
    // k, stores the row in its page and forms the RMSNorm when x is given):
    // the bits of rope_store then attention given partials (split).
    void attend_row(int layer, const void *qk, void *qk_out, int q_heads, int seq_k,
                    const RopeTable &rope, const void *values, void *out, const float *x,
                    const void *norm_weight, void *normed, int hidden, float eps);
    // The layer's store target for a step whose projection writes its row
    // (launch_qkv_step): the open page (the step's row goes there unless it
    // is the page's last) and the page table row for the seal; `keys` and
    // `values` are where the step's k and v rows are, which the seal reads
    // for the last row. The store is recorded by stored_on_device as any
    // store_step's.
    StepStore step_store(int layer, const void *keys, const void *values, const int *position);
    // With `seal` (step_store's target), the combine's extra workgroup seals
    // the step's page when its position is the page's last row.
    void attention_step(int layer, const void *q, const void *k_bias, const RopeTable *rope,
                        void *out, const int *live_seq_k, int max_seq_k, int heads,
                        int kv_heads, int head_dim, const void *keys, const void *values,
                        float *keep, const StepStore *seal = nullptr);
    void fold_step(float *keep, const int *live_seq_k, int max_seq_k, int heads, int kv_heads,
                   int head_dim, int score_every, float *scores, long long scores_stride,
                   float alpha);
    void stored_on_device(int end);
    void downgrade(int layer, int page, int target);
    void upgrade(int layer, int page, int target);
    void move_pages(const std::vector<PageMove> &moves);
    void evict(int layer, int page);
    void mask(int layer, int page);
    // Pins host memory for `pages` more FP16 shadows now, so that first
    // downgrades later take none of their time pinning (ADR-0015's "pinning
    // ahead of need"). No counterpart in the reference.
    void pin_shadows(std::size_t pages) { shadows_.reserve(pages); }

    bool evicted(PageKey key) const { return flag(key, kEvicted); }
    bool masked(PageKey key) const { return flag(key, kMasked); }
    int page_tier(PageKey key) const { return allocator_.locate(key).tier; }
    const ShadowStore &shadows() const { return shadows_; }
    const std::optional<MoveRecord> &last_move() const { return last_move_; }
    const std::optional<BatchRecord> &last_batch() const { return last_batch_; }
    int page_tokens() const { return page_tokens_; }
    int pages_per_layer() const { return pages_; }
    int layers() const { return layers_; }
    int capacity_tokens() const { return (pages_ + (seals_ ? 1 : 0)) * page_tokens_; }
    std::size_t page_bytes() const { return page_bytes_; }
    int tier() const { return tier_; }
    Halves halves() const { return halves_; }
    bool seals() const { return seals_; }
    bool born_at_one_tier() const { return !mixed_; }
    int storage_tier() const { return storage_tier_; }
    int birth_tier(int layer, int page) const;
    std::size_t kv_width() const { return kv_width_; }
    int kv_heads() const { return kv_heads_; }
    int head_dim() const { return head_dim_; }

  private:
    static constexpr std::uint8_t kEvicted = 1;
    static constexpr std::uint8_t kMasked = 2;

    // PlacementObserver: the allocator moved or dropped one of its pages.
    void placed(PageKey key, int tier, std::size_t slot) override;
    void removed(PageKey key) override;

    bool flag(PageKey key, std::uint8_t bit) const
    {
      if (key.layer < 0 || key.layer >= layers_ || key.page < 0 || key.page >= pages_)
      {
        return false;
      }
      return (flags_[static_cast<std::size_t>(key.layer) * flag_stride_ + key.page] & bit) != 0;
    }
    void set_flag(PageKey key, std::uint8_t bit);
    void grow(int pages); // flags and table room for `pages` a layer
    void refresh_entry(int layer, int page);
    void sync_tables(hipStream_t stream);

    void store_sealed(int layer, const std::uint16_t *keys, const std::uint16_t *values, int start,
                      int n);
    PageKey require_movable(int layer, int page, const char *verb) const;
    PageKey require_held(int layer, int page, const char *verb) const;
    // The tier moves of a batch: validated already, every page held.
    void run_moves(const std::vector<PageKey> &keys, const std::vector<int> &from,
                   const std::vector<int> &targets, double *shadow_seconds);
    // One page's move as one launch (launch_move_one), where its shape
    // allows: false, and nothing changed, where it does not.
    bool run_one_move(PageKey key, int from, int target, double *shadow_seconds);
    // Two timing events around a single move's copies, made on first use.
    void ensure_move_events();
    hipEvent_t move_events_[2] = {nullptr, nullptr};
    double phases_[3] = {0.0, 0.0, 0.0}; // the last run_moves': prepare, allocate, finish
    void require_layer(int layer) const;
    std::size_t bytes_at(int tier) const;
    void require_page_size(int tier, const char *what) const;
    std::uint16_t *open_page(int layer, int which) const
    {
      return reinterpret_cast<std::uint16_t *>(open_address_[2 * layer + which]);
    }
    // Every layer's open page as the next attention reads it, on the device.
    const unsigned long long *open_table(hipStream_t stream);
    static std::string page_name(PageKey key);

    PagedKVCache &allocator_;
    int layers_;
    int page_tokens_;
    int kv_heads_;
    int head_dim_;
    std::size_t kv_width_;
    int tier_;
    Halves halves_;
    int storage_tier_;
    TierMap tier_map_;
    std::array<bool, kTierCount> may_be_at_{};
    bool seals_ = false;
    bool mixed_ = false;
    std::size_t page_bytes_;
    int pages_ = 0;
    bool open_pages_ = false;
    std::vector<int> current_open_;
    std::vector<int> attend_open_;
    std::vector<int> sealed_;
    std::vector<unsigned long long> open_address_; // [layer][2]
    std::vector<std::uint8_t> flags_;              // [layer][flag_stride_]
    int flag_stride_ = 0;
    ShadowStore shadows_;
    std::optional<MoveRecord> last_move_;
    std::optional<BatchRecord> last_batch_;
    PageTable table_;
    std::unique_ptr<DeviceBuffer> open_table_;
    std::vector<unsigned long long> open_uploaded_;
    UploadBuffer pairs_upload_;
    StagedPairs shadow_pairs_; // a batch's first-downgrade shadows, sent as validated
    // FP16 pages brought from their shadows to device memory before they are
    // quantised (read once over the host link, then twice from HBM).
    std::unique_ptr<DeviceBuffer> staging_;
    // The decode path's split partials and page statistics: this cache's own.
    OwnedWorkspace workspace_;
    // Page statistics kept for fold_kept, every layer's (decode_kept_floats
    // a layer), and the step they belong to.
    OwnedWorkspace kept_;
    std::vector<char> kept_layers_;
    int kept_seq_k_ = -1;
    int kept_heads_ = 0;
    int kept_kv_heads_ = 0;
    int kept_head_dim_ = 0;
  };

  // The stream every launch of the runtime goes on, per host thread: the
  // null stream unless set, as it must be to capture a graph.
  hipStream_t runtime_stream();
  void set_runtime_stream(hipStream_t stream);

} // namespace mi
