// The cache runtime on the host: the per-tier VMM page allocator, the pinned
// FP16 shadow store, the importance scores, the RoPE table, and KVPages, the
// cache manager that seals, attends, and moves pages between tiers.
//
// Semantics follow the reference's classes of the same names
// (src/core_kernels/paged_kv_cache.{h,cu}, shadow_store.{h,cu},
// importance_scores.{h,cu}, rope_table.{h,cu}, kv_pages.{h,cu}); the device
// side is HIP on one MI355X, every launch on one stream.
#pragma once

#include "common.hpp"
#include "kernels.hpp"

#include <array>
#include <condition_variable>
#include <deque>
#include <map>
#include <memory>
#include <mutex>
#include <optional>
#include <set>
#include <thread>
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

  // Test hook: the next `n` granule maps fail as if the device were out of
  // memory, so rollback paths are exercised without exhausting real VRAM.
  void fail_next_granules(int n);

  // The driver's allocation granularity for device memory on the current
  // device: never assumed.
  std::size_t granule_bytes();

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

  struct PageLocation
  {
    int tier;
    std::size_t slot;
  };

  // ADR-0007's allocator (reference: paged_kv_cache.h:88-227): one reserved
  // virtual range per tier, pages packed from slot 0 with no holes, physical
  // granules mapped only as far as the packed pages reach and unmapped and
  // released as the tail retracts. Freeing a page moves its tier's tail page
  // into the vacated slot. A page's address is never handed out.
  class PagedKVCache
  {
  public:
    PagedKVCache(const std::array<std::size_t, kTierCount> &page_bytes,
                 const std::array<std::size_t, kTierCount> &capacity_pages);
    ~PagedKVCache();
    PagedKVCache(const PagedKVCache &) = delete;
    PagedKVCache &operator=(const PagedKVCache &) = delete;

    void allocate(PageKey key, int tier);
    void free(PageKey key);
    void free_pages(const std::vector<PageKey> &keys);
    void replace(PageKey key, PageKey staged);
    void replace_pages(const std::vector<std::pair<PageKey, PageKey>> &pairs);
    void write(PageKey key, const void *host, std::size_t bytes);
    void read(PageKey key, void *host, std::size_t bytes) const;
    PageLocation locate(PageKey key) const;
    bool contains(PageKey key) const { return table_.count(key) != 0; }
    const std::vector<PageKey> &pages(int tier) const { return ranges_.at(tier).slots; }
    std::size_t page_bytes(int tier) const { return ranges_.at(tier).page_bytes; }
    std::size_t reserved_bytes(int tier) const { return ranges_.at(tier).reserved; }
    std::size_t mapped_bytes(int tier) const { return ranges_.at(tier).granules.size() * granule_; }
    void keep_spare_granules(int tier, std::size_t granules);
    std::size_t spare_granules(int tier) const { return ranges_.at(tier).spare; }
    std::size_t granule() const { return granule_; }
    std::uint64_t generation() const { return generation_; }
    // Waits until every granule given up so far is back with the driver.
    void drain_releases();
    // Valid until the next allocator operation: for the cache's own launches.
    char *address(PageKey key, std::size_t bytes) const;

  private:
    struct Range
    {
      char *base = nullptr;
      std::size_t reserved = 0;
      std::size_t page_bytes = 0;
      std::size_t capacity = 0;
      std::vector<PageKey> slots;
      std::vector<hipMemGenericAllocationHandle_t> granules;
      std::size_t spare = 0;
    };
    // A granule given up by a range: unmapped and released by the release
    // thread, off the caller's path (each unmap costs the driver a fraction
    // of a millisecond, and a batch can give up hundreds).
    struct Retired
    {
      char *at;
      hipMemGenericAllocationHandle_t handle;
    };
    static void check_tier(int tier);
    void fit_granules(Range &r, bool map_spares);
    void map_granule(Range &r);
    void roll_back(Range &r);
    void release_everything() noexcept;
    void retire(char *at, hipMemGenericAllocationHandle_t handle);
    void wait_for_release(const char *at);
    void release_loop();

    std::uint64_t generation_ = 0;
    int device_ = 0;
    hipMemAllocationProp prop_{};
    std::size_t granule_ = 0;
    std::array<Range, kTierCount> ranges_;
    std::map<PageKey, PageLocation> table_;
    std::mutex release_mutex_;
    std::condition_variable release_wake_; // the release thread: work or stop
    std::condition_variable release_done_; // waiters: a granule was released
    std::deque<Retired> retired_;          // oldest first
    const char *releasing_ = nullptr;      // the granule the thread is releasing
    bool release_stop_ = false;
    std::string release_error_;            // the first failure, raised to the next waiter
    std::thread releaser_;
  };

  // FP16 shadows of downgraded pages in pinned host memory mapped for the
  // device, packed into allocations of about 2 MiB (reference:
  // shadow_store.h:11-86). Only ever added; freed with the store.
  class ShadowStore
  {
  public:
    static constexpr std::size_t kAllocationBytes = std::size_t{2} << 20;
    explicit ShadowStore(std::size_t page_bytes);
    ~ShadowStore();
    ShadowStore(const ShadowStore &) = delete;
    ShadowStore &operator=(const ShadowStore &) = delete;

    void take(PageKey key, const void *device_page, hipStream_t stream);
    void reserve(std::size_t count);
    std::uint8_t *add(PageKey key);           // device address to write the shadow at
    bool contains(PageKey key) const { return shadows_.count(key) != 0; }
    const std::uint8_t *shadow(PageKey key) const;
    const std::uint8_t *device_shadow(PageKey key) const;
    std::size_t page_bytes() const { return page_bytes_; }
    std::size_t count() const { return shadows_.size(); }
    std::size_t bytes() const { return capacity_ * page_bytes_; }

  private:
    struct Allocation
    {
      std::uint8_t *host;
      std::uint8_t *device;
      std::size_t pages;
      std::size_t used;
    };
    std::size_t page_bytes_;
    std::size_t per_allocation_;
    std::vector<Allocation> allocations_;
    std::size_t capacity_ = 0;
    std::map<const std::uint8_t *, std::size_t> by_address_;
    std::map<PageKey, std::uint8_t *> shadows_;
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
  };

  // The engine's KV cache on pages (reference: kv_pages.h:66-412).
  class KVPages
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
    void downgrade(int layer, int page, int target);
    void upgrade(int layer, int page, int target);
    void move_pages(const std::vector<PageMove> &moves);
    void evict(int layer, int page);
    void mask(int layer, int page);

    bool evicted(PageKey key) const { return evicted_.count(key) != 0; }
    bool masked(PageKey key) const { return masked_.count(key) != 0; }
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

    // The device table of one layer, resolved now: page addresses, then tiers.
    struct LayerTable
    {
      const unsigned long long *pages;
      const std::uint8_t *tiers;
    };
    LayerTable resolve(int layer);

  private:
    struct Seal
    {
      int span;
      const std::uint16_t *keys;
      const std::uint16_t *values;
    };
    void seal_batch(int layer, const std::vector<Seal> &seals);
    void store_sealed(int layer, const std::uint16_t *keys, const std::uint16_t *values, int start,
                      int n);
    PageKey require_movable(int layer, int page, const char *verb) const;
    PageKey require_held(int layer, int page, const char *verb) const;
    void move(PageKey key, int current, int target);
    void require_layer(int layer) const;
    std::size_t bytes_at(int tier) const;
    void require_page_size(int tier, const char *what) const;
    std::uint16_t *open_page(int layer, int which);
    // Every layer's open page as the next attention reads it, on the device.
    const unsigned long long *open_table();
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
    ShadowStore shadows_;
    std::set<PageKey> evicted_;
    std::set<PageKey> masked_;
    std::optional<MoveRecord> last_move_;
    std::optional<BatchRecord> last_batch_;
    std::unique_ptr<DeviceBuffer> scratch_page_;
    std::unique_ptr<DeviceBuffer> scratch_halves_;
    std::unique_ptr<DeviceBuffer> tables_;
    int table_stride_ = 0;
    int resolved_pages_ = -1;
    std::uint64_t resolved_generation_ = 0;
    std::unique_ptr<DeviceBuffer> open_table_;
    std::vector<unsigned long long> open_uploaded_;
    // Address tables for batched launches, grown as needed.
    std::unique_ptr<DeviceBuffer> batch_table_;
    // The decode path's split partials and page statistics: this cache's own.
    OwnedWorkspace workspace_;
  };

  // The stream every launch of the runtime goes on, per host thread: the
  // null stream unless set, as it must be to capture a graph.
  hipStream_t runtime_stream();
  void set_runtime_stream(hipStream_t stream);

} // namespace mi
