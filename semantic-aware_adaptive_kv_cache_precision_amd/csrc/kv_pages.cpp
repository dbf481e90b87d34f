// KVPages, the cache manager, with its shadow store, importance scores and
// RoPE table.
//
// Semantics follow the reference's src/core_kernels/kv_pages.cu (reserve
// :219-264, resolve :287-352, store/seal :360-475, evict/mask :522-543,
// downgrade/upgrade/move :551-711, move_pages :713-899, attention :901-947),
// shadow_store.cu, importance_scores.cu and rope_table.cu. What differs is
// how the device is driven: a store that seals many pages (a prefill chunk,
// or building a cache) quantises them in one launch per tier and copies FP16
// ones in one batched copy, instead of a launch pair per page; and every
// launch goes on the runtime stream.

#include "runtime.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>

namespace mi
{
  namespace
  {
    using Clock = std::chrono::steady_clock;

    double since(Clock::time_point t)
    {
      return std::chrono::duration<double>(Clock::now() - t).count();
    }

    // Uploads a host table of addresses into `buffer`, growing it as needed.
    const void *const *upload_table(std::unique_ptr<DeviceBuffer> &buffer,
                                    const std::vector<const void *> &table)
    {
      const std::size_t bytes = table.size() * sizeof(void *);
      if (bytes == 0)
      {
        return nullptr;
      }
      if (!buffer || buffer->bytes() < bytes)
      {
        buffer.reset(); // waits for launches that may read the old one
        buffer = std::make_unique<DeviceBuffer>(std::max<std::size_t>(bytes, 4096));
      }
      // Ordered after every launch already enqueued on the runtime stream,
      // which may still read the previous table.
      hip_check(hipMemcpy(buffer->raw(), table.data(), bytes, hipMemcpyHostToDevice),
                "hipMemcpy a batch's page addresses");
      return buffer->as<const void *const>();
    }
  } // namespace

  // ---- ShadowStore ------------------------------------------------------------

  ShadowStore::ShadowStore(std::size_t page_bytes)
      : page_bytes_(page_bytes),
        per_allocation_(page_bytes == 0 || page_bytes >= kAllocationBytes
                            ? 1
                            : kAllocationBytes / page_bytes)
  {
  }

  ShadowStore::~ShadowStore()
  {
    for (const Allocation &a : allocations_)
    {
      (void)hipHostFree(a.host);
    }
  }

  void ShadowStore::take(PageKey key, const void *device_page, hipStream_t stream)
  {
    std::uint8_t *to = add(key);
    (void)to;
    std::uint8_t *host = shadows_.at(key);
    hip_check(hipMemcpyAsync(host, device_page, page_bytes_, hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync a page to its FP16 shadow");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize after a shadow copy");
  }

  void ShadowStore::reserve(std::size_t count)
  {
    const std::size_t room =
        allocations_.empty() ? 0 : allocations_.back().pages - allocations_.back().used;
    if (count <= room)
    {
      return;
    }
    const std::size_t pages = std::max(count, per_allocation_);
    void *host = nullptr;
    hip_check(hipHostMalloc(&host, pages * page_bytes_, hipHostMallocMapped),
              "hipHostMalloc pinned memory for FP16 shadows");
    void *on_device = nullptr;
    const hipError_t mapped = hipHostGetDevicePointer(&on_device, host, 0);
    if (mapped != hipSuccess)
    {
      (void)hipHostFree(host);
      hip_check(mapped, "hipHostGetDevicePointer for FP16 shadows");
    }
    by_address_[static_cast<std::uint8_t *>(host)] = allocations_.size();
    allocations_.push_back({static_cast<std::uint8_t *>(host),
                            static_cast<std::uint8_t *>(on_device), pages, 0});
    capacity_ += pages;
  }

  std::uint8_t *ShadowStore::add(PageKey key)
  {
    if (contains(key))
    {
      throw LogicError("page " + std::to_string(key.page) + " of layer " +
                       std::to_string(key.layer) + " has a shadow already; a page has one");
    }
    reserve(1);
    Allocation &a = allocations_.back();
    const std::size_t slot = a.used++;
    shadows_[key] = a.host + slot * page_bytes_;
    return a.device + slot * page_bytes_;
  }

  const std::uint8_t *ShadowStore::shadow(PageKey key) const
  {
    const auto it = shadows_.find(key);
    if (it == shadows_.end())
    {
      throw PageNotFound(describe(key) + " has no FP16 shadow");
    }
    return it->second;
  }

  const std::uint8_t *ShadowStore::device_shadow(PageKey key) const
  {
    const std::uint8_t *host = shadow(key);
    const Allocation &a = allocations_[std::prev(by_address_.upper_bound(host))->second];
    return a.device + (host - a.host);
  }

  // ---- ImportanceScores -----------------------------------------------------------

  ImportanceScores::ImportanceScores(int layers, int max_pages, float alpha)
      : layers_(layers), max_pages_(max_pages), alpha_(alpha)
  {
    if (layers <= 0 || max_pages <= 0)
    {
      throw InvalidArgument("layers and max_pages must be positive");
    }
    if (!(alpha > 0.0f && alpha <= 1.0f))
    {
      throw InvalidArgument("alpha, the newest observation's weight, is in (0, 1]; got " +
                            std::to_string(alpha));
    }
    const std::size_t count = static_cast<std::size_t>(layers) * max_pages;
    scores_ = std::make_unique<DeviceBuffer>(count * sizeof(float));
    launch_fill(scores_->as<float>(), count, NAN, runtime_stream());
  }

  float *ImportanceScores::layer_scores(int layer) const
  {
    if (layer < 0 || layer >= layers_)
    {
      throw OutOfRange("layer " + std::to_string(layer) + " of " + std::to_string(layers_));
    }
    return scores_->as<float>() + static_cast<std::size_t>(layer) * max_pages_;
  }

  void ImportanceScores::fold(int layer, const float *mass, int heads, int pages,
                              hipStream_t stream)
  {
    float *row = layer_scores(layer);
    if (pages < 0 || pages > max_pages_ || heads <= 0)
    {
      throw InvalidArgument(std::to_string(pages) + " pages of " + std::to_string(heads) +
                            " heads; the scores hold up to " + std::to_string(max_pages_) +
                            " pages, and a mass has a head at least");
    }
    launch_fold(row, mass, heads, pages, alpha_, stream);
  }

  std::vector<float> ImportanceScores::download()
  {
    std::vector<float> host(static_cast<std::size_t>(layers_) * max_pages_);
    hip_check(hipMemcpy(host.data(), scores_->raw(), host.size() * sizeof(float),
                        hipMemcpyDeviceToHost),
              "hipMemcpy importance scores device-to-host");
    ++downloads_;
    return host;
  }

  void ImportanceScores::upload(const float *host, int layers, int max_pages)
  {
    if (layers != layers_ || max_pages != max_pages_)
    {
      throw InvalidArgument("scores to put back are (layers, max_pages), (" +
                            std::to_string(layers_) + ", " + std::to_string(max_pages_) +
                            "); got (" + std::to_string(layers) + ", " +
                            std::to_string(max_pages) + ")");
    }
    hip_check(hipMemcpy(scores_->raw(), host, nbytes(), hipMemcpyHostToDevice),
              "hipMemcpy importance scores host-to-device");
  }

  // ---- RopeTable --------------------------------------------------------------------

  RopeTable::RopeTable(int head_dim, double theta) : head_dim_(head_dim), theta_(theta)
  {
    if (head_dim <= 0 || head_dim % 2 != 0)
    {
      throw InvalidArgument("head_dim must be positive and even, got " + std::to_string(head_dim));
    }
    if (!(theta > 0.0))
    {
      throw InvalidArgument("theta must be positive, got " + std::to_string(theta));
    }
  }

  void RopeTable::cover(int count)
  {
    if (count <= positions_)
    {
      return;
    }
    const int grown = std::max({count, 2 * positions_, kAngleRows});
    auto table = std::make_unique<DeviceBuffer>(static_cast<std::size_t>(grown) * head_dim_ *
                                                sizeof(float));
    launch_rope_table(table->as<float>(), grown, head_dim_, theta_, runtime_stream());
    auto angles = std::make_unique<DeviceBuffer>(static_cast<std::size_t>(kAngleRows) * head_dim_ *
                                                 2 * sizeof(std::uint16_t));
    launch_rope_angles(table->as<const float>(), angles->as<std::uint16_t>(), kAngleRows,
                       head_dim_, runtime_stream());
    table_ = std::move(table);
    angles_ = std::move(angles);
    positions_ = grown;
  }

  // ---- KVPages ------------------------------------------------------------------------

  bool KVPages::seals_for(int tier, const TierMap &tier_map, bool always_seal)
  {
    if (always_seal || tier != kFP16)
    {
      return true;
    }
    for (const auto &row : tier_map)
    {
      for (int t : row)
      {
        if (t != tier)
        {
          return true;
        }
      }
    }
    return false;
  }

  KVPages::KVPages(PagedKVCache &allocator, int layers, int page_tokens, int kv_heads,
                   int head_dim, int tier, Halves halves, TierMap tier_map, bool always_seal)
      : allocator_(allocator), layers_(layers), page_tokens_(page_tokens), kv_heads_(kv_heads),
        head_dim_(head_dim), kv_width_(static_cast<std::size_t>(std::max(kv_heads, 0)) *
                                       std::max(head_dim, 0)),
        tier_(tier), halves_(halves),
        storage_tier_(tier != kFP16 && halves != Halves::kBoth ? kFP16 : tier),
        tier_map_(std::move(tier_map)), current_open_(std::max(layers, 0), 0),
        attend_open_(std::max(layers, 0), 0), sealed_(std::max(layers, 0), 0),
        shadows_(fp16_page_bytes(std::max(page_tokens, 0), kv_width_))
  {
    if (layers <= 0 || page_tokens <= 0 || kv_heads <= 0 || head_dim <= 0)
    {
      throw InvalidArgument("layers, page_tokens, kv_heads and head_dim must be positive");
    }
    if (tier < 0 || tier >= kTierCount)
    {
      throw InvalidArgument("tier " + std::to_string(tier) + " is not one of the four");
    }
    if (tier == kFP16 && halves != Halves::kBoth)
    {
      throw InvalidArgument("only a quantised tier can quantise one half of a page");
    }
    if (!tier_map_.empty() && static_cast<int>(tier_map_.size()) != layers)
    {
      throw InvalidArgument("a tier map needs a row for every layer: " +
                            std::to_string(tier_map_.size()) + " rows for " +
                            std::to_string(layers) + " layers");
    }
    if (!tier_map_.empty() && halves != Halves::kBoth)
    {
      throw InvalidArgument("a diagnostic Halves rounds every page at the cache's one tier, and "
                            "takes no tier map");
    }
    may_be_at_[storage_tier_] = true;
    for (const auto &row : tier_map_)
    {
      for (int t : row)
      {
        if (t < 0 || t >= kTierCount)
        {
          throw InvalidArgument("a tier map names tier " + std::to_string(t) +
                                ", not one of the four");
        }
        may_be_at_[t] = true;
        mixed_ = mixed_ || t != tier;
      }
    }
    seals_ = seals_for(tier, tier_map_, always_seal);
    page_bytes_ = bytes_at(storage_tier_);
    for (int t = 0; t < kTierCount; ++t)
    {
      if (may_be_at_[t])
      {
        require_page_size(t, "a page of positions");
      }
    }
    if (seals_)
    {
      require_page_size(kFP16, "an open page");
    }
    if (halves != Halves::kBoth)
    {
      scratch_page_ = std::make_unique<DeviceBuffer>(bytes_at(tier));
      scratch_halves_ = std::make_unique<DeviceBuffer>(bytes_at(kFP16));
    }
  }

  KVPages::~KVPages()
  {
    try
    {
      for (int page = pages_ - 1; page >= 0; --page)
      {
        for (int layer = layers_ - 1; layer >= 0; --layer)
        {
          if (!evicted({layer, page}))
          {
            allocator_.free({layer, page});
          }
        }
      }
      if (open_pages_)
      {
        for (int k = 1; k >= 0; --k)
        {
          for (int layer = layers_ - 1; layer >= 0; --layer)
          {
            allocator_.free({layer, kOpenPages[k]});
          }
        }
      }
    }
    catch (...)
    {
    }
  }

  void KVPages::require_layer(int layer) const
  {
    if (layer < 0 || layer >= layers_)
    {
      throw OutOfRange("layer " + std::to_string(layer) + " of " + std::to_string(layers_));
    }
  }

  std::size_t KVPages::bytes_at(int tier) const
  {
    return page_bytes_at(tier, page_tokens_, kv_heads_, head_dim_);
  }

  void KVPages::require_page_size(int tier, const char *what) const
  {
    const std::size_t needed = bytes_at(tier);
    if (allocator_.page_bytes(tier) != needed)
    {
      throw InvalidArgument(std::string("the allocator's ") + tier_name(tier) + " pages hold " +
                            std::to_string(allocator_.page_bytes(tier)) + " bytes; " + what +
                            " of " + std::to_string(page_tokens_) + " positions at " +
                            std::to_string(kv_width_) + " elements needs " +
                            std::to_string(needed));
    }
  }

  int KVPages::birth_tier(int layer, int page) const
  {
    if (layer >= 0 && layer < static_cast<int>(tier_map_.size()) && page >= 0 &&
        page < static_cast<int>(tier_map_[layer].size()))
    {
      return tier_map_[layer][page];
    }
    return storage_tier_;
  }

  void KVPages::reserve(int tokens)
  {
    std::vector<PageKey> taken;
    try
    {
      if (seals_ && !open_pages_ && tokens > 0)
      {
        for (int page : kOpenPages)
        {
          for (int layer = 0; layer < layers_; ++layer)
          {
            allocator_.allocate({layer, page}, kFP16);
            taken.push_back({layer, page});
          }
        }
      }
      const int needed = seals_ ? tokens / page_tokens_ : (tokens + page_tokens_ - 1) / page_tokens_;
      for (int page = pages_; page < needed; ++page)
      {
        for (int layer = 0; layer < layers_; ++layer)
        {
          allocator_.allocate({layer, page}, birth_tier(layer, page));
          taken.push_back({layer, page});
        }
      }
      if (seals_ && tokens > 0)
      {
        open_pages_ = true;
      }
      pages_ = std::max(needed, pages_);
    }
    catch (...)
    {
      while (!taken.empty())
      {
        allocator_.free(taken.back());
        taken.pop_back();
      }
      throw;
    }
  }

  KVPages::LayerTable KVPages::resolve(int layer)
  {
    require_layer(layer);
    if (pages_ == 0)
    {
      return {nullptr, nullptr};
    }
    if (resolved_pages_ != pages_ || resolved_generation_ != allocator_.generation())
    {
      if (pages_ > table_stride_)
      {
        table_stride_ = pages_ > 2 * table_stride_ ? pages_ : 2 * table_stride_;
        tables_.reset();
        tables_ = std::make_unique<DeviceBuffer>(static_cast<std::size_t>(layers_) * table_stride_ *
                                                 (sizeof(unsigned long long) + 1));
      }
      const std::size_t entries = static_cast<std::size_t>(layers_) * table_stride_;
      std::vector<unsigned long long> host(entries + (entries + 7) / 8, 0);
      auto *tiers = reinterpret_cast<std::uint8_t *>(host.data() + entries);
      for (int l = 0; l < layers_; ++l)
      {
        for (int page = 0; page < pages_; ++page)
        {
          const std::size_t at = static_cast<std::size_t>(l) * table_stride_ + page;
          if (evicted({l, page}))
          {
            tiers[at] = kUnreadPage;
            continue;
          }
          const PageLocation loc = allocator_.locate({l, page});
          host[at] = reinterpret_cast<unsigned long long>(
              allocator_.address({l, page}, allocator_.page_bytes(loc.tier)));
          tiers[at] = masked({l, page}) ? kUnreadPage : static_cast<std::uint8_t>(loc.tier);
        }
      }
      hip_check(hipMemcpy(tables_->raw(), host.data(),
                          entries * (sizeof(unsigned long long) + 1), hipMemcpyHostToDevice),
                "hipMemcpy page tables host-to-device");
      resolved_pages_ = pages_;
      resolved_generation_ = allocator_.generation();
    }
    const std::size_t entries = static_cast<std::size_t>(layers_) * table_stride_;
    const std::size_t at = static_cast<std::size_t>(layer) * table_stride_;
    return {tables_->as<const unsigned long long>() + at,
            tables_->as<const std::uint8_t>() + entries * sizeof(unsigned long long) + at};
  }

  std::uint16_t *KVPages::open_page(int layer, int which)
  {
    return reinterpret_cast<std::uint16_t *>(
        allocator_.address({layer, kOpenPages[which]}, allocator_.page_bytes(kFP16)));
  }

  void KVPages::store(int layer, const void *keys, const void *values, int start, int n)
  {
    if (start < 0 || n < 0 || start + n > capacity_tokens())
    {
      throw OutOfRange("positions [" + std::to_string(start) + ", " + std::to_string(start + n) +
                       ") are not all on pages; " + std::to_string(capacity_tokens()) +
                       " positions are reserved");
    }
    require_layer(layer);
    if (n == 0)
    {
      return;
    }
    if (seals_)
    {
      store_sealed(layer, static_cast<const std::uint16_t *>(keys),
                   static_cast<const std::uint16_t *>(values), start, n);
      return;
    }
    launch_store_pages(keys, values, resolve(layer).pages, page_tokens_, kv_width_, start, n,
                       runtime_stream());
  }

  void KVPages::store_sealed(int layer, const std::uint16_t *keys, const std::uint16_t *values,
                             int start, int n)
  {
    const std::size_t half = static_cast<std::size_t>(page_tokens_) * kv_width_;
    const int first = start / page_tokens_;
    const int current = current_open_[layer];
    attend_open_[layer] = current;
    std::vector<Seal> seals;
    const int end = start + n;
    for (int at = start; at < end;)
    {
      const int span = at / page_tokens_;
      const int span_start = span * page_tokens_;
      const int take = std::min(end, span_start + page_tokens_) - at;
      const std::size_t from = static_cast<std::size_t>(at - start) * kv_width_;
      if (take == page_tokens_)
      {
        seals.push_back({span, keys + from, values + from});
      }
      else
      {
        const int which = span == first ? current : 1 - current;
        std::uint16_t *open = open_page(layer, which);
        const std::size_t row = static_cast<std::size_t>(at - span_start);
        const std::size_t bytes = static_cast<std::size_t>(take) * kv_width_ * 2;
        hip_check(hipMemcpyAsync(open + row * kv_width_, keys + from, bytes,
                                 hipMemcpyDeviceToDevice, runtime_stream()),
                  "hipMemcpyAsync keys into an open page");
        hip_check(hipMemcpyAsync(open + half + row * kv_width_, values + from, bytes,
                                 hipMemcpyDeviceToDevice, runtime_stream()),
                  "hipMemcpyAsync values into an open page");
        if (at + take == span_start + page_tokens_)
        {
          seals.push_back({span, open, open + half});
        }
        current_open_[layer] = which;
      }
      at += take;
    }
    seal_batch(layer, seals);
  }

  void KVPages::seal_batch(int layer, const std::vector<Seal> &seals)
  {
    if (seals.empty())
    {
      return;
    }
    const std::size_t half = static_cast<std::size_t>(page_tokens_) * kv_width_;
    const hipStream_t stream = runtime_stream();
    // Resolved now, between allocator operations, and used at once.
    struct Job
    {
      const std::uint16_t *keys;
      const std::uint16_t *values;
      char *page;
    };
    std::array<std::vector<Job>, kTierCount> by_tier;
    for (const Seal &s : seals)
    {
      const PageLocation loc = allocator_.locate({layer, s.span});
      char *page = allocator_.address({layer, s.span}, allocator_.page_bytes(loc.tier));
      sealed_[layer] = std::max(sealed_[layer], s.span + 1);
      if (halves_ != Halves::kBoth)
      {
        // The diagnostic: the tier's round trip for one half, the other as it
        // came, both into an FP16 page.
        auto *round_trip = scratch_halves_->as<std::uint16_t>();
        launch_quantise_pages(nullptr, nullptr, s.keys, scratch_page_->raw(),
                              reinterpret_cast<const char *>(s.values) -
                                  reinterpret_cast<const char *>(s.keys),
                              1, tier_, page_tokens_, kv_heads_, head_dim_, stream);
        launch_dequantise_page(scratch_page_->raw(), round_trip, round_trip + half, tier_,
                               page_tokens_, kv_heads_, head_dim_, stream);
        const std::uint16_t *k = halves_ == Halves::kKeys ? round_trip : s.keys;
        const std::uint16_t *v = halves_ == Halves::kValues ? round_trip + half : s.values;
        hip_check(hipMemcpyAsync(page, k, half * 2, hipMemcpyDeviceToDevice, stream),
                  "hipMemcpyAsync sealed keys");
        hip_check(hipMemcpyAsync(page + half * 2, v, half * 2, hipMemcpyDeviceToDevice, stream),
                  "hipMemcpyAsync sealed values");
        continue;
      }
      by_tier[loc.tier].push_back({s.keys, s.values, page});
    }
    // A page or two goes by value; a larger batch through address tables.
    std::vector<const void *> table;
    struct Launch
    {
      int tier;
      std::ptrdiff_t values_offset;
      std::size_t at;
      int count;
      bool fp16_values; // for FP16: the second copy, values into the pages' second half
    };
    std::vector<Launch> launches;
    for (int t = 0; t < kTierCount; ++t)
    {
      // Group by the distance from keys to values: uniform per launch.
      std::map<std::ptrdiff_t, std::vector<const Job *>> groups;
      for (const Job &j : by_tier[t])
      {
        groups[reinterpret_cast<const char *>(j.values) - reinterpret_cast<const char *>(j.keys)]
            .push_back(&j);
      }
      for (const auto &[offset, jobs] : groups)
      {
        if (jobs.size() == 1)
        {
          const Job &j = *jobs[0];
          if (t == kFP16)
          {
            hip_check(hipMemcpyAsync(j.page, j.keys, half * 2, hipMemcpyDeviceToDevice, stream),
                      "hipMemcpyAsync sealed keys");
            hip_check(hipMemcpyAsync(j.page + half * 2, j.values, half * 2,
                                     hipMemcpyDeviceToDevice, stream),
                      "hipMemcpyAsync sealed values");
          }
          else
          {
            launch_quantise_pages(nullptr, nullptr, j.keys, j.page, offset, 1, t, page_tokens_,
                                  kv_heads_, head_dim_, stream);
          }
          continue;
        }
        if (t == kFP16)
        {
          const std::size_t keys_at = table.size();
          for (const Job *j : jobs) table.push_back(j->keys);
          for (const Job *j : jobs) table.push_back(j->page);
          launches.push_back({t, offset, keys_at, static_cast<int>(jobs.size()), false});
          const std::size_t values_at = table.size();
          for (const Job *j : jobs) table.push_back(j->values);
          for (const Job *j : jobs) table.push_back(j->page + half * 2);
          launches.push_back({t, offset, values_at, static_cast<int>(jobs.size()), true});
        }
        else
        {
          const std::size_t at = table.size();
          for (const Job *j : jobs) table.push_back(j->keys);
          for (const Job *j : jobs) table.push_back(j->page);
          launches.push_back({t, offset, at, static_cast<int>(jobs.size()), false});
        }
      }
    }
    if (launches.empty())
    {
      return;
    }
    const void *const *on_device = upload_table(batch_table_, table);
    for (const Launch &l : launches)
    {
      const void *const *from = on_device + l.at;
      void *const *to = const_cast<void *const *>(on_device + l.at + l.count);
      if (l.tier == kFP16)
      {
        launch_copy_pages(from, to, half * 2, l.count, stream);
      }
      else
      {
        launch_quantise_pages(from, to, nullptr, nullptr, l.values_offset, l.count, l.tier,
                              page_tokens_, kv_heads_, head_dim_, stream);
      }
    }
  }

  PageKey KVPages::require_movable(int layer, int page, const char *verb) const
  {
    if (!seals_)
    {
      throw InvalidArgument(std::string("only a cache that seals can ") + verb +
                            " a page: in one that does not, every page is FP16 and its last is "
                            "still being written");
    }
    if (halves_ != Halves::kBoth)
    {
      throw InvalidArgument(std::string("a diagnostic Halves stores every page at FP16 by its "
                                        "definition; none can ") +
                            verb);
    }
    require_layer(layer);
    if (page < 0 || page >= pages_)
    {
      throw InvalidArgument(page_name({layer, page}) +
                            " is not a page of positions this cache holds; only one of those moves");
    }
    if (page >= sealed_[layer])
    {
      throw InvalidArgument(page_name({layer, page}) +
                            " is not sealed: its positions are reserved, not all stored");
    }
    return {layer, page};
  }

  PageKey KVPages::require_held(int layer, int page, const char *verb) const
  {
    const PageKey key = require_movable(layer, page, verb);
    if (evicted(key))
    {
      throw InvalidArgument(page_name(key) + " is evicted: its positions are gone, and nothing can " +
                            verb + " it");
    }
    return key;
  }

  std::string KVPages::page_name(PageKey key)
  {
    return "page " + std::to_string(key.page) + " of layer " + std::to_string(key.layer);
  }

  void KVPages::evict(int layer, int page)
  {
    const PageKey key = require_held(layer, page, "evict");
    if (masked(key))
    {
      throw InvalidArgument(page_name(key) +
                            " is masked, the reference an eviction is measured against; evict "
                            "another cache's page");
    }
    allocator_.free(key);
    evicted_.insert(key);
  }

  void KVPages::mask(int layer, int page)
  {
    const PageKey key = require_held(layer, page, "mask");
    masked_.insert(key);
    resolved_pages_ = -1;
  }

  void KVPages::downgrade(int layer, int page, int target)
  {
    const PageKey key = require_held(layer, page, "downgrade");
    if (target < 0 || target >= kTierCount)
    {
      throw InvalidArgument("tier " + std::to_string(target) + " is not one of the four");
    }
    const int current = page_tier(key);
    if (!is_lower(target, current))
    {
      throw InvalidArgument(page_name(key) + " is at " + tier_name(current) +
                            "; a downgrade is to a lower tier, and " + tier_name(target) +
                            " is not");
    }
    if (current != kFP16 && !shadows_.contains(key))
    {
      throw InvalidArgument(page_name(key) + " was born at " + tier_name(current) +
                            " and has no FP16 shadow to quantise from; only a page sealed at "
                            "FP16 downgrades");
    }
    move(key, current, target);
  }

  void KVPages::upgrade(int layer, int page, int target)
  {
    const PageKey key = require_held(layer, page, "upgrade");
    if (target < 0 || target >= kTierCount)
    {
      throw InvalidArgument("tier " + std::to_string(target) + " is not one of the four");
    }
    const int current = page_tier(key);
    if (!is_lower(current, target))
    {
      throw InvalidArgument(page_name(key) + " is at " + tier_name(current) +
                            "; an upgrade is to a higher tier, and " + tier_name(target) +
                            " is not");
    }
    if (!shadows_.contains(key))
    {
      throw InvalidArgument(page_name(key) + " was born at " + tier_name(current) +
                            " and has no FP16 shadow to restore it from");
    }
    move(key, current, target);
  }

  void KVPages::move(PageKey key, int current, int target)
  {
    require_page_size(target, "a page of positions");
    const hipStream_t stream = runtime_stream();
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before a move");
    const Clock::time_point began = Clock::now();
    double shadow_seconds = 0.0;
    const bool from_shadow = current != kFP16;
    const bool upload_shadow = from_shadow && target != kFP16;
    const PageKey staged{key.layer, kStagingPage};
    const PageKey upload{key.layer, kShadowUploadPage};
    allocator_.allocate(staged, target);
    if (upload_shadow)
    {
      try
      {
        allocator_.allocate(upload, kFP16);
      }
      catch (...)
      {
        allocator_.free(staged);
        throw;
      }
    }
    try
    {
      const std::size_t fp16_bytes = bytes_at(kFP16);
      char *staged_bytes = allocator_.address(staged, allocator_.page_bytes(target));
      if (!from_shadow && !shadows_.contains(key))
      {
        const Clock::time_point copying = Clock::now();
        shadows_.take(key, allocator_.address(key, fp16_bytes), stream);
        shadow_seconds = since(copying);
      }
      const void *rows = nullptr;
      if (from_shadow)
      {
        void *to = target == kFP16 ? static_cast<void *>(staged_bytes)
                                   : static_cast<void *>(allocator_.address(upload, fp16_bytes));
        const Clock::time_point copying = Clock::now();
        hip_check(hipMemcpy(to, shadows_.shadow(key), fp16_bytes, hipMemcpyHostToDevice),
                  "hipMemcpy a page's FP16 shadow host-to-device");
        shadow_seconds = since(copying);
        rows = to;
      }
      else
      {
        rows = allocator_.address(key, fp16_bytes);
      }
      if (target != kFP16)
      {
        launch_quantise_pages(nullptr, nullptr, rows, staged_bytes,
                              static_cast<std::ptrdiff_t>(fp16_bytes / 2), 1, target, page_tokens_,
                              kv_heads_, head_dim_, stream);
      }
      if (upload_shadow)
      {
        allocator_.free(upload); // its tier's tail; the free synchronises
      }
    }
    catch (...)
    {
      if (upload_shadow && allocator_.contains(upload))
      {
        allocator_.free(upload);
      }
      allocator_.free(staged);
      throw;
    }
    allocator_.replace(key, staged);
    may_be_at_[target] = true;
    last_move_ = MoveRecord{key, current, target, bytes_at(current), bytes_at(target),
                            since(began), shadow_seconds};
  }

  void KVPages::move_pages(const std::vector<PageMove> &moves)
  {
    std::vector<PageKey> keys;
    std::vector<int> current;
    std::set<PageKey> named;
    for (const PageMove &m : moves)
    {
      const PageKey key = require_held(m.key.layer, m.key.page, "move");
      if (!named.insert(key).second)
      {
        throw InvalidArgument(page_name(key) +
                              " is named twice in one batch; a batch moves a page once, to the "
                              "tier it ends at");
      }
      if (m.target < 0 || m.target >= kTierCount)
      {
        throw InvalidArgument("tier " + std::to_string(m.target) + " is not one of the four");
      }
      const int from = page_tier(key);
      if (from == m.target)
      {
        throw InvalidArgument(page_name(key) + " is already at " + tier_name(from));
      }
      if (from != kFP16 && !shadows_.contains(key))
      {
        throw InvalidArgument(page_name(key) + " was born at " + tier_name(from) +
                              " and has no FP16 shadow to move from; only a page sealed at FP16 "
                              "moves");
      }
      require_page_size(m.target, "a page of positions");
      keys.push_back(key);
      current.push_back(from);
    }
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before a batch");
    const Clock::time_point began = Clock::now();
    const std::size_t n = moves.size();
    if (n == 0)
    {
      last_batch_ = BatchRecord{0, 0, 0.0};
      return;
    }
    const hipStream_t stream = runtime_stream();

    // 1. Every new page under a key of its own, and room for the shadows.
    std::size_t first_downgrades = 0;
    for (std::size_t i = 0; i < n; ++i)
    {
      first_downgrades += current[i] == kFP16 && !shadows_.contains(keys[i]);
    }
    auto addresses = std::make_unique<DeviceBuffer>(2 * (first_downgrades + n) * sizeof(void *));
    std::vector<PageKey> staged;
    try
    {
      for (std::size_t i = 0; i < n; ++i)
      {
        const PageKey stage{keys[i].layer, kBatchStagingPage - static_cast<int>(i)};
        allocator_.allocate(stage, moves[i].target);
        staged.push_back(stage);
      }
      shadows_.reserve(first_downgrades);
    }
    catch (...)
    {
      allocator_.free_pages(staged);
      throw;
    }

    // 2. The device's work: shadows out, restores in, one quantise launch per
    // target tier, all reading pages before any is freed.
    std::vector<const void *> shadow_from, restore_from;
    std::vector<void *> shadow_to, restore_to;
    std::array<std::vector<const void *>, kTierCount> rows;
    std::array<std::vector<void *>, kTierCount> pages;
    const std::size_t fp16_bytes = bytes_at(kFP16);
    for (std::size_t i = 0; i < n; ++i)
    {
      const PageKey key = keys[i];
      void *to = allocator_.address(staged[i], allocator_.page_bytes(moves[i].target));
      const void *fp16 = nullptr;
      if (current[i] == kFP16)
      {
        fp16 = allocator_.address(key, fp16_bytes);
        if (!shadows_.contains(key))
        {
          shadow_from.push_back(fp16);
          shadow_to.push_back(shadows_.add(key));
        }
      }
      else
      {
        fp16 = shadows_.device_shadow(key);
      }
      const int target = moves[i].target;
      if (target == kFP16)
      {
        restore_from.push_back(fp16);
        restore_to.push_back(to);
      }
      else
      {
        rows[target].push_back(fp16);
        pages[target].push_back(to);
      }
    }
    std::vector<const void *> table;
    const auto place = [&table](const auto &from, const auto &to) {
      const std::size_t at = table.size();
      table.insert(table.end(), from.begin(), from.end());
      table.insert(table.end(), to.begin(), to.end());
      return at;
    };
    const std::size_t shadow_at = place(shadow_from, shadow_to);
    const std::size_t restore_at = place(restore_from, restore_to);
    std::array<std::size_t, kTierCount> tier_at{};
    for (int t = 0; t < kTierCount; ++t)
    {
      tier_at[t] = place(rows[t], pages[t]);
    }
    hip_check(hipMemcpy(addresses->raw(), table.data(), table.size() * sizeof(void *),
                        hipMemcpyHostToDevice),
              "hipMemcpy a batch's page addresses");
    const auto *on_device = addresses->as<const void *const>();
    const auto writable = [](const void *const *p) { return const_cast<void *const *>(p); };
    launch_copy_pages(on_device + shadow_at, writable(on_device + shadow_at + shadow_from.size()),
                      fp16_bytes, static_cast<int>(shadow_from.size()), stream);
    launch_copy_pages(on_device + restore_at,
                      writable(on_device + restore_at + restore_from.size()), fp16_bytes,
                      static_cast<int>(restore_from.size()), stream);
    for (int t = 0; t < kTierCount; ++t)
    {
      if (rows[t].empty())
      {
        continue;
      }
      launch_quantise_pages(on_device + tier_at[t], writable(on_device + tier_at[t] + rows[t].size()),
                            nullptr, nullptr, static_cast<std::ptrdiff_t>(fp16_bytes / 2),
                            static_cast<int>(rows[t].size()), t, page_tokens_, kv_heads_,
                            head_dim_, stream);
    }

    // 3. The page table names the new pages; the old ones are freed together.
    std::vector<std::pair<PageKey, PageKey>> pairs;
    for (std::size_t i = 0; i < n; ++i)
    {
      pairs.emplace_back(keys[i], staged[i]);
      may_be_at_[moves[i].target] = true;
    }
    try
    {
      allocator_.replace_pages(pairs);
    }
    catch (...)
    {
      (void)hipDeviceSynchronize();
      allocator_.free_pages(staged);
      throw;
    }
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize after a batch");
    last_batch_ = BatchRecord{n, shadow_from.size(), since(began)};
  }

  void KVPages::attention(int layer, const void *q, const void *k_bias, const RopeTable *rope,
                          void *out, int seq_q, int seq_k, int heads, int kv_heads, int head_dim,
                          const void *keys, const void *values, float *mass, float *scores,
                          float alpha, float *partials)
  {
    if (static_cast<std::size_t>(kv_heads) * head_dim != kv_width_)
    {
      throw InvalidArgument("kv_heads * head_dim is " + std::to_string(kv_heads * head_dim) +
                            "; this cache holds " + std::to_string(kv_width_) + " per token");
    }
    if (seq_k < 0 || seq_k > capacity_tokens())
    {
      throw OutOfRange("seq_k " + std::to_string(seq_k) + " exceeds the " +
                       std::to_string(capacity_tokens()) + " positions on pages");
    }
    require_layer(layer);
    if (seq_q <= 0)
    {
      return;
    }
    if (k_bias != nullptr && (rope == nullptr || rope->head_dim() != head_dim))
    {
      throw InvalidArgument("a key bias needs a RoPE table for head_dim " +
                            std::to_string(head_dim) + " covering " + std::to_string(seq_k) +
                            " positions");
    }
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    AttentionArgs a{};
    a.q = static_cast<const std::uint16_t *>(q);
    a.out = static_cast<std::uint16_t *>(out);
    a.k_bias = static_cast<const std::uint16_t *>(k_bias);
    a.rope = k_bias != nullptr ? rope->data() : nullptr;
    a.rope_positions = k_bias != nullptr ? rope->positions() : 0;
    a.rope_angles = k_bias != nullptr ? rope->angles() : nullptr;
    a.seq_q = seq_q;
    a.seq_k = seq_k;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.mass = mass;
    a.scores = scores;
    a.alpha = alpha;
    a.partials = partials;
    a.workspace = &workspace_;
    if (!seals_)
    {
      kv.layout = Layout::kPaged;
      kv.pages = resolve(layer).pages;
      kv.may_be_at[kFP16] = true;
      launch_attention(kv, a, runtime_stream());
      return;
    }
    if (keys == nullptr || values == nullptr)
    {
      throw InvalidArgument("attention at a quantised tier reads each query's own page from the "
                            "rows the queries stored; pass them");
    }
    if (!open_pages_)
    {
      throw LogicError("attention before any position was reserved");
    }
    const LayerTable table = resolve(layer);
    kv.layout = Layout::kCausal;
    kv.pages = table.pages;
    kv.tiers = table.tiers;
    kv.open = open_page(layer, attend_open_[layer]);
    kv.chunk_k = static_cast<const std::uint16_t *>(keys);
    kv.chunk_v = static_cast<const std::uint16_t *>(values);
    kv.start = seq_k - seq_q;
    for (int t = 0; t < kTierCount; ++t)
    {
      kv.may_be_at[t] = may_be_at_[t];
    }
    if (seq_q == 1 && layer + 1 < layers_)
    {
      // A decode step visits the layers in order.
      const LayerTable next = resolve(layer + 1);
      kv.warm_pages = next.pages;
      kv.warm_tiers = next.tiers;
      // The next layer's sealed pages only: the table holds pages_ entries.
      kv.warm_count = std::min((seq_k - 1) / page_tokens_, pages_);
    }
    launch_attention(kv, a, runtime_stream());
  }

  const unsigned long long *KVPages::open_table()
  {
    std::vector<unsigned long long> now(static_cast<std::size_t>(layers_));
    for (int l = 0; l < layers_; ++l)
    {
      now[l] = reinterpret_cast<unsigned long long>(open_page(l, attend_open_[l]));
    }
    if (open_table_ == nullptr)
    {
      open_table_ = std::make_unique<DeviceBuffer>(now.size() * sizeof(unsigned long long));
    }
    if (now != open_uploaded_)
    {
      hip_check(hipMemcpy(open_table_->raw(), now.data(), now.size() * sizeof(unsigned long long),
                          hipMemcpyHostToDevice),
                "hipMemcpy open-page table host-to-device");
      open_uploaded_ = now;
    }
    return open_table_->as<const unsigned long long>();
  }

  void KVPages::attention_layers(int first_layer, int layers, const void *q, long long q_stride,
                                 void *out, long long out_stride, int seq_k, int heads,
                                 int kv_heads, int head_dim, const void *keys, const void *values,
                                 long long kv_stride, float *mass, long long mass_stride,
                                 float *scores, long long scores_stride, float alpha)
  {
    if (layers < 0 || first_layer < 0 || first_layer + layers > layers_)
    {
      throw OutOfRange("layers [" + std::to_string(first_layer) + ", " +
                       std::to_string(first_layer + layers) + ") are not all in this cache's " +
                       std::to_string(layers_));
    }
    if (layers == 0)
    {
      return;
    }
    if (static_cast<std::size_t>(kv_heads) * head_dim != kv_width_)
    {
      throw InvalidArgument("kv_heads * head_dim is " + std::to_string(kv_heads * head_dim) +
                            "; this cache holds " + std::to_string(kv_width_) + " per token");
    }
    if (seq_k <= 0 || seq_k > capacity_tokens())
    {
      throw OutOfRange("seq_k " + std::to_string(seq_k) + " is not within the " +
                       std::to_string(capacity_tokens()) + " positions on pages");
    }
    if (seals_ && (keys == nullptr || values == nullptr))
    {
      throw InvalidArgument("attention at a quantised tier reads each query's own page from the "
                            "rows the queries stored; pass them");
    }
    if (seals_ && !open_pages_)
    {
      throw LogicError("attention before any position was reserved");
    }
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    AttentionArgs a{};
    a.q = static_cast<const std::uint16_t *>(q);
    a.out = static_cast<std::uint16_t *>(out);
    a.seq_q = 1;
    a.seq_k = seq_k;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.mass = mass;
    a.scores = scores;
    a.alpha = alpha;
    a.workspace = &workspace_;
    const LayerTable base = resolve(0);
    kv.pages = base.pages;
    if (seals_)
    {
      kv.layout = Layout::kCausal;
      kv.tiers = base.tiers;
      kv.open = open_page(first_layer, attend_open_[first_layer]);
      kv.chunk_k = static_cast<const std::uint16_t *>(keys);
      kv.chunk_v = static_cast<const std::uint16_t *>(values);
      kv.start = seq_k - 1;
      for (int t = 0; t < kTierCount; ++t)
      {
        kv.may_be_at[t] = may_be_at_[t];
      }
    }
    else
    {
      kv.layout = Layout::kPaged;
      kv.may_be_at[kFP16] = true;
    }
    if (decode_fast_applies(kv, a))
    {
      DecodeLayers ls{};
      ls.split = true;
      ls.first_layer = first_layer;
      ls.layers = layers;
      ls.table_stride = table_stride_;
      ls.open_table = seals_ ? open_table() : nullptr;
      ls.q_stride = q_stride;
      ls.chunk_stride = kv_stride;
      ls.out_stride = out_stride;
      ls.mass_stride = mass_stride;
      ls.scores_stride = scores_stride;
      launch_decode_layers(kv, a, ls, runtime_stream());
      return;
    }
    throw InvalidArgument("attention over several layers in one launch takes one query per "
                          "head, 32-token pages, head_dim 64 or 128 and at most 16 query heads "
                          "per KV head, 16-byte aligned; got head_dim " +
                          std::to_string(head_dim) + ", " + std::to_string(heads) + "/" +
                          std::to_string(kv_heads) + " heads, " + std::to_string(page_tokens_) +
                          "-token pages");
  }

} // namespace mi
