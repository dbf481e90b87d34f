// The per-tier page allocator on HIP's virtual memory API, and the small
// device-memory helpers of the runtime.
//
// Contract (reference: src/core_kernels/paged_kv_cache.cu, ADR-0007): each
// tier's pages are packed from slot 0; a single free moves the tier's last
// page into the hole; a batched free keeps the first `held - freed` slots,
// filling each hole among them, lowest first, with the surviving pages from
// above, lowest first; a tier maps whole granules up to what its pages reach
// (plus the spares kept) and gives back the rest.
//
// How it is done here:
//   - a key is one 64-bit word; where each key lives is one hash-map entry,
//     and each tier's slot array names its owners, so a batched free costs
//     the freed pages' sort and the survivors' moves, not a walk of the
//     tier;
//   - every compaction copy of a call, over all four tiers, is one launch of
//     copy_refs (slot references, addresses formed on the device), queued on
//     the runtime stream without waiting for it;
//   - a granule the tail gives up is unmapped by the releaser thread once an
//     event recorded after the call's copies has completed, so no caller
//     waits for the device or for the driver's unmap; an address about to be
//     mapped again waits for its own release only;
//   - every page whose slot changes is reported to the watching KVPages,
//     which edit their device page tables instead of rebuilding them.

#include "runtime.hpp"

#include <algorithm>
#include <atomic>

namespace mi
{
  namespace
  {
    std::atomic<int> g_fail_granules{0};
    thread_local hipStream_t g_stream = nullptr;

    std::size_t round_up(std::size_t n, std::size_t m) { return (n + m - 1) / m * m; }

    hipMemAllocationProp device_prop(int device)
    {
      hipMemAllocationProp prop{};
      prop.type = hipMemAllocationTypePinned;
      prop.location.type = hipMemLocationTypeDevice;
      prop.location.id = device;
      return prop;
    }

    // The unit each tier's range is backed and released in: the driver's
    // recommended granularity, and at least 2 MiB, as a whole multiple of its
    // minimum. On MI355X the minimum is 4 KiB; a 32K-context cache mapped at
    // that would take hundreds of thousands of physical allocations, past
    // what the driver hands out (hipMemCreate then fails with VRAM free), so
    // the allocator maps 2 MiB granules, the reference's own.
    constexpr std::size_t kMinGranule = std::size_t{2} << 20;

    std::size_t mapping_unit(const hipMemAllocationProp &prop)
    {
      std::size_t minimum = 0, recommended = 0;
      hip_check(hipMemGetAllocationGranularity(&minimum, &prop, hipMemAllocationGranularityMinimum),
                "hipMemGetAllocationGranularity");
      if (hipMemGetAllocationGranularity(&recommended, &prop,
                                         hipMemAllocationGranularityRecommended) != hipSuccess)
      {
        (void)hipGetLastError();
        recommended = minimum;
      }
      const std::size_t unit = std::max({minimum, recommended, kMinGranule});
      return minimum > 0 ? round_up(unit, minimum) : unit;
    }
  } // namespace

  hipStream_t runtime_stream() { return g_stream; }
  void set_runtime_stream(hipStream_t stream) { g_stream = stream; }

  std::string describe(PageKey key)
  {
    return "page (layer " + std::to_string(key.layer) + ", page_index " +
           std::to_string(key.page) + ")";
  }

  void fail_next_granules(int n) { g_fail_granules = n; }

  DeviceBuffer::DeviceBuffer(std::size_t bytes) : bytes_(bytes)
  {
    if (bytes > 0)
    {
      hip_check(hipMalloc(&ptr_, bytes), "hipMalloc");
    }
  }

  DeviceBuffer::~DeviceBuffer()
  {
    if (ptr_ != nullptr)
    {
      // A launch may still read it: the free waits for the device first.
      (void)hipDeviceSynchronize();
      (void)hipFree(ptr_);
    }
  }

  const void *UploadBuffer::send_bytes(const void *host, std::size_t bytes, hipStream_t stream)
  {
    if (bytes == 0)
    {
      return nullptr;
    }
    if (!buffer_ || buffer_->bytes() < bytes)
    {
      buffer_.reset(); // waits for launches that may read the old one
      buffer_ = std::make_unique<DeviceBuffer>(std::max<std::size_t>(2 * bytes, 4096));
    }
    // Ordered after every launch already queued on the stream, which may
    // still read what the buffer held; pageable host memory is staged by the
    // runtime before the call returns, so `host` may go at once.
    hip_check(hipMemcpyAsync(buffer_->raw(), host, bytes, hipMemcpyHostToDevice, stream),
              "hipMemcpyAsync an upload");
    return buffer_->raw();
  }

  std::size_t granule_bytes()
  {
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    return mapping_unit(device_prop(device));
  }

  // ---- the releaser --------------------------------------------------------------

  // Unmaps and releases granules off the caller's thread. Each batch of
  // granules given up together waits for an event recorded on the runtime
  // stream when they were given up: every launch that could read them was
  // queued before it.
  class GranuleReleaser
  {
  public:
    GranuleReleaser(int device, std::size_t granule) : device_(device), granule_(granule) {}

    ~GranuleReleaser()
    {
      {
        std::lock_guard<std::mutex> lock(mutex_);
        stop_ = true;
      }
      wake_.notify_one();
      if (thread_.joinable())
      {
        thread_.join();
      }
    }

    void retire(std::vector<std::pair<char *, hipMemGenericAllocationHandle_t>> granules,
                hipStream_t stream)
    {
      if (granules.empty())
      {
        return;
      }
      auto gate = std::make_shared<Gate>();
      if (hipEventCreateWithFlags(&gate->event, hipEventDisableTiming) != hipSuccess ||
          hipEventRecord(gate->event, stream) != hipSuccess)
      {
        // No event: wait for the stream here instead.
        (void)hipGetLastError();
        if (gate->event != nullptr)
        {
          (void)hipEventDestroy(gate->event);
          gate->event = nullptr;
        }
        hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize before a release");
      }
      {
        std::lock_guard<std::mutex> lock(mutex_);
        for (const auto &[at, handle] : granules)
        {
          queue_.push_back({at, handle, gate});
        }
        if (!thread_.joinable())
        {
          thread_ = std::thread([this] { loop(); });
        }
      }
      wake_.notify_one();
    }

    // Waits until the granule at `at` (nullptr: every granule) is released;
    // raises the first failure of the thread.
    void wait_for(const char *at)
    {
      std::unique_lock<std::mutex> lock(mutex_);
      const auto pending = [&] {
        if (at == nullptr)
        {
          return !queue_.empty() || busy_ != nullptr;
        }
        if (busy_ == at)
        {
          return true;
        }
        return std::any_of(queue_.begin(), queue_.end(),
                           [at](const Item &i) { return i.at == at; });
      };
      done_.wait(lock, [&] { return !pending(); });
      if (!error_.empty())
      {
        const std::string e = error_;
        error_.clear();
        throw DeviceError(e);
      }
    }

  private:
    struct Gate
    {
      hipEvent_t event = nullptr;
      ~Gate()
      {
        if (event != nullptr)
        {
          (void)hipEventDestroy(event);
        }
      }
    };
    struct Item
    {
      char *at;
      hipMemGenericAllocationHandle_t handle;
      std::shared_ptr<Gate> gate;
    };

    void loop()
    {
      const hipError_t set = hipSetDevice(device_);
      std::unique_lock<std::mutex> lock(mutex_);
      for (;;)
      {
        wake_.wait(lock, [this] { return stop_ || !queue_.empty(); });
        if (queue_.empty())
        {
          return;
        }
        Item item = std::move(queue_.front());
        queue_.pop_front();
        busy_ = item.at;
        lock.unlock();
        hipError_t e = set;
        if (e == hipSuccess && item.gate->event != nullptr)
        {
          e = hipEventSynchronize(item.gate->event);
        }
        if (e == hipSuccess)
        {
          e = hipMemUnmap(item.at, granule_);
        }
        const hipError_t released = hipMemRelease(item.handle);
        if (e == hipSuccess)
        {
          e = released;
        }
        item.gate.reset();
        lock.lock();
        busy_ = nullptr;
        if (e != hipSuccess && error_.empty())
        {
          error_ = std::string("releasing a granule: ") + hipGetErrorString(e);
        }
        done_.notify_all();
      }
    }

    int device_;
    std::size_t granule_;
    std::mutex mutex_;
    std::condition_variable wake_;
    std::condition_variable done_;
    std::deque<Item> queue_;
    const char *busy_ = nullptr;
    bool stop_ = false;
    std::string error_;
    std::thread thread_;
  };

  // ---- the allocator -----------------------------------------------------------------

  PagedKVCache::PagedKVCache(const std::array<std::size_t, kTierCount> &page_bytes,
                             const std::array<std::size_t, kTierCount> &capacity_pages)
  {
    for (int t = 0; t < kTierCount; ++t)
    {
      if (page_bytes[t] == 0)
      {
        throw InvalidArgument("page_bytes for tier " + std::to_string(t) + " must be positive");
      }
    }
    hip_check(hipGetDevice(&device_), "hipGetDevice");
    prop_ = device_prop(device_);
    granule_ = mapping_unit(prop_);
    releaser_ = std::make_unique<GranuleReleaser>(device_, granule_);
    for (int t = 0; t < kTierCount; ++t)
    {
      Range &r = ranges_[t];
      r.page_bytes = page_bytes[t];
      r.capacity = capacity_pages[t];
      r.reserved = round_up(page_bytes[t] * capacity_pages[t], granule_);
      if (r.reserved == 0)
      {
        continue;
      }
      void *base = nullptr;
      const hipError_t e = hipMemAddressReserve(&base, r.reserved, granule_, nullptr, 0);
      if (e != hipSuccess)
      {
        for (int u = 0; u < t; ++u)
        {
          if (ranges_[u].base != nullptr)
          {
            (void)hipMemAddressFree(ranges_[u].base, ranges_[u].reserved);
          }
        }
        hip_check(e, "hipMemAddressReserve");
      }
      r.base = static_cast<char *>(base);
    }
  }

  PagedKVCache::~PagedKVCache()
  {
    (void)hipDeviceSynchronize();
    releaser_.reset(); // finishes every release queued
    for (Range &r : ranges_)
    {
      for (std::size_t g = r.granules.size(); g-- > 0;)
      {
        (void)hipMemUnmap(r.base + g * granule_, granule_);
        (void)hipMemRelease(r.granules[g]);
      }
      r.granules.clear();
      if (r.base != nullptr)
      {
        (void)hipMemAddressFree(r.base, r.reserved);
      }
    }
  }

  void PagedKVCache::check_tier(int tier)
  {
    if (tier < 0 || tier >= kTierCount)
    {
      throw InvalidArgument("tier " + std::to_string(tier) + " is not one of the four");
    }
  }

  void PagedKVCache::unwatch(PlacementObserver *o)
  {
    observers_.erase(std::remove(observers_.begin(), observers_.end(), o), observers_.end());
  }

  void PagedKVCache::tell_placed(std::uint64_t key, int tier, std::size_t slot)
  {
    for (PlacementObserver *o : observers_)
    {
      o->placed(unpack(key), tier, slot);
    }
  }

  void PagedKVCache::tell_removed(std::uint64_t key)
  {
    for (PlacementObserver *o : observers_)
    {
      o->removed(unpack(key));
    }
  }

  void PagedKVCache::allocate(PageKey key, int tier) { allocate_run({key}, tier, true); }

  void PagedKVCache::allocate_run(const std::vector<PageKey> &keys, int tier, bool top_up_spares)
  {
    check_tier(tier);
    Range &r = ranges_[tier];
    if (keys.empty())
    {
      return;
    }
    std::vector<std::uint64_t> words;
    words.reserve(keys.size());
    for (const PageKey &k : keys)
    {
      const std::uint64_t w = pack(k);
      if (where_.count(w) != 0)
      {
        throw InvalidArgument(describe(k) + " is already allocated");
      }
      words.push_back(w);
    }
    if (keys.size() > 1)
    {
      std::vector<std::uint64_t> sorted = words;
      std::sort(sorted.begin(), sorted.end());
      const auto dup = std::adjacent_find(sorted.begin(), sorted.end());
      if (dup != sorted.end())
      {
        throw InvalidArgument(describe(unpack(*dup)) + " is already allocated");
      }
    }
    if (r.owners.size() + keys.size() > r.capacity)
    {
      throw Full(std::string(tier_name(tier)) + " is full at " + std::to_string(r.capacity) +
                 " pages");
    }
    const std::size_t first = r.owners.size();
    r.owners.insert(r.owners.end(), words.begin(), words.end());
    try
    {
      // Spare granules are taken first. A batch's staging run maps only
      // what its pages need: it is on its caller's critical path, and the
      // next allocation that tops the spares up maps them then.
      fit(r, top_up_spares);
    }
    catch (const OutOfMemory &e)
    {
      std::size_t free_bytes = 0, total_bytes = 0;
      const bool known = hipMemGetInfo(&free_bytes, &total_bytes) == hipSuccess;
      r.owners.resize(first);
      try
      {
        fit(r, false);
      }
      catch (...)
      {
      }
      throw OutOfMemory(std::string("out of device memory: the ") + tier_name(tier) +
                        " range could not map " +
                        std::to_string(granule_) + " more bytes for " + describe(keys.front()) +
                        (keys.size() > 1 ? " (+" + std::to_string(keys.size() - 1) + " pages)"
                                         : std::string()) +
                        " (" + e.what() + ")" +
                        (known ? ", with " + std::to_string(free_bytes) + " B free on the device"
                               : std::string()));
    }
    catch (...)
    {
      r.owners.resize(first);
      try
      {
        fit(r, false);
      }
      catch (...)
      {
      }
      throw;
    }
    for (std::size_t i = 0; i < words.size(); ++i)
    {
      where_[words[i]] = loc_word(tier, first + i);
      tell_placed(words[i], tier, first + i);
    }
    ++generation_;
  }

  void PagedKVCache::free(PageKey key) { release_keys({key}); }

  void PagedKVCache::free_pages(const std::vector<PageKey> &keys) { release_keys(keys); }

  void PagedKVCache::release_keys(const std::vector<PageKey> &keys)
  {
    // Everything is checked before anything changes.
    std::array<std::vector<std::size_t>, kTierCount> freed; // slots, per tier
    std::vector<std::uint64_t> words;
    words.reserve(keys.size());
    for (const PageKey &k : keys)
    {
      const PageLocation at = locate(k);
      freed[at.tier].push_back(at.slot);
      words.push_back(pack(k));
    }
    if (keys.size() > 1)
    {
      std::vector<std::uint64_t> sorted = words;
      std::sort(sorted.begin(), sorted.end());
      const auto dup = std::adjacent_find(sorted.begin(), sorted.end());
      if (dup != sorted.end())
      {
        throw InvalidArgument(describe(unpack(*dup)) + " is named twice in one free");
      }
    }
    if (keys.empty())
    {
      return;
    }
    // Per tier: the holes below the kept count, filled in order by the
    // survivors above it.
    std::vector<RefPair> copies;
    for (int t = 0; t < kTierCount; ++t)
    {
      std::vector<std::size_t> &gone = freed[t];
      if (gone.empty())
      {
        continue;
      }
      Range &r = ranges_[t];
      std::sort(gone.begin(), gone.end());
      const std::size_t kept = r.owners.size() - gone.size();
      std::size_t next_gone = 0; // into gone, for slots at or above kept
      while (next_gone < gone.size() && gone[next_gone] < kept)
      {
        ++next_gone;
      }
      std::size_t above = kept;
      for (std::size_t h = 0; h < gone.size() && gone[h] < kept; ++h)
      {
        // The next surviving slot at or above `kept`.
        while (next_gone < gone.size() && gone[next_gone] == above)
        {
          ++next_gone;
          ++above;
        }
        const std::size_t hole = gone[h];
        const std::uint64_t mover = r.owners[above];
        copies.push_back({page_ref(t, static_cast<std::uint32_t>(above)),
                          page_ref(t, static_cast<std::uint32_t>(hole))});
        r.owners[hole] = mover;
        where_[mover] = loc_word(t, hole);
        tell_placed(mover, t, hole);
        ++above;
      }
      r.owners.resize(kept);
    }
    for (const std::uint64_t w : words)
    {
      where_.erase(w);
      tell_removed(w);
    }
    ++generation_;
    if (!copies.empty())
    {
      const hipStream_t stream = runtime_stream();
      launch_copy_refs(moves_upload_.send(copies, stream), static_cast<int>(copies.size()),
                       spaces(), stream);
    }
    for (int t = 0; t < kTierCount; ++t)
    {
      if (!freed[t].empty())
      {
        fit(ranges_[t], false);
      }
    }
  }

  void PagedKVCache::replace_pages(const std::vector<std::pair<PageKey, PageKey>> &pairs)
  {
    std::vector<std::uint64_t> staged;
    std::vector<PageKey> keys;
    for (const auto &[key, stage] : pairs)
    {
      if (key == stage)
      {
        throw InvalidArgument("a page cannot replace itself");
      }
      locate(stage);
      staged.push_back(pack(stage));
      keys.push_back(key);
    }
    std::sort(staged.begin(), staged.end());
    const auto dup = std::adjacent_find(staged.begin(), staged.end());
    if (dup != staged.end())
    {
      throw InvalidArgument(describe(unpack(*dup)) + " is named twice in one replace");
    }
    for (const PageKey &key : keys)
    {
      if (std::binary_search(staged.begin(), staged.end(), pack(key)))
      {
        throw InvalidArgument(describe(key) + " is both replaced and staged");
      }
    }
    release_keys(keys);
    // Each staged page now answers to the key it replaces, where it is.
    for (const auto &[key, stage] : pairs)
    {
      const auto it = where_.find(pack(stage));
      const std::uint64_t loc = it->second;
      where_.erase(it);
      tell_removed(pack(stage));
      const PageLocation at = loc_of(loc);
      where_[pack(key)] = loc;
      ranges_[at.tier].owners[at.slot] = pack(key);
      tell_placed(pack(key), at.tier, at.slot);
    }
    ++generation_;
  }

  void PagedKVCache::replace(PageKey key, PageKey staged) { replace_pages({{key, staged}}); }

  void PagedKVCache::map_to(Range &r, std::size_t count)
  {
    // Each granule is made and mapped on its own (so that each can be
    // given back on its own); the access to the whole new span is granted
    // in one call, the driver's dearest of the three.
    const std::size_t first = r.granules.size();
    const auto undo = [&]() {
      for (std::size_t g = first; g < r.granules.size(); ++g)
      {
        (void)hipMemUnmap(r.base + g * granule_, granule_);
        (void)hipMemRelease(r.granules[g]);
      }
      r.granules.resize(first);
    };
    try
    {
      while (r.granules.size() < count)
      {
        if (g_fail_granules > 0)
        {
          --g_fail_granules;
          throw OutOfMemory("hipMemCreate: out of memory (injected by the test hook)");
        }
        char *at = r.base + r.granules.size() * granule_;
        // The address may be one the releaser still holds.
        releaser_->wait_for(at);
        hipMemGenericAllocationHandle_t handle;
        hipError_t created = hipMemCreate(&handle, granule_, &prop_, 0);
        if (created == hipErrorOutOfMemory || created == hipErrorMemoryAllocation)
        {
          // Memory the releaser has yet to give back may be what is short.
          (void)hipGetLastError();
          releaser_->wait_for(nullptr);
          created = hipMemCreate(&handle, granule_, &prop_, 0);
        }
        hip_check(created, "hipMemCreate");
        const hipError_t mapped = hipMemMap(at, granule_, 0, handle, 0);
        if (mapped != hipSuccess)
        {
          (void)hipMemRelease(handle);
          hip_check(mapped, "hipMemMap");
        }
        r.granules.push_back(handle);
      }
      if (r.granules.size() > first)
      {
        hipMemAccessDesc access{};
        access.location = prop_.location;
        access.flags = hipMemAccessFlagsProtReadWrite;
        hip_check(hipMemSetAccess(r.base + first * granule_, (r.granules.size() - first) * granule_,
                                  &access, 1),
                  "hipMemSetAccess");
      }
    }
    catch (...)
    {
      undo();
      throw;
    }
  }

  void PagedKVCache::fit(Range &r, bool map_spares)
  {
    const std::size_t needed = round_up(r.owners.size() * r.page_bytes, granule_) / granule_;
    const std::size_t keep = std::min(needed + r.spare, r.reserved / granule_);
    if (r.granules.size() < needed)
    {
      map_to(r, needed);
    }
    if (map_spares && r.granules.size() < keep)
    {
      try
      {
        map_to(r, keep);
      }
      catch (const OutOfMemory &)
      {
        // A spare is room kept for later, not room a page needs now.
      }
    }
    if (r.granules.size() > keep)
    {
      std::vector<std::pair<char *, hipMemGenericAllocationHandle_t>> going;
      for (std::size_t g = keep; g < r.granules.size(); ++g)
      {
        going.emplace_back(r.base + g * granule_, r.granules[g]);
      }
      r.granules.resize(keep);
      releaser_->retire(std::move(going), runtime_stream());
    }
  }

  void PagedKVCache::keep_spare_granules(int tier, std::size_t granules)
  {
    check_tier(tier);
    Range &r = ranges_[tier];
    r.spare = granules;
    fit(r, true);
  }

  void PagedKVCache::drain_releases() { releaser_->wait_for(nullptr); }

  std::vector<PageKey> PagedKVCache::pages(int tier) const
  {
    const Range &r = ranges_.at(tier);
    std::vector<PageKey> out;
    out.reserve(r.owners.size());
    for (const std::uint64_t w : r.owners)
    {
      out.push_back(unpack(w));
    }
    return out;
  }

  void PagedKVCache::write(PageKey key, const void *host, std::size_t bytes)
  {
    char *at = address(key, bytes);
    hip_check(hipMemcpy(at, host, bytes, hipMemcpyHostToDevice), "hipMemcpy page host-to-device");
  }

  void PagedKVCache::read(PageKey key, void *host, std::size_t bytes) const
  {
    const char *at = address(key, bytes);
    hip_check(hipMemcpy(host, at, bytes, hipMemcpyDeviceToHost), "hipMemcpy page device-to-host");
  }

  char *PagedKVCache::address(PageKey key, std::size_t bytes) const
  {
    const PageLocation loc = locate(key);
    const Range &r = ranges_[loc.tier];
    if (bytes != r.page_bytes)
    {
      throw InvalidArgument(describe(key) + " holds " + std::to_string(r.page_bytes) +
                            " bytes, not " + std::to_string(bytes));
    }
    return r.base + loc.slot * r.page_bytes;
  }

  PageLocation PagedKVCache::locate(PageKey key) const
  {
    const auto it = where_.find(pack(key));
    if (it == where_.end())
    {
      throw PageNotFound(describe(key) + " is not in the page table");
    }
    return loc_of(it->second);
  }

  PageSpaces PagedKVCache::spaces() const
  {
    PageSpaces s{};
    for (int t = 0; t < kTierCount; ++t)
    {
      s.base[t] = reinterpret_cast<unsigned long long>(ranges_[t].base);
      s.bytes[t] = ranges_[t].page_bytes;
    }
    s.shadow_bytes = ranges_[kFP16].page_bytes;
    return s;
  }

  std::uint32_t PagedKVCache::ref_of(PageKey key) const
  {
    const PageLocation at = locate(key);
    if (at.slot > kRefIndexMask)
    {
      throw OutOfRange(describe(key) + " sits at slot " + std::to_string(at.slot) +
                       ", beyond what a page reference holds");
    }
    return page_ref(at.tier, static_cast<std::uint32_t>(at.slot));
  }

} // namespace mi
