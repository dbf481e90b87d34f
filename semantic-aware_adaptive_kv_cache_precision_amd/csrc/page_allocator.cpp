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
//   - granules are mapped in runs (one physical allocation and one map call
//     for up to kMaxRunGranules of them): the driver's unmap costs the same
//     ~0.2 ms for a run of any length, so a range gives back a 704 MB tail
//     in six calls, not 352;
//   - whole runs the tail gives up are unmapped by the releaser thread once
//     an event recorded after the call's copies has completed, so no caller
//     waits for the driver's unmap; a run the new tail cuts is replaced, on
//     the caller's thread, by a shorter one holding the same bytes;
//   - access is granted over a range from its base only (an unmapped guard
//     granule before it) once nothing past the new end is mapped: the
//     driver refuses a span that starts where another mapping ends or that
//     a mapping follows, and then leaves the span without access;
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

  StagedPairs::~StagedPairs()
  {
    if (host_ != nullptr)
    {
      (void)hipDeviceSynchronize(); // a queued copy may still read it
      (void)hipHostFree(host_);
    }
  }

  void StagedPairs::reserve(std::size_t count)
  {
    if (count <= capacity_)
    {
      return;
    }
    if (host_ != nullptr)
    {
      (void)hipDeviceSynchronize();
      (void)hipHostFree(host_);
      host_ = nullptr;
    }
    device_.reset();
    capacity_ = 0;
    const std::size_t room = std::max<std::size_t>(count, 4096);
    void *host = nullptr;
    hip_check(hipHostMalloc(&host, room * sizeof(RefPair), 0), "hipHostMalloc page pairs");
    host_ = static_cast<RefPair *>(host);
    device_ = std::make_unique<DeviceBuffer>(room * sizeof(RefPair));
    capacity_ = room;
  }

  const RefPair *StagedPairs::send(std::size_t first, std::size_t count, hipStream_t stream)
  {
    if (first + count > capacity_)
    {
      throw LogicError("page pairs past the staged capacity");
    }
    RefPair *dst = device_->as<RefPair>() + first;
    hip_check(hipMemcpyAsync(dst, host_ + first, count * sizeof(RefPair), hipMemcpyHostToDevice,
                             stream),
              "hipMemcpyAsync page pairs");
    return dst;
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
    explicit GranuleReleaser(int device) : device_(device) {}

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

    struct Retired
    {
      char *at;
      std::size_t bytes;
      hipMemGenericAllocationHandle_t handle;
    };

    void retire(std::vector<Retired> granules, hipStream_t stream)
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
        for (const Retired &g : granules)
        {
          queue_.push_back({g.at, g.bytes, g.handle, gate});
        }
        if (!thread_.joinable())
        {
          thread_ = std::thread([this] { loop(); });
        }
      }
      wake_.notify_one();
    }

    // Waits until no run queued or being released holds an address of
    // [at, at + bytes) (at nullptr: every run is released); raises the first
    // failure of the thread.
    void wait_for(const char *at, std::size_t bytes = 0)
    {
      std::unique_lock<std::mutex> lock(mutex_);
      const auto meets = [&](const char *from, std::size_t n) {
        return from < at + bytes && at < from + n;
      };
      const auto pending = [&] {
        if (at == nullptr)
        {
          return !queue_.empty() || busy_ != nullptr;
        }
        if (busy_ != nullptr && meets(busy_, busy_bytes_))
        {
          return true;
        }
        return std::any_of(queue_.begin(), queue_.end(),
                           [&](const Item &i) { return meets(i.at, i.bytes); });
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
      std::size_t bytes;
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
        busy_bytes_ = item.bytes;
        lock.unlock();
        hipError_t e = set;
        if (e == hipSuccess && item.gate->event != nullptr)
        {
          e = hipEventSynchronize(item.gate->event);
        }
        if (e == hipSuccess)
        {
          e = hipMemUnmap(item.at, item.bytes);
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
          error_ = std::string("releasing a run of granules: ") + hipGetErrorString(e);
        }
        done_.notify_all();
      }
    }

    int device_;
    std::mutex mutex_;
    std::condition_variable wake_;
    std::condition_variable done_;
    std::deque<Item> queue_;
    const char *busy_ = nullptr;
    std::size_t busy_bytes_ = 0;
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
    releaser_ = std::make_unique<GranuleReleaser>(device_);
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
      // A guard granule, never mapped, before the range: no mapping ever
      // ends where the range begins (the driver takes a mapping that ends
      // at an address for the one that begins there when access is granted
      // from it, and refuses it when their lengths differ).
      void *base = nullptr;
      const hipError_t e = hipMemAddressReserve(&base, r.reserved + granule_, granule_, nullptr, 0);
      if (e != hipSuccess)
      {
        for (int u = 0; u < t; ++u)
        {
          if (ranges_[u].reservation != nullptr)
          {
            (void)hipMemAddressFree(ranges_[u].reservation, ranges_[u].reserved + granule_);
          }
        }
        hip_check(e, "hipMemAddressReserve");
      }
      r.reservation = static_cast<char *>(base);
      r.base = r.reservation + granule_;
    }
  }

  PagedKVCache::~PagedKVCache()
  {
    // Nothing here can be reported to a caller; a failure is dropped, and
    // the thread's last error cleared so that no later call reports it.
    (void)hipDeviceSynchronize();
    releaser_.reset(); // finishes every release queued
    for (Range &r : ranges_)
    {
      for (std::size_t i = r.runs.size(); i-- > 0;)
      {
        const Run &run = r.runs[i];
        (void)hipMemUnmap(r.base + run.first * granule_, run.count * granule_);
        (void)hipMemRelease(run.handle);
      }
      r.runs.clear();
      r.mapped = 0;
      if (r.reservation != nullptr)
      {
        (void)hipMemAddressFree(r.reservation, r.reserved + granule_);
      }
    }
    split_buffer_.reset();
    (void)hipGetLastError();
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
    if (!copies.empty() && deferred_copies_ != nullptr)
    {
      deferred_copies_->insert(deferred_copies_->end(), copies.begin(), copies.end());
    }
    else if (!copies.empty())
    {
      const hipStream_t stream = runtime_stream();
      const RefPair *uploaded =
          copies.size() > static_cast<std::size_t>(kHeldRefs) ? moves_upload_.send(copies, stream)
                                                              : nullptr;
      launch_copy_refs(ref_list(copies, 0, copies.size(), uploaded), static_cast<int>(copies.size()),
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

  hipMemGenericAllocationHandle_t PagedKVCache::create_physical(std::size_t granules)
  {
    if (g_fail_granules > 0)
    {
      --g_fail_granules;
      throw OutOfMemory("hipMemCreate: out of memory (injected by the test hook)");
    }
    hipMemGenericAllocationHandle_t handle;
    hipError_t created = hipMemCreate(&handle, granules * granule_, &prop_, 0);
    if (created == hipErrorOutOfMemory || created == hipErrorMemoryAllocation)
    {
      // Memory the releaser has yet to give back may be what is short.
      (void)hipGetLastError();
      releaser_->wait_for(nullptr);
      created = hipMemCreate(&handle, granules * granule_, &prop_, 0);
    }
    hip_check(created, "hipMemCreate");
    return handle;
  }

  void PagedKVCache::map_to(Range &r, std::size_t count)
  {
    // A run the tail cut still holds its granules: those are counted back
    // first. Then the new granules in runs of up to kMaxRunGranules, each
    // one physical allocation mapped by one call; access is then granted in
    // one call over the range from its base.
    const std::size_t first_run = r.runs.size();
    const std::size_t first = r.mapped;
    const auto undo = [&]() {
      for (std::size_t i = first_run; i < r.runs.size(); ++i)
      {
        const Run &run = r.runs[i];
        (void)hipMemUnmap(r.base + run.first * granule_, run.count * granule_);
        (void)hipMemRelease(run.handle);
      }
      r.runs.resize(first_run);
      r.mapped = first;
    };
    try
    {
      r.mapped = std::max(r.mapped, std::min(count, r.runs_end()));
      const std::size_t held = r.mapped;
      while (r.mapped < count)
      {
        const std::size_t n = std::min(count - r.mapped, kMaxRunGranules);
        char *at = r.base + r.mapped * granule_;
        // The addresses may be ones the releaser still holds.
        releaser_->wait_for(at, n * granule_);
        const hipMemGenericAllocationHandle_t handle = create_physical(n);
        const hipError_t mapped = hipMemMap(at, n * granule_, 0, handle, 0);
        if (mapped != hipSuccess)
        {
          (void)hipMemRelease(handle);
          hip_check(mapped, "hipMemMap");
        }
        r.runs.push_back({r.mapped, n, handle});
        r.mapped += n;
      }
      if (r.mapped > held)
      {
        grant_access(r, held, r.mapped);
      }
    }
    catch (...)
    {
      undo();
      throw;
    }
  }

  void PagedKVCache::grant_access(Range &r, std::size_t from, std::size_t granules)
  {
    hipMemAccessDesc access{};
    access.location = prop_.location;
    access.flags = hipMemAccessFlagsProtReadWrite;
    // The driver grants access over a span only where no mapping ends at
    // its start and none lies past its end: it is granted from the range's
    // base (which has an unmapped guard granule before it) once every run
    // given up before has been unmapped.
    releaser_->wait_for(nullptr);
    hip_check(hipMemSetAccess(r.base, granules * granule_, &access, 1), "hipMemSetAccess");
    // Every new run reads and writes before any page there is used.
    for (const Run &run : r.runs)
    {
      if (run.first + run.count <= from)
      {
        continue;
      }
      for (const std::size_t g : {run.first, run.first + run.count - 1})
      {
        unsigned long long flags = 0;
        hip_check(hipMemGetAccess(&flags, &prop_.location, r.base + g * granule_),
                  "hipMemGetAccess");
        if (flags != hipMemAccessFlagsProtReadWrite)
        {
          throw DeviceError("granule " + std::to_string(g) + " of a range is mapped without "
                            "read and write access");
        }
      }
    }
  }

  void PagedKVCache::split_run(Range &r, std::size_t keep)
  {
    Run &run = r.runs.back();
    const std::size_t n = keep - run.first;
    char *at = r.base + run.first * granule_;
    // The caller synchronised the device: nothing reads or writes the run
    // while, for a moment, its addresses hold nothing. The shorter run's
    // memory is made first, so that a failure changes nothing.
    hipMemGenericAllocationHandle_t handle;
    try
    {
      handle = create_physical(n);
      if (split_buffer_ == nullptr)
      {
        split_buffer_ = std::make_unique<DeviceBuffer>(kMaxRunGranules * granule_);
      }
    }
    catch (const std::exception &)
    {
      // No room for the shorter copy: the run stays whole and cut, its
      // granules past `keep` given back when a later settle can make it.
      return;
    }
    hipError_t e = hipMemcpy(split_buffer_->raw(), at, n * granule_, hipMemcpyDeviceToDevice);
    if (e != hipSuccess)
    {
      (void)hipMemRelease(handle);
      hip_check(e, "hipMemcpy a split run's bytes out");
    }
    // The old run goes; the new one takes its place at the same addresses.
    e = hipMemUnmap(at, run.count * granule_);
    if (e != hipSuccess)
    {
      (void)hipMemRelease(handle);
      hip_check(e, "hipMemUnmap a split run");
    }
    (void)hipMemRelease(run.handle);
    e = hipMemMap(at, n * granule_, 0, handle, 0);
    if (e != hipSuccess)
    {
      // The driver failed between the two mappings: the run is gone.
      (void)hipMemRelease(handle);
      r.mapped = run.first;
      r.runs.pop_back();
      hip_check(e, "hipMemMap a split run");
    }
    run.handle = handle;
    run.count = n;
    r.mapped = keep;
    grant_access(r, run.first, keep);
    hip_check(hipMemcpy(at, split_buffer_->raw(), n * granule_, hipMemcpyDeviceToDevice),
              "hipMemcpy a split run's bytes back");
  }

  void PagedKVCache::retract(Range &r, std::size_t keep)
  {
    std::vector<GranuleReleaser::Retired> going;
    while (!r.runs.empty() && r.runs.back().first >= keep)
    {
      const Run &run = r.runs.back();
      going.push_back({r.base + run.first * granule_, run.count * granule_, run.handle});
      r.runs.pop_back();
    }
    // A run that `keep` cuts stays whole (its bytes past `keep` are past
    // the tail) until settle_cuts; the granules are no longer counted.
    r.mapped = std::min(r.mapped, keep);
    if (deferred_copies_ != nullptr)
    {
      // The caller's launch may still read them: released after it.
      for (const GranuleReleaser::Retired &run : going)
      {
        deferred_runs_.push_back({run.at, run.bytes, run.handle});
      }
      return;
    }
    // Whole runs go off the caller's path, once the launches queued so far
    // (which may read them) are done.
    releaser_->retire(std::move(going), runtime_stream());
  }

  void PagedKVCache::finish_deferred()
  {
    deferred_copies_ = nullptr;
    std::vector<GranuleReleaser::Retired> going;
    for (const HeldRun &run : deferred_runs_)
    {
      going.push_back({run.at, run.bytes, run.handle});
    }
    deferred_runs_.clear();
    releaser_->retire(std::move(going), runtime_stream());
  }

  void PagedKVCache::settle_cuts()
  {
    bool cut = false;
    for (const Range &r : ranges_)
    {
      cut = cut || r.runs_end() > r.mapped;
    }
    if (!cut)
    {
      return;
    }
    // Nothing may read or write a cut run while, for a moment, its
    // addresses hold nothing; and access is granted over a range only once
    // nothing is mapped past it (the runs given up are unmapped first).
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize before a cut run is settled");
    releaser_->wait_for(nullptr);
    for (Range &r : ranges_)
    {
      if (r.runs_end() > r.mapped)
      {
        split_run(r, r.mapped);
      }
    }
  }

  void PagedKVCache::fit(Range &r, bool map_spares)
  {
    const std::size_t needed = round_up(r.owners.size() * r.page_bytes, granule_) / granule_;
    const std::size_t keep = std::min(needed + r.spare, r.reserved / granule_);
    if (r.mapped < needed)
    {
      map_to(r, needed);
    }
    if (map_spares && r.mapped < keep)
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
    if (r.mapped > keep)
    {
      retract(r, keep);
    }
  }

  void PagedKVCache::keep_spare_granules(int tier, std::size_t granules)
  {
    check_tier(tier);
    Range &r = ranges_[tier];
    r.spare = granules;
    fit(r, true);
  }

  void PagedKVCache::drain_releases()
  {
    releaser_->wait_for(nullptr);
    settle_cuts();
  }

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
