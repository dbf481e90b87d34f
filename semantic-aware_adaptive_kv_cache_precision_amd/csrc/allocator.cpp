// The per-tier VMM page allocator and the device buffer, on HIP's virtual
// memory API: hipMemAddressReserve for each tier's range, hipMemCreate +
// hipMemMap + hipMemSetAccess for each granule the packed pages reach, and
// hipMemUnmap + hipMemRelease as the tail retracts, so emptied memory goes
// back to the driver where the system's memory readings see it.
//
// Semantics follow src/core_kernels/paged_kv_cache.cu of the reference
// (allocate :145-185, free :202-225, free_pages :227-359, replace(_pages)
// :361-416, fit_granules :437-470); the compaction of a batched free is one
// batched copy kernel, and every copy is ordered on the runtime stream and
// synchronised before any granule it reads is unmapped.

#include "runtime.hpp"

#include <algorithm>
#include <atomic>

namespace mi
{
  namespace
  {
    std::atomic<int> g_fail_granules{0};

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

  namespace
  {
    thread_local hipStream_t g_stream = nullptr;
  }

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

  std::size_t granule_bytes()
  {
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    return mapping_unit(device_prop(device));
  }

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
    try
    {
      for (int t = 0; t < kTierCount; ++t)
      {
        Range &r = ranges_[t];
        r.page_bytes = page_bytes[t];
        r.capacity = capacity_pages[t];
        r.reserved = round_up(page_bytes[t] * capacity_pages[t], granule_);
        if (r.reserved > 0)
        {
          void *base = nullptr;
          hip_check(hipMemAddressReserve(&base, r.reserved, granule_, nullptr, 0),
                    "hipMemAddressReserve");
          r.base = static_cast<char *>(base);
        }
      }
    }
    catch (...)
    {
      release_everything();
      throw;
    }
  }

  PagedKVCache::~PagedKVCache() { release_everything(); }

  void PagedKVCache::retire(char *at, hipMemGenericAllocationHandle_t handle)
  {
    {
      std::lock_guard<std::mutex> lock(release_mutex_);
      retired_.push_back(Retired{at, handle});
    }
    if (!releaser_.joinable())
    {
      releaser_ = std::thread([this] { release_loop(); });
    }
    release_wake_.notify_one();
  }

  void PagedKVCache::release_loop()
  {
    const hipError_t set = hipSetDevice(device_);
    std::unique_lock<std::mutex> lock(release_mutex_);
    for (;;)
    {
      release_wake_.wait(lock, [this] { return release_stop_ || !retired_.empty(); });
      if (retired_.empty())
      {
        return; // stopping, and nothing left
      }
      const Retired g = retired_.front();
      releasing_ = g.at;
      retired_.pop_front();
      lock.unlock();
      hipError_t e = set;
      if (e == hipSuccess)
      {
        e = hipMemUnmap(g.at, granule_);
      }
      const hipError_t released = hipMemRelease(g.handle);
      if (e == hipSuccess)
      {
        e = released;
      }
      lock.lock();
      releasing_ = nullptr;
      if (e != hipSuccess && release_error_.empty())
      {
        release_error_ = std::string("releasing a granule: ") + hipGetErrorString(e);
      }
      release_done_.notify_all();
    }
  }

  // Waits until the granule at `at` (or, for nullptr, every granule) given
  // up earlier is back with the driver, so that its address can be mapped
  // again; raises a failure of the release thread.
  void PagedKVCache::wait_for_release(const char *at)
  {
    std::unique_lock<std::mutex> lock(release_mutex_);
    const auto pending = [&] {
      if (at == nullptr)
      {
        return !retired_.empty() || releasing_ != nullptr;
      }
      if (releasing_ == at)
      {
        return true;
      }
      for (const Retired &g : retired_)
      {
        if (g.at == at)
        {
          return true;
        }
      }
      return false;
    };
    release_done_.wait(lock, [&] { return !pending(); });
    if (!release_error_.empty())
    {
      const std::string error = release_error_;
      release_error_.clear();
      throw DeviceError(error);
    }
  }

  void PagedKVCache::drain_releases() { wait_for_release(nullptr); }

  void PagedKVCache::release_everything() noexcept
  {
    (void)hipDeviceSynchronize();
    if (releaser_.joinable())
    {
      {
        std::lock_guard<std::mutex> lock(release_mutex_);
        release_stop_ = true;
      }
      release_wake_.notify_one();
      releaser_.join();
    }
    for (Range &r : ranges_)
    {
      while (!r.granules.empty())
      {
        const std::size_t last = r.granules.size() - 1;
        (void)hipMemUnmap(r.base + last * granule_, granule_);
        (void)hipMemRelease(r.granules.back());
        r.granules.pop_back();
      }
      if (r.base != nullptr)
      {
        (void)hipMemAddressFree(r.base, r.reserved);
        r.base = nullptr;
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

  void PagedKVCache::allocate(PageKey key, int tier)
  {
    check_tier(tier);
    if (contains(key))
    {
      throw InvalidArgument(describe(key) + " is already allocated");
    }
    Range &r = ranges_[tier];
    if (r.slots.size() == r.capacity)
    {
      throw Full(std::string(tier_name(tier)) + " is full at " + std::to_string(r.capacity) +
                 " pages");
    }
    r.slots.push_back(key);
    try
    {
      fit_granules(r, true);
    }
    catch (const OutOfMemory &e)
    {
      std::size_t free_bytes = 0, total_bytes = 0;
      const bool known = hipMemGetInfo(&free_bytes, &total_bytes) == hipSuccess;
      roll_back(r);
      throw OutOfMemory("allocating " + describe(key) + " at " + tier_name(tier) + " needed a " +
                        std::to_string(granule_) + "-byte granule: " + e.what() +
                        (known ? "; " + std::to_string(free_bytes) + " bytes were free"
                               : std::string()));
    }
    catch (...)
    {
      roll_back(r);
      throw;
    }
    table_[key] = PageLocation{tier, r.slots.size() - 1};
    ++generation_;
  }

  void PagedKVCache::roll_back(Range &r)
  {
    r.slots.pop_back();
    try
    {
      fit_granules(r, false);
    }
    catch (...)
    {
    }
  }

  void PagedKVCache::free(PageKey key)
  {
    const PageLocation loc = locate(key);
    Range &r = ranges_[loc.tier];
    const std::size_t tail = r.slots.size() - 1;
    if (loc.slot != tail)
    {
      const PageKey moved = r.slots[tail];
      hip_check(hipMemcpyAsync(r.base + loc.slot * r.page_bytes, r.base + tail * r.page_bytes,
                               r.page_bytes, hipMemcpyDeviceToDevice, runtime_stream()),
                "hipMemcpyAsync (tail swap)");
      r.slots[loc.slot] = moved;
      table_[moved].slot = loc.slot;
    }
    r.slots.pop_back();
    table_.erase(key);
    ++generation_;
    // The copy lands, and whatever read the freed granule finishes, before
    // the granule is unmapped.
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    fit_granules(r, false);
  }

  void PagedKVCache::free_pages(const std::vector<PageKey> &keys)
  {
    std::set<PageKey> freeing;
    for (const PageKey &key : keys)
    {
      locate(key);
      if (!freeing.insert(key).second)
      {
        throw InvalidArgument(describe(key) + " is named twice in one free");
      }
    }
    if (keys.empty())
    {
      return;
    }
    // Per tier: the first `kept` slots stay. A freed slot below `kept` is a
    // hole; a kept page at or above it moves into one. Copies read only slots
    // the tier gives up and write only slots it keeps.
    struct TierMoves
    {
      std::size_t kept = 0;
      std::vector<std::size_t> holes;
      std::vector<std::size_t> movers;
      bool touched = false;
    };
    std::array<TierMoves, kTierCount> moves;
    std::size_t copies = 0;
    for (int t = 0; t < kTierCount; ++t)
    {
      const Range &r = ranges_[t];
      std::size_t freed = 0;
      for (const PageKey &k : r.slots)
      {
        freed += freeing.count(k);
      }
      if (freed == 0)
      {
        continue;
      }
      TierMoves &m = moves[t];
      m.touched = true;
      m.kept = r.slots.size() - freed;
      for (std::size_t slot = 0; slot < r.slots.size(); ++slot)
      {
        const bool going = freeing.count(r.slots[slot]) != 0;
        if (slot < m.kept && going)
        {
          m.holes.push_back(slot);
        }
        else if (slot >= m.kept && !going)
        {
          m.movers.push_back(slot);
        }
      }
      copies += m.holes.size();
    }
    // Every copy's addresses, sources then destinations, tier after tier,
    // on the device before anything changes.
    std::vector<const void *> table;
    table.reserve(2 * copies);
    for (int t = 0; t < kTierCount; ++t)
    {
      const Range &r = ranges_[t];
      for (std::size_t slot : moves[t].movers)
      {
        table.push_back(r.base + slot * r.page_bytes);
      }
      for (std::size_t slot : moves[t].holes)
      {
        table.push_back(r.base + slot * r.page_bytes);
      }
    }
    std::unique_ptr<DeviceBuffer> addresses;
    if (copies > 0)
    {
      addresses = std::make_unique<DeviceBuffer>(table.size() * sizeof(void *));
      hip_check(hipMemcpy(addresses->raw(), table.data(), table.size() * sizeof(void *),
                          hipMemcpyHostToDevice),
                "hipMemcpy a free's tail moves");
    }
    // From here on nothing fails but the device.
    std::size_t at = 0;
    for (int t = 0; t < kTierCount; ++t)
    {
      Range &r = ranges_[t];
      const TierMoves &m = moves[t];
      if (!m.holes.empty())
      {
        const auto *on_device = addresses->as<const void *const>() + at;
        launch_copy_pages(on_device, const_cast<void *const *>(on_device + m.holes.size()),
                          r.page_bytes, static_cast<int>(m.holes.size()), runtime_stream());
        at += 2 * m.holes.size();
      }
      for (std::size_t i = 0; i < m.holes.size(); ++i)
      {
        const PageKey moved = r.slots[m.movers[i]];
        r.slots[m.holes[i]] = moved;
        table_[moved].slot = m.holes[i];
      }
      if (m.touched)
      {
        r.slots.resize(m.kept);
      }
    }
    for (const PageKey &key : keys)
    {
      table_.erase(key);
    }
    ++generation_;
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    for (int t = 0; t < kTierCount; ++t)
    {
      if (moves[t].touched)
      {
        fit_granules(ranges_[t], false);
      }
    }
  }

  void PagedKVCache::replace_pages(const std::vector<std::pair<PageKey, PageKey>> &pairs)
  {
    std::set<PageKey> staged;
    std::vector<PageKey> keys;
    for (const auto &[key, stage] : pairs)
    {
      if (key == stage)
      {
        throw InvalidArgument("a page cannot replace itself");
      }
      locate(stage);
      if (!staged.insert(stage).second)
      {
        throw InvalidArgument(describe(stage) + " is named twice in one replace");
      }
      keys.push_back(key);
    }
    for (const PageKey &key : keys)
    {
      if (staged.count(key) != 0)
      {
        throw InvalidArgument(describe(key) + " is both replaced and staged");
      }
    }
    free_pages(keys);
    for (const auto &[key, stage] : pairs)
    {
      const PageLocation loc = table_.at(stage);
      table_.erase(stage);
      table_[key] = loc;
      ranges_[loc.tier].slots[loc.slot] = key;
    }
    ++generation_;
  }

  void PagedKVCache::replace(PageKey key, PageKey staged)
  {
    if (key == staged)
    {
      throw InvalidArgument("a page cannot replace itself");
    }
    locate(staged);
    free(key);
    const PageLocation loc = table_.at(staged);
    table_.erase(staged);
    table_[key] = loc;
    ranges_[loc.tier].slots[loc.slot] = key;
    ++generation_;
  }

  void PagedKVCache::map_granule(Range &r)
  {
    if (g_fail_granules > 0)
    {
      --g_fail_granules;
      throw OutOfMemory("hipMemCreate: out of memory (injected by the test hook)");
    }
    char *at = r.base + r.granules.size() * granule_;
    // The address may be one a release still holds.
    wait_for_release(at);
    hipMemGenericAllocationHandle_t handle;
    hipError_t created = hipMemCreate(&handle, granule_, &prop_, 0);
    if (created == hipErrorOutOfMemory || created == hipErrorMemoryAllocation)
    {
      // Memory the release thread has yet to give back may be what is short.
      (void)hipGetLastError();
      drain_releases();
      created = hipMemCreate(&handle, granule_, &prop_, 0);
    }
    hip_check(created, "hipMemCreate");
    const hipError_t mapped = hipMemMap(at, granule_, 0, handle, 0);
    if (mapped != hipSuccess)
    {
      (void)hipMemRelease(handle);
      hip_check(mapped, "hipMemMap");
    }
    hipMemAccessDesc access{};
    access.location = prop_.location;
    access.flags = hipMemAccessFlagsProtReadWrite;
    const hipError_t set = hipMemSetAccess(at, granule_, &access, 1);
    if (set != hipSuccess)
    {
      (void)hipMemUnmap(at, granule_);
      (void)hipMemRelease(handle);
      hip_check(set, "hipMemSetAccess");
    }
    r.granules.push_back(handle);
  }

  void PagedKVCache::fit_granules(Range &r, bool map_spares)
  {
    const std::size_t needed = round_up(r.slots.size() * r.page_bytes, granule_) / granule_;
    const std::size_t kept = std::min(needed + r.spare, r.reserved / granule_);
    while (r.granules.size() < needed)
    {
      map_granule(r);
    }
    try
    {
      while (map_spares && r.granules.size() < kept)
      {
        map_granule(r);
      }
    }
    catch (const OutOfMemory &)
    {
      // A spare is room kept for later, not room this page needs.
    }
    while (r.granules.size() > kept)
    {
      const std::size_t last = r.granules.size() - 1;
      retire(r.base + last * granule_, r.granules.back());
      r.granules.pop_back();
    }
  }

  void PagedKVCache::keep_spare_granules(int tier, std::size_t granules)
  {
    check_tier(tier);
    Range &r = ranges_[tier];
    r.spare = granules;
    fit_granules(r, true);
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
    const auto it = table_.find(key);
    if (it == table_.end())
    {
      throw PageNotFound(describe(key) + " is not in the page table");
    }
    return it->second;
  }

} // namespace mi
