// The FP16 shadow store: pinned host memory mapped for the device, numbered
// shadows, and the device table of their mapped addresses that the page
// kernels read shadows through.
//
// Contract (reference: src/core_kernels/shadow_store.h:11-86): a page has at
// most one shadow, taken once and kept until the store goes; shadows pack
// into pinned allocations of whole pages. Here the store also pins ahead of
// need (reserve), so that a batch of first downgrades pins nothing on its
// own path (ADR-0015: pinning runs at about 4 GB/s and otherwise dominates
// a first downgrade).

#include "runtime.hpp"

#include <algorithm>

namespace mi
{

  ShadowStore::ShadowStore(std::size_t page_bytes) : page_bytes_(page_bytes) {}

  ShadowStore::~ShadowStore()
  {
    if (!blocks_.empty())
    {
      // A kernel may still read or write a shadow.
      (void)hipDeviceSynchronize();
    }
    for (const Block &b : blocks_)
    {
      (void)hipHostFree(b.host);
    }
  }

  void ShadowStore::reserve(std::size_t count)
  {
    const std::size_t room = pinned_pages_ - host_.size();
    if (count <= room || page_bytes_ == 0)
    {
      return;
    }
    // One block for what is missing, at least an allocation's worth.
    const std::size_t per_allocation = std::max<std::size_t>(1, kAllocationBytes / page_bytes_);
    const std::size_t pages = std::max(count - room, per_allocation);
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
    blocks_.push_back({static_cast<std::uint8_t *>(host), static_cast<std::uint8_t *>(on_device),
                       pages, 0});
    pinned_pages_ += pages;
  }

  std::uint32_t ShadowStore::add(PageKey key)
  {
    if (contains(key))
    {
      throw LogicError("page " + std::to_string(key.page) + " of layer " +
                       std::to_string(key.layer) + " has a shadow already; a page has one");
    }
    reserve(1);
    // Blocks fill in the order they were pinned.
    while (blocks_[cursor_].used == blocks_[cursor_].pages)
    {
      ++cursor_;
    }
    Block *block = &blocks_[cursor_];
    const std::size_t at = block->used++;
    const auto number = static_cast<std::uint32_t>(host_.size());
    host_.push_back(block->host + at * page_bytes_);
    device_.push_back(reinterpret_cast<unsigned long long>(block->device + at * page_bytes_));
    keys_.push_back(pack(key));
    block_of_.push_back(cursor_);
    number_[pack(key)] = number;
    return number;
  }

  void ShadowStore::truncate(std::size_t count)
  {
    while (host_.size() > count)
    {
      // The last shadow is the last used place of its block; blocks before
      // it are full, so the cursor goes back to it.
      const std::size_t b = block_of_.back();
      --blocks_[b].used;
      cursor_ = b;
      number_.erase(keys_.back());
      host_.pop_back();
      device_.pop_back();
      keys_.pop_back();
      block_of_.pop_back();
    }
    sent_ = std::min(sent_, host_.size());
  }

  void ShadowStore::take(PageKey key, const void *device_page, hipStream_t stream)
  {
    const std::uint32_t n = add(key);
    hip_check(hipMemcpyAsync(host_[n], device_page, page_bytes_, hipMemcpyDeviceToHost, stream),
              "hipMemcpyAsync a page to its FP16 shadow");
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize after a shadow copy");
  }

  std::uint32_t ShadowStore::number(PageKey key) const
  {
    const auto it = number_.find(pack(key));
    if (it == number_.end())
    {
      throw PageNotFound(describe(key) + " has no FP16 shadow");
    }
    return it->second;
  }

  const std::uint8_t *ShadowStore::shadow(PageKey key) const { return host_[number(key)]; }

  const unsigned long long *ShadowStore::device_table(hipStream_t stream)
  {
    const std::size_t n = device_.size();
    if (table_ == nullptr || table_->bytes() < n * sizeof(unsigned long long))
    {
      // A launch queued earlier may still read the old table: it is kept.
      if (table_ != nullptr)
      {
        outgrown_.push_back(std::move(table_));
      }
      table_ = std::make_unique<DeviceBuffer>(std::max<std::size_t>(2 * n, 1024) *
                                              sizeof(unsigned long long));
      sent_ = 0;
    }
    if (sent_ < n)
    {
      // Only the entries added since the last call; pageable memory is
      // staged before the call returns.
      hip_check(hipMemcpyAsync(table_->as<unsigned long long>() + sent_, device_.data() + sent_,
                               (n - sent_) * sizeof(unsigned long long), hipMemcpyHostToDevice,
                               stream),
                "hipMemcpyAsync shadow addresses");
      sent_ = n;
    }
    return table_->as<const unsigned long long>();
  }

} // namespace mi
