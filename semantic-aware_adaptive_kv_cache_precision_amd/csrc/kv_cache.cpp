// KVPages, the cache manager: pages reserved per layer, rows stored and
// sealed, decode and chunk attention over the page tables, tier moves.
//
// Contract (reference: src/core_kernels/kv_pages.h and kv_pages.cu): a page
// is born at its tier (the tier map's, else the cache's) and sealed when its
// last row arrives; a cache that seals keeps each layer's partial page in
// one of two FP16 open pages; a page at tier T always holds quantise_page of
// its FP16 rows at T, and a page back at FP16 its FP16 shadow; a batch of
// moves leaves every byte, tier and shadow as the same moves one at a time;
// a refused call changes nothing.
//
// How it is done here (this build's own design):
//   - page tables: the device copy is edited, not rebuilt. The allocator
//     reports each page whose slot changes (PlacementObserver); the cache
//     sets that entry in a host mirror and marks it, and the next launch
//     that reads the tables first sends the marked entries (one small copy
//     and a scatter launch, or the whole table when that is smaller);
//   - a store is one launch: every page it seals (quantised at its birth
//     tier from the open page's rows and the rows just brought, or copied at
//     FP16) and the rows it leaves in an open page, as row jobs passed by
//     value;
//   - a batch of moves sends the device 8 bytes a page pair: 32-bit
//     references to a tier slot or a shadow number, from which the kernels
//     form addresses; shadows out, restores, one quantise launch per target
//     tier, then the allocator's compaction, all queued on one stream with
//     one wait at the end; the single-page downgrade and upgrade are a batch
//     of one.

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
  } // namespace

  // ---- PageTable --------------------------------------------------------------------

  void PageTable::ensure(int pages)
  {
    if (pages <= stride_)
    {
      return;
    }
    const int grown = std::max(pages, 2 * stride_);
    std::vector<unsigned long long> address(static_cast<std::size_t>(layers_) * grown, 0);
    std::vector<std::uint8_t> tier(address.size(), kUnreadPage);
    for (int l = 0; l < layers_; ++l)
    {
      std::copy_n(address_.begin() + static_cast<std::ptrdiff_t>(l) * stride_, stride_,
                  address.begin() + static_cast<std::ptrdiff_t>(l) * grown);
      std::copy_n(tier_.begin() + static_cast<std::ptrdiff_t>(l) * stride_, stride_,
                  tier.begin() + static_cast<std::ptrdiff_t>(l) * grown);
    }
    address_.swap(address);
    tier_.swap(tier);
    stride_ = grown;
    dirty_.assign(address_.size(), 0);
    marked_.clear();
    // The device copy is made anew, whole (the old one may still be read by
    // a queued launch: its free waits for the device).
    device_.reset();
    device_ = std::make_unique<DeviceBuffer>(address_.size() * (sizeof(unsigned long long) + 1));
    whole_ = true;
  }

  void PageTable::set(int layer, int page, unsigned long long address, std::uint8_t tier)
  {
    const std::size_t at = static_cast<std::size_t>(layer) * stride_ + page;
    address_[at] = address;
    tier_[at] = tier;
    if (!whole_ && !dirty_[at])
    {
      dirty_[at] = 1;
      marked_.push_back(static_cast<std::uint32_t>(at));
    }
  }

  void PageTable::commit(hipStream_t stream)
  {
    if (device_ == nullptr)
    {
      return;
    }
    const std::size_t n = address_.size();
    // An edit is 16 bytes and a launch; the whole table 9 bytes an entry.
    if (!whole_ && marked_.size() * 16 > n * 9)
    {
      whole_ = true;
    }
    if (whole_)
    {
      hip_check(hipMemcpyAsync(device_->raw(), address_.data(), n * sizeof(unsigned long long),
                               hipMemcpyHostToDevice, stream),
                "hipMemcpyAsync page addresses");
      hip_check(hipMemcpyAsync(device_->as<unsigned long long>() + n, tier_.data(), n,
                               hipMemcpyHostToDevice, stream),
                "hipMemcpyAsync page tiers");
      whole_ = false;
    }
    else if (!marked_.empty())
    {
      std::vector<TableEdit> edits;
      edits.reserve(marked_.size());
      for (const std::uint32_t at : marked_)
      {
        edits.push_back({address_[at], at, tier_[at]});
      }
      launch_table_edits(edit_upload_.send(edits, stream), static_cast<int>(edits.size()),
                         device_->as<unsigned long long>(),
                         reinterpret_cast<std::uint8_t *>(device_->as<unsigned long long>() + n),
                         stream);
    }
    for (const std::uint32_t at : marked_)
    {
      dirty_[at] = 0;
    }
    marked_.clear();
  }

  // ---- KVPages: set-up --------------------------------------------------------------

  bool KVPages::seals_for(int tier, const TierMap &tier_map, bool always_seal)
  {
    // Only a cache all of whose pages stay FP16 can leave its last page in
    // the page table, partly written.
    if (always_seal || tier != kFP16)
    {
      return true;
    }
    return std::any_of(tier_map.begin(), tier_map.end(), [tier](const std::vector<int> &row) {
      return std::any_of(row.begin(), row.end(), [tier](int t) { return t != tier; });
    });
  }

  KVPages::KVPages(PagedKVCache &allocator, int layers, int page_tokens, int kv_heads,
                   int head_dim, int tier, Halves halves, TierMap tier_map, bool always_seal)
      : allocator_(allocator), layers_(layers), page_tokens_(page_tokens), kv_heads_(kv_heads),
        head_dim_(head_dim), kv_width_(static_cast<std::size_t>(std::max(kv_heads, 0)) *
                                       std::max(head_dim, 0)),
        tier_(tier), halves_(halves),
        storage_tier_(tier != kFP16 && halves != Halves::kBoth ? kFP16 : tier),
        tier_map_(std::move(tier_map)), shadows_(fp16_page_bytes(std::max(page_tokens, 0), kv_width_)),
        table_(std::max(layers, 0))
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
      for (const int t : row)
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
      // The diagnostic's round trip needs the tier's layout.
      page_layout(tier, page_tokens, kv_heads, head_dim);
    }
    current_open_.assign(layers, 0);
    attend_open_.assign(layers, 0);
    sealed_.assign(layers, 0);
    open_address_.assign(2 * static_cast<std::size_t>(layers), 0);
    allocator_.watch(this);
  }

  KVPages::~KVPages()
  {
    allocator_.unwatch(this);
    try
    {
      // Every page in one free: the ranges retract once, whole runs going.
      std::vector<PageKey> held;
      for (int page = pages_ - 1; page >= 0; --page)
      {
        for (int layer = layers_ - 1; layer >= 0; --layer)
        {
          if (!evicted({layer, page}))
          {
            held.push_back({layer, page});
          }
        }
      }
      if (open_pages_)
      {
        for (int k = 1; k >= 0; --k)
        {
          for (int layer = layers_ - 1; layer >= 0; --layer)
          {
            held.push_back({layer, kOpenPages[k]});
          }
        }
      }
      allocator_.free_pages(held);
    }
    catch (...)
    {
    }
    for (hipEvent_t e : move_events_)
    {
      if (e != nullptr)
      {
        (void)hipEventDestroy(e);
      }
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

  std::string KVPages::page_name(PageKey key)
  {
    return "page " + std::to_string(key.page) + " of layer " + std::to_string(key.layer);
  }

  // ---- the tables follow the allocator ------------------------------------------------

  void KVPages::placed(PageKey key, int tier, std::size_t slot)
  {
    if (key.layer < 0 || key.layer >= layers_)
    {
      return;
    }
    const auto address =
        reinterpret_cast<unsigned long long>(allocator_.address_of({tier, slot}));
    if (key.page == kOpenPages[0] || key.page == kOpenPages[1])
    {
      open_address_[2 * static_cast<std::size_t>(key.layer) + (key.page == kOpenPages[0] ? 0 : 1)] =
          address;
      return;
    }
    if (key.page >= 0 && key.page < table_.stride())
    {
      const bool unread = flag(key, kMasked) || flag(key, kEvicted);
      table_.set(key.layer, key.page, address,
                 unread ? kUnreadPage : static_cast<std::uint8_t>(tier));
    }
  }

  void KVPages::removed(PageKey key)
  {
    if (key.layer >= 0 && key.layer < layers_ && key.page >= 0 && key.page < table_.stride())
    {
      table_.set(key.layer, key.page, 0, kUnreadPage);
    }
  }

  void KVPages::set_flag(PageKey key, std::uint8_t bit)
  {
    flags_[static_cast<std::size_t>(key.layer) * flag_stride_ + key.page] |= bit;
  }

  void KVPages::grow(int pages)
  {
    if (pages > flag_stride_)
    {
      const int grown = std::max(pages, 2 * flag_stride_);
      std::vector<std::uint8_t> flags(static_cast<std::size_t>(layers_) * grown, 0);
      for (int l = 0; l < layers_; ++l)
      {
        std::copy_n(flags_.begin() + static_cast<std::ptrdiff_t>(l) * flag_stride_, flag_stride_,
                    flags.begin() + static_cast<std::ptrdiff_t>(l) * grown);
      }
      flags_.swap(flags);
      flag_stride_ = grown;
    }
    const int old_stride = table_.stride();
    table_.ensure(pages);
    if (table_.stride() != old_stride)
    {
      // A new table: every page held so far written into it.
      for (int l = 0; l < layers_; ++l)
      {
        for (int p = 0; p < pages_; ++p)
        {
          refresh_entry(l, p);
        }
      }
    }
  }

  void KVPages::refresh_entry(int layer, int page)
  {
    const PageKey key{layer, page};
    if (!allocator_.contains(key))
    {
      table_.set(layer, page, 0, kUnreadPage);
      return;
    }
    const PageLocation at = allocator_.locate(key);
    table_.set(layer, page, reinterpret_cast<unsigned long long>(allocator_.address_of(at)),
               masked(key) ? kUnreadPage : static_cast<std::uint8_t>(at.tier));
  }

  void KVPages::sync_tables(hipStream_t stream) { table_.commit(stream); }

  // ---- reserve and store ---------------------------------------------------------------

  void KVPages::reserve(int tokens)
  {
    const int needed = seals_ ? tokens / page_tokens_ : (tokens + page_tokens_ - 1) / page_tokens_;
    // Table room first, so the allocator's reports land in it.
    grow(std::max(needed, pages_));
    // Open pages (all of the first, then all of the second), then each new
    // page of positions for every layer, at its birth tier; the pages of one
    // tier are allocated in this order in one call.
    std::vector<PageKey> taken;
    try
    {
      if (seals_ && !open_pages_ && tokens > 0)
      {
        std::vector<PageKey> open;
        for (const int page : kOpenPages)
        {
          for (int layer = 0; layer < layers_; ++layer)
          {
            open.push_back({layer, page});
          }
        }
        allocator_.allocate_run(open, kFP16);
        taken.insert(taken.end(), open.begin(), open.end());
      }
      std::array<std::vector<PageKey>, kTierCount> runs;
      for (int page = pages_; page < needed; ++page)
      {
        for (int layer = 0; layer < layers_; ++layer)
        {
          runs[birth_tier(layer, page)].push_back({layer, page});
        }
      }
      for (int t = 0; t < kTierCount; ++t)
      {
        allocator_.allocate_run(runs[t], t);
        taken.insert(taken.end(), runs[t].begin(), runs[t].end());
      }
    }
    catch (...)
    {
      // Every page taken is its tier's latest: giving them back moves none.
      allocator_.free_pages(taken);
      throw;
    }
    if (seals_ && tokens > 0)
    {
      open_pages_ = true;
    }
    pages_ = std::max(needed, pages_);
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
    const hipStream_t stream = runtime_stream();
    if (seals_)
    {
      store_sealed(layer, static_cast<const std::uint16_t *>(keys),
                   static_cast<const std::uint16_t *>(values), start, n);
      return;
    }
    sync_tables(stream);
    launch_store_pages(keys, values, table_.addresses() + static_cast<std::size_t>(layer) * table_.stride(),
                       page_tokens_, kv_width_, start, n, stream);
  }

  void KVPages::store_sealed(int layer, const std::uint16_t *keys, const std::uint16_t *values,
                             int start, int n)
  {
    const std::size_t W = kv_width_;
    const std::size_t half = static_cast<std::size_t>(page_tokens_) * W;
    const int cur = current_open_[layer];
    attend_open_[layer] = cur;
    const int first_span = start / page_tokens_;
    const int end = start + n;
    std::vector<RowJob> jobs;
    for (int span = first_span; span * page_tokens_ < end; ++span)
    {
      const int span_start = span * page_tokens_;
      const int a = std::max(start, span_start);
      const int b = std::min(end, span_start + page_tokens_);
      const std::uint16_t *k_rows = keys + static_cast<std::size_t>(a - start) * W;
      const std::uint16_t *v_rows = values + static_cast<std::size_t>(a - start) * W;
      RowJob j{};
      if (b == span_start + page_tokens_)
      {
        // The page's last row is here: it is sealed from the rows the open
        // page holds before `a` and the rows brought from `a` on.
        const PageKey key{layer, span};
        const PageLocation at = allocator_.locate(key);
        const std::uint16_t *open = open_page(layer, cur);
        j.k_lo = open;
        j.v_lo = open + half;
        j.k_hi = k_rows;
        j.v_hi = v_rows;
        j.split = a - span_start;
        j.dst = reinterpret_cast<std::uint8_t *>(allocator_.address_of(at));
        j.tier = halves_ != Halves::kBoth ? tier_ : at.tier;
        if (halves_ == Halves::kKeys)
        {
          j.kind = static_cast<int>(RowJobKind::kRoundKeys);
        }
        else if (halves_ == Halves::kValues)
        {
          j.kind = static_cast<int>(RowJobKind::kRoundValues);
        }
        else
        {
          j.kind = static_cast<int>(at.tier == kFP16 ? RowJobKind::kCopy : RowJobKind::kQuantise);
        }
        sealed_[layer] = std::max(sealed_[layer], span + 1);
      }
      else
      {
        // A partial page: its rows wait in an open page, the current one if
        // the page was begun before this store, else the other.
        const int which = span == first_span ? cur : 1 - cur;
        j.kind = static_cast<int>(RowJobKind::kFill);
        j.k_lo = j.k_hi = k_rows;
        j.v_lo = j.v_hi = v_rows;
        j.split = 0;
        j.rows = b - a;
        j.dst_row = a - span_start;
        j.dst = reinterpret_cast<std::uint8_t *>(open_page(layer, which));
        j.tier = kFP16;
        current_open_[layer] = which;
      }
      jobs.push_back(j);
    }
    launch_row_jobs(jobs.data(), static_cast<int>(jobs.size()), page_tokens_, kv_heads_,
                    head_dim_, runtime_stream());
  }

  // ---- evict, mask ---------------------------------------------------------------------

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

  void KVPages::evict(int layer, int page)
  {
    const PageKey key = require_held(layer, page, "evict");
    if (masked(key))
    {
      throw InvalidArgument(page_name(key) +
                            " is masked, the reference an eviction is measured against; evict "
                            "another cache's page");
    }
    set_flag(key, kEvicted);
    allocator_.free(key); // its entry turns unread as the allocator reports it gone
  }

  void KVPages::mask(int layer, int page)
  {
    const PageKey key = require_held(layer, page, "mask");
    set_flag(key, kMasked);
    refresh_entry(layer, page);
  }

  // ---- tier moves ----------------------------------------------------------------------

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
    require_page_size(target, "a page of positions");
    hip_check(hipStreamSynchronize(runtime_stream()), "hipStreamSynchronize before a move");
    const Clock::time_point began = Clock::now();
    double shadow_seconds = 0.0;
    run_moves({key}, {current}, {target}, &shadow_seconds);
    last_move_ = MoveRecord{key, current, target, bytes_at(current), bytes_at(target),
                            since(began), shadow_seconds};
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
    require_page_size(target, "a page of positions");
    hip_check(hipStreamSynchronize(runtime_stream()), "hipStreamSynchronize before a move");
    const Clock::time_point began = Clock::now();
    double shadow_seconds = 0.0;
    run_moves({key}, {current}, {target}, &shadow_seconds);
    last_move_ = MoveRecord{key, current, target, bytes_at(current), bytes_at(target),
                            since(began), shadow_seconds};
  }

  void KVPages::move_pages(const std::vector<PageMove> &moves)
  {
    const hipStream_t stream = runtime_stream();
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize before a batch");
    const Clock::time_point began = Clock::now();
    const std::size_t n = moves.size();
    std::vector<PageKey> keys;
    std::vector<int> from, targets;
    keys.reserve(n);
    from.reserve(n);
    targets.reserve(n);
    // A large batch's first downgrades: each page's shadow is numbered as
    // the page is validated, and every kShadowPiece of them start over the
    // host link at once, so that the link (the batch's bound) is busy while
    // the host validates and plans the rest. A later refusal forgets the
    // shadows (the copies into their places are harmless: the places are
    // free again, and a later copy into one is ordered after them).
    constexpr std::size_t kShadowPiece = 1024;
    const bool early_shadows = n >= 256;
    const std::size_t shadows_before = shadows_.count();
    if (early_shadows)
    {
      shadow_pairs_.reserve(n);
    }
    std::size_t staged = 0, sent = 0;
    const auto send_shadows = [&]() {
      PageSpaces spaces = allocator_.spaces();
      spaces.shadows = shadows_.device_table(stream);
      RefList l{};
      l.pairs = shadow_pairs_.send(sent, staged - sent, stream);
      launch_copy_refs(l, static_cast<int>(staged - sent), spaces, stream);
      sent = staged;
    };
    // Pages named so far, one bit a (layer, page) position.
    const std::size_t stride = static_cast<std::size_t>(pages_);
    std::vector<std::uint64_t> named((static_cast<std::size_t>(layers_) * stride + 63) / 64, 0);
    try
    {
      for (const PageMove &m : moves)
      {
        const PageKey key = require_held(m.key.layer, m.key.page, "move");
        if (m.target < 0 || m.target >= kTierCount)
        {
          throw InvalidArgument("tier " + std::to_string(m.target) + " is not one of the four");
        }
        const std::size_t bit = static_cast<std::size_t>(key.layer) * stride + key.page;
        if ((named[bit / 64] >> (bit % 64)) & 1u)
        {
          throw InvalidArgument(page_name(key) +
                                " is named twice in one batch; a batch moves a page once, to the "
                                "tier it ends at");
        }
        named[bit / 64] |= std::uint64_t{1} << (bit % 64);
        const int now = page_tier(key);
        if (now == m.target)
        {
          throw InvalidArgument(page_name(key) + " is already at " + tier_name(now));
        }
        if (now != kFP16 && !shadows_.contains(key))
        {
          throw InvalidArgument(page_name(key) + " was born at " + tier_name(now) +
                                " and has no FP16 shadow to move from; only a page sealed at "
                                "FP16 moves");
        }
        require_page_size(m.target, "a page of positions");
        keys.push_back(key);
        from.push_back(now);
        targets.push_back(m.target);
        if (early_shadows && now == kFP16 && !shadows_.contains(key))
        {
          shadow_pairs_.host()[staged++] = {allocator_.ref_of(key),
                                            page_ref(kShadowSpace, shadows_.add(key))};
          if (staged - sent == kShadowPiece)
          {
            send_shadows();
          }
        }
      }
      if (staged > sent)
      {
        send_shadows();
      }
      if (!keys.empty())
      {
        run_moves(keys, from, targets, nullptr);
      }
    }
    catch (...)
    {
      shadows_.truncate(shadows_before);
      throw;
    }
    last_batch_ = BatchRecord{keys.size(), shadows_.count() - shadows_before, since(began),
                              phases_[0], phases_[1], phases_[2]};
  }

  bool KVPages::run_one_move(PageKey key, int from, int target, double *shadow_seconds)
  {
    if (!move_one_applies(from, target, page_tokens_, kv_heads_, head_dim_))
    {
      return false;
    }
    const hipStream_t stream = runtime_stream();
    const bool first_downgrade = from == kFP16 && !shadows_.contains(key);
    shadows_.reserve(first_downgrade ? 1 : 0);
    // The page's FP16 rows (the page itself, or its shadow) and, before its
    // first downgrade, its shadow's place. A quantised page's rows are its
    // shadow's: copied as they are to FP16, or staged in device memory
    // first for a quantised tier.
    const std::size_t fp16_bytes = bytes_at(kFP16);
    if (from != kFP16 && target != kFP16 &&
        (staging_ == nullptr || staging_->bytes() < fp16_bytes))
    {
      staging_.reset(); // waits for launches that may read the old one
      staging_ = std::make_unique<DeviceBuffer>(fp16_bytes);
    }
    const std::size_t shadows_before = shadows_.count();
    OneMove m{};
    if (from == kFP16)
    {
      m.page.from = allocator_.ref_of(key);
      if (first_downgrade)
      {
        m.has_shadow = 1;
        m.shadow = {m.page.from, page_ref(kShadowSpace, shadows_.add(key))};
        m.shadow_at = shadows_.device_address(m.shadow.to & kRefIndexMask);
      }
    }
    else
    {
      m.page.from = page_ref(kShadowSpace, shadows_.number(key));
      if (target != kFP16)
      {
        m.has_stage = 1;
        m.stage = {m.page.from, page_ref(kStagingSpace, 0)};
        m.page.from = m.stage.to;
      }
    }
    m.tier = target;
    // The new page at the target tier's tail, under a staging key; a page
    // that landed anywhere else is refused before the device names it.
    const PageKey staged{key.layer, kBatchStagingPage};
    m.page.to = page_ref(target, static_cast<std::uint32_t>(allocator_.held(target)));
    try
    {
      allocator_.allocate_run({staged}, target, false);
      if (allocator_.ref_of(staged) != m.page.to)
      {
        allocator_.free(staged);
        throw LogicError("a staged page did not land in the slot its move named");
      }
    }
    catch (...)
    {
      shadows_.truncate(shadows_before);
      throw;
    }
    PageSpaces spaces = allocator_.spaces();
    // The shadow table is brought up to date only for a move that reads a
    // shadow (its upload from pageable memory costs a first downgrade, which
    // writes its new shadow by address, a few microseconds); later launches
    // that read shadows send what is pending first.
    spaces.shadows = from != kFP16 ? shadows_.device_table(stream) : nullptr;
    spaces.staging = staging_ ? reinterpret_cast<unsigned long long>(staging_->raw()) : 0;
    // The page table names the new page and the old one goes; its tier's
    // compaction copies ride in the move's launch, after the reads of the
    // old page, and the granules that tier gives up are released after it.
    std::vector<RefPair> compaction;
    allocator_.defer_copies(&compaction);
    try
    {
      allocator_.replace_pages({{key, staged}});
    }
    catch (...)
    {
      allocator_.finish_deferred();
      throw;
    }
    may_be_at_[target] = true;
    const std::size_t held = std::min<std::size_t>(compaction.size(), kHeldRefs);
    m.compact_count = static_cast<int>(held);
    for (std::size_t i = 0; i < held; ++i)
    {
      m.compact[i] = compaction[i];
    }
    try
    {
      // The shadow's time (the launch's device time) is reported for a move
      // that writes or reads a shadow only: the events cost ~1.3 us of host
      // time a move, so no other move records them.
      const bool touches_shadow = first_downgrade || from != kFP16;
      const bool timed = shadow_seconds != nullptr && touches_shadow;
      if (timed)
      {
        ensure_move_events();
        hip_check(hipEventRecord(move_events_[0], stream), "hipEventRecord before a move");
      }
      if (!launch_move_one(m, spaces, page_tokens_, kv_heads_, head_dim_, stream))
      {
        throw LogicError("a single move's launch refused a shape move_one_applies took");
      }
      if (timed)
      {
        hip_check(hipEventRecord(move_events_[1], stream), "hipEventRecord after a move");
      }
      if (compaction.size() > held)
      {
        // More than a launch holds (never for one free): the rest after it.
        const std::vector<RefPair> rest(compaction.begin() + held, compaction.end());
        const RefPair *up = rest.size() > kHeldRefs ? pairs_upload_.send(rest, stream) : nullptr;
        launch_copy_refs(ref_list(rest, 0, rest.size(), up), static_cast<int>(rest.size()),
                         spaces, stream);
      }
    }
    catch (...)
    {
      allocator_.finish_deferred();
      throw;
    }
    allocator_.finish_deferred();
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize after a move");
    if (shadow_seconds != nullptr)
    {
      // The launch that takes the shadow also makes the page: its device
      // time, when it takes one.
      float ms = 0.0f;
      if (first_downgrade || from != kFP16)
      {
        hip_check(hipEventElapsedTime(&ms, move_events_[0], move_events_[1]),
                  "hipEventElapsedTime of a move");
      }
      *shadow_seconds = ms * 1e-3;
    }
    return true;
  }

  void KVPages::run_moves(const std::vector<PageKey> &keys, const std::vector<int> &from,
                          const std::vector<int> &targets, double *shadow_seconds)
  {
    if (keys.size() == 1 && run_one_move(keys[0], from[0], targets[0], shadow_seconds))
    {
      return;
    }
    const hipStream_t stream = runtime_stream();
    const std::size_t n = keys.size();
    const Clock::time_point entered = Clock::now();
    // 1. Pinned room for the shadows first downgrades take (nothing, if it
    // was pinned ahead). A failure here changes nothing.
    std::size_t first_downgrades = 0;
    for (std::size_t i = 0; i < n; ++i)
    {
      first_downgrades += from[i] == kFP16 && !shadows_.contains(keys[i]);
    }
    shadows_.reserve(first_downgrades);

    // 2. Every new page under a staging key of its own, a tier's pages in
    // one allocator call later. A run is appended at its tier's tail, so
    // the slots the new pages will take are known now: the device's work is
    // named by page reference before the host allocates, and the shadows
    // start over the host link while it does.
    std::vector<PageKey> staged(n);
    std::array<std::vector<PageKey>, kTierCount> runs;
    std::array<std::size_t, kTierCount> next{};
    for (int t = 0; t < kTierCount; ++t)
    {
      next[t] = allocator_.held(t);
    }
    std::vector<std::uint32_t> to(n);
    for (std::size_t i = 0; i < n; ++i)
    {
      staged[i] = {keys[i].layer, kBatchStagingPage - static_cast<int>(i)};
      runs[targets[i]].push_back(staged[i]);
      to[i] = page_ref(targets[i], static_cast<std::uint32_t>(next[targets[i]]++));
    }
    for (int t = 0; t < kTierCount; ++t)
    {
      if (next[t] > kRefIndexMask)
      {
        throw OutOfRange(std::string("a batch would take ") + tier_name(t) + " past slot " +
                         std::to_string(kRefIndexMask) + ", beyond what a page reference holds");
      }
    }

    // The device's work, by page reference: shadows out, restores in, one
    // quantise launch per target tier, each reading pages before any is
    // freed. A page quantised from its shadow is first brought to device
    // memory in one copy (the quantiser reads its rows twice, and host
    // memory is not cached on the device).
    const std::size_t shadows_before = shadows_.count();
    std::vector<RefPair> shadows_out, restores, restage;
    std::array<std::vector<RefPair>, kTierCount> requant;
    bool touches_shadow = false;
    for (std::size_t i = 0; i < n; ++i)
    {
      std::uint32_t rows;
      if (from[i] == kFP16)
      {
        rows = allocator_.ref_of(keys[i]);
        if (!shadows_.contains(keys[i]))
        {
          shadows_out.push_back({rows, page_ref(kShadowSpace, shadows_.add(keys[i]))});
        }
      }
      else
      {
        rows = page_ref(kShadowSpace, shadows_.number(keys[i]));
        touches_shadow = true;
        if (targets[i] != kFP16)
        {
          const auto slot = static_cast<std::uint32_t>(restage.size());
          restage.push_back({rows, page_ref(kStagingSpace, slot)});
          rows = page_ref(kStagingSpace, slot);
        }
      }
      if (targets[i] == kFP16)
      {
        restores.push_back({rows, to[i]});
      }
      else
      {
        requant[targets[i]].push_back({rows, to[i]});
      }
    }
    touches_shadow = touches_shadow || !shadows_out.empty();
    std::vector<RefPair> all;
    all.reserve(2 * n);
    all.insert(all.end(), shadows_out.begin(), shadows_out.end());
    all.insert(all.end(), restage.begin(), restage.end());
    all.insert(all.end(), restores.begin(), restores.end());
    for (const auto &r : requant)
    {
      all.insert(all.end(), r.begin(), r.end());
    }
    const std::size_t fp16_bytes = bytes_at(kFP16);
    if (!restage.empty() && (staging_ == nullptr || staging_->bytes() < restage.size() * fp16_bytes))
    {
      staging_.reset(); // waits for launches that may read the old one
      staging_ = std::make_unique<DeviceBuffer>(restage.size() * fp16_bytes);
    }
    PageSpaces spaces = allocator_.spaces();
    spaces.shadows = shadows_.device_table(stream);
    spaces.staging = staging_ ? reinterpret_cast<unsigned long long>(staging_->raw()) : 0;
    // A launch of a few pairs holds them in its arguments; the rest are
    // uploaded together, once.
    const bool upload = shadows_out.size() > kHeldRefs || restores.size() > kHeldRefs ||
                        restage.size() > kHeldRefs ||
                        std::any_of(requant.begin(), requant.end(),
                                    [](const std::vector<RefPair> &r) { return r.size() > kHeldRefs; });
    const RefPair *on_device = upload ? pairs_upload_.send(all, stream) : nullptr;
    std::size_t at = 0;
    const auto group = [&](std::size_t count) {
      const RefList l = ref_list(all, at, count, on_device);
      at += count;
      return l;
    };
    if (shadow_seconds != nullptr)
    {
      ensure_move_events();
      hip_check(hipEventRecord(move_events_[0], stream), "hipEventRecord before a move's copies");
    }
    // Shadows out, and the shadows that restores quantise from brought into
    // device staging: neither needs the new pages.
    launch_copy_refs(group(shadows_out.size()), static_cast<int>(shadows_out.size()), spaces,
                     stream);
    launch_copy_refs(group(restage.size()), static_cast<int>(restage.size()), spaces, stream);
    phases_[0] = since(entered);
    const Clock::time_point allocating = Clock::now();

    // The new pages, while the shadows travel. A failure gives back what was
    // taken and forgets the shadows just numbered (the copies into their
    // places are harmless: the places are free again, and a later copy into
    // one is ordered after them on the stream).
    // A staged page that landed anywhere but the slot its batch named is
    // refused the same way, before any device work names that slot.
    std::vector<PageKey> taken;
    try
    {
      for (int t = 0; t < kTierCount; ++t)
      {
        allocator_.allocate_run(runs[t], t, false);
        taken.insert(taken.end(), runs[t].begin(), runs[t].end());
      }
      for (std::size_t i = 0; i < n; ++i)
      {
        if (allocator_.ref_of(staged[i]) != to[i])
        {
          throw LogicError("a staged page did not land in the slot its batch named");
        }
      }
    }
    catch (...)
    {
      allocator_.free_pages(taken);
      shadows_.truncate(shadows_before);
      throw;
    }
    phases_[1] = since(allocating);
    launch_copy_refs(group(restores.size()), static_cast<int>(restores.size()), spaces, stream);
    for (int t = kINT8; t <= kINT2; ++t)
    {
      launch_requant_refs(group(requant[t].size()), static_cast<int>(requant[t].size()), t, spaces,
                          page_tokens_, kv_heads_, head_dim_, stream);
    }
    if (shadow_seconds != nullptr)
    {
      hip_check(hipEventRecord(move_events_[1], stream), "hipEventRecord after a move's copies");
    }

    // 3. The page table names the new pages; the old ones go together.
    std::vector<std::pair<PageKey, PageKey>> pairs(n);
    for (std::size_t i = 0; i < n; ++i)
    {
      pairs[i] = {keys[i], staged[i]};
      may_be_at_[targets[i]] = true;
    }
    const Clock::time_point finishing = Clock::now();
    allocator_.replace_pages(pairs);
    hip_check(hipStreamSynchronize(stream), "hipStreamSynchronize after a batch");
    phases_[2] = since(finishing);
    if (shadow_seconds != nullptr)
    {
      // A single move reports what its shadow's trip over the host link
      // took: the device time of the work that reads or writes the shadow.
      float ms = 0.0f;
      hip_check(hipEventElapsedTime(&ms, move_events_[0], move_events_[1]),
                "hipEventElapsedTime of a move's copies");
      *shadow_seconds = touches_shadow ? ms * 1e-3 : 0.0;
    }
  }

  void KVPages::ensure_move_events()
  {
    for (hipEvent_t &e : move_events_)
    {
      if (e == nullptr)
      {
        hip_check(hipEventCreate(&e), "hipEventCreate for a move's timing");
      }
    }
  }

  // ---- attention ---------------------------------------------------------------------

  const unsigned long long *KVPages::open_table(hipStream_t stream)
  {
    std::vector<unsigned long long> now(static_cast<std::size_t>(layers_));
    for (int l = 0; l < layers_; ++l)
    {
      now[l] = open_address_[2 * static_cast<std::size_t>(l) + attend_open_[l]];
    }
    if (open_table_ == nullptr)
    {
      open_table_ = std::make_unique<DeviceBuffer>(now.size() * sizeof(unsigned long long));
    }
    if (now != open_uploaded_)
    {
      hip_check(hipMemcpyAsync(open_table_->raw(), now.data(), now.size() * sizeof(unsigned long long),
                               hipMemcpyHostToDevice, stream),
                "hipMemcpyAsync open-page table");
      open_uploaded_ = now;
    }
    return open_table_->as<const unsigned long long>();
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
    const hipStream_t stream = runtime_stream();
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
    a.partials_floats = partials != nullptr ? attention_partials_floats(head_dim) : 0;
    a.workspace = &workspace_;
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    const std::size_t row = static_cast<std::size_t>(layer) * table_.stride();
    if (!seals_)
    {
      sync_tables(stream);
      kv.layout = Layout::kPaged;
      kv.pages = pages_ > 0 ? table_.addresses() + row : nullptr;
      kv.may_be_at[kFP16] = true;
      launch_attention(kv, a, stream);
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
    sync_tables(stream);
    kv.layout = Layout::kCausal;
    kv.pages = pages_ > 0 ? table_.addresses() + row : nullptr;
    kv.tiers = pages_ > 0 ? table_.tiers() + row : nullptr;
    kv.open = open_page(layer, attend_open_[layer]);
    kv.chunk_k = static_cast<const std::uint16_t *>(keys);
    kv.chunk_v = static_cast<const std::uint16_t *>(values);
    kv.start = seq_k - seq_q;
    std::copy(may_be_at_.begin(), may_be_at_.end(), kv.may_be_at);
    if (seq_q == 1 && layer + 1 < layers_ && pages_ > 0)
    {
      // A decode step visits the layers in order: the next layer's sealed
      // entries are read ahead into the caches.
      const std::size_t next = row + table_.stride();
      kv.warm_pages = table_.addresses() + next;
      kv.warm_tiers = table_.tiers() + next;
      kv.warm_count = std::min((seq_k - 1) / page_tokens_, pages_);
    }
    launch_attention(kv, a, stream);
  }

  void KVPages::attention_kept(int layer, const void *q, const void *k_bias,
                               const RopeTable *rope, void *out, int seq_k, int heads,
                               int kv_heads, int head_dim, const void *keys, const void *values)
  {
    require_layer(layer);
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
    if (k_bias != nullptr && (rope == nullptr || rope->head_dim() != head_dim))
    {
      throw InvalidArgument("a key bias needs a RoPE table for head_dim " +
                            std::to_string(head_dim) + " covering " + std::to_string(seq_k) +
                            " positions");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    AttentionArgs a{};
    a.q = static_cast<const std::uint16_t *>(q);
    a.out = static_cast<std::uint16_t *>(out);
    a.k_bias = static_cast<const std::uint16_t *>(k_bias);
    a.rope = k_bias != nullptr ? rope->data() : nullptr;
    a.rope_positions = k_bias != nullptr ? rope->positions() : 0;
    a.rope_angles = k_bias != nullptr ? rope->angles() : nullptr;
    a.seq_q = 1;
    a.seq_k = seq_k;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.workspace = &workspace_;
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    const std::size_t row = static_cast<std::size_t>(layer) * table_.stride();
    kv.pages = pages_ > 0 ? table_.addresses() + row : nullptr;
    if (seals_)
    {
      kv.layout = Layout::kCausal;
      kv.tiers = pages_ > 0 ? table_.tiers() + row : nullptr;
      kv.open = open_page(layer, attend_open_[layer]);
      kv.chunk_k = static_cast<const std::uint16_t *>(keys);
      kv.chunk_v = static_cast<const std::uint16_t *>(values);
      kv.start = seq_k - 1;
      std::copy(may_be_at_.begin(), may_be_at_.end(), kv.may_be_at);
      if (layer + 1 < layers_ && pages_ > 0)
      {
        const std::size_t next = row + table_.stride();
        kv.warm_pages = table_.addresses() + next;
        kv.warm_tiers = table_.tiers() + next;
        kv.warm_count = std::min((seq_k - 1) / page_tokens_, pages_);
      }
    }
    else
    {
      kv.layout = Layout::kPaged;
      kv.may_be_at[kFP16] = true;
    }
    if (!decode_fast_applies(kv, a))
    {
      throw InvalidArgument("a decode that keeps its statistics takes one query per head, "
                            "32-token pages, head_dim 64 or 128 and at most 16 query heads per "
                            "KV head, 16-byte aligned");
    }
    // A new step (or a new shape) starts a new set of kept statistics.
    if (seq_k != kept_seq_k_ || heads != kept_heads_ || kv_heads != kept_kv_heads_ ||
        head_dim != kept_head_dim_)
    {
      kept_layers_.assign(layers_, 0);
      kept_seq_k_ = seq_k;
      kept_heads_ = heads;
      kept_kv_heads_ = kv_heads;
      kept_head_dim_ = head_dim;
    }
    const int pages = (seq_k + page_tokens_ - 1) / page_tokens_;
    const std::size_t per_layer = decode_kept_floats(heads, kv_heads, seq_k);
    float *kept = kept_.floats(per_layer * layers_);
    const std::size_t ml_floats = per_layer - static_cast<std::size_t>(heads) * pages * 2;
    DecodeLayers ls{};
    ls.split = true;
    ls.layers = 1;
    ls.keep_ml = kept + layer * ml_floats;
    ls.keep_stats = kept + layers_ * ml_floats + static_cast<std::size_t>(layer) * heads * pages * 2;
    launch_decode_layers(kv, a, ls, stream);
    kept_layers_[layer] = 1;
  }

  void KVPages::fold_kept(float *mass, long long mass_stride, float *scores,
                          long long scores_stride, float alpha)
  {
    if (kept_seq_k_ < 0 ||
        std::find(kept_layers_.begin(), kept_layers_.end(), 0) != kept_layers_.end())
    {
      throw LogicError("a fold of kept statistics needs every layer of the step attended by "
                       "attention_kept since the last fold");
    }
    DecodeFold f{};
    f.layers = layers_;
    f.heads = kept_heads_;
    f.kv_heads = kept_kv_heads_;
    f.head_dim = kept_head_dim_;
    f.seq_k = kept_seq_k_;
    f.kept = kept_.floats(decode_kept_floats(kept_heads_, kept_kv_heads_, kept_seq_k_) * layers_);
    f.mass = mass;
    f.mass_stride = mass_stride;
    f.scores = scores;
    f.scores_stride = scores_stride;
    f.alpha = alpha;
    launch_decode_fold(f, runtime_stream());
    kept_layers_.assign(layers_, 0);
  }

  // ---- a decode step with its position on the device ------------------------------------

  void KVPages::prepare_step(int max_seq_k, int heads, int head_dim)
  {
    if (!seals_ || halves_ != Halves::kBoth)
    {
      throw InvalidArgument("a decode step with its position on the device runs on a cache that "
                            "seals its pages, with both halves at their tiers");
    }
    if (max_seq_k <= 0 || max_seq_k > capacity_tokens())
    {
      throw OutOfRange("a step run to " + std::to_string(max_seq_k) + " positions needs them "
                       "reserved; " + std::to_string(capacity_tokens()) + " are");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    // The split decode's partials, split maxima and page statistics at
    // max_seq_k (the largest launch of the run).
    const int pages = (max_seq_k + page_tokens_ - 1) / page_tokens_;
    const int splits = (pages + 7) / 8;
    workspace_.floats(static_cast<std::size_t>(heads) * splits * (head_dim + 2) +
                      static_cast<std::size_t>(heads) * pages * 2);
  }

  void KVPages::store_step(int layer, const void *keys, const void *values, const int *position)
  {
    require_layer(layer);
    if (!seals_ || !open_pages_)
    {
      throw LogicError("a store with its position on the device needs a sealing cache with "
                       "positions reserved");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    StepStore st{};
    st.keys = static_cast<const std::uint16_t *>(keys);
    st.values = static_cast<const std::uint16_t *>(values);
    st.position = position;
    st.open = open_page(layer, current_open_[layer]);
    const std::size_t row = static_cast<std::size_t>(layer) * table_.stride();
    st.addresses = table_.addresses() + row;
    st.tiers = table_.tiers() + row;
    st.kv_heads = kv_heads_;
    launch_step_store(st, head_dim_, stream);
    attend_open_[layer] = current_open_[layer];
  }

  void KVPages::rope_store(int layer, const void *qk, void *qk_out, int q_heads,
                           const int *position, const RopeTable &rope, const void *values,
                           const float *x, const void *norm_weight, void *normed, int hidden,
                           float eps)
  {
    require_layer(layer);
    if (seals_)
    {
      throw LogicError("the row launch stores into FP16 pages; this cache seals its pages");
    }
    if (rope.head_dim() != head_dim_ || rope.data() == nullptr)
    {
      throw InvalidArgument("the RoPE table is for head_dim " + std::to_string(rope.head_dim()) +
                            " with " + std::to_string(rope.positions()) +
                            " positions; the cache's head_dim is " + std::to_string(head_dim_));
    }
    if (q_heads < 0 || qk == nullptr || qk_out == nullptr || values == nullptr ||
        (x != nullptr && (norm_weight == nullptr || normed == nullptr || hidden <= 0)))
    {
      throw InvalidArgument("the row launch needs q and k rows, their output, the values and, "
                            "with x, the norm weight, its output and a positive hidden size");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    RowPrep r{};
    r.x = x;
    r.norm_weight = static_cast<const std::uint16_t *>(norm_weight);
    r.normed = static_cast<std::uint16_t *>(normed);
    r.hidden = hidden;
    r.eps = eps;
    r.qk = static_cast<const std::uint16_t *>(qk);
    r.qk_out = static_cast<std::uint16_t *>(qk_out);
    r.q_heads = q_heads;
    r.kv_heads = kv_heads_;
    r.head_dim = head_dim_;
    r.position = position;
    r.table = rope.data();
    r.table_positions = rope.positions();
    r.values = static_cast<const std::uint16_t *>(values);
    r.pages = table_.addresses() + static_cast<std::size_t>(layer) * table_.stride();
    r.page_tokens = page_tokens_;
    r.positions = capacity_tokens();
    launch_row_prep(r, stream);
  }

  void KVPages::attend_row(int layer, const void *qk, void *qk_out, int q_heads, int seq_k,
                           const RopeTable &rope, const void *values, void *out, const float *x,
                           const void *norm_weight, void *normed, int hidden, float eps)
  {
    require_layer(layer);
    if (seals_)
    {
      throw LogicError("the row's attention stores into FP16 pages; this cache seals its pages");
    }
    if (rope.head_dim() != head_dim_ || rope.data() == nullptr || rope.positions() < seq_k)
    {
      throw InvalidArgument("the RoPE table is for head_dim " + std::to_string(rope.head_dim()) +
                            " with " + std::to_string(rope.positions()) +
                            " positions; the row needs head_dim " + std::to_string(head_dim_) +
                            " covering " + std::to_string(seq_k));
    }
    if (seq_k <= 0 || seq_k > capacity_tokens())
    {
      throw OutOfRange("seq_k " + std::to_string(seq_k) + " is not a position on pages (1 to " +
                       std::to_string(capacity_tokens()) + ")");
    }
    if (q_heads <= 0 || q_heads % kv_heads_ != 0 || qk == nullptr || values == nullptr ||
        out == nullptr ||
        (x != nullptr && (norm_weight == nullptr || normed == nullptr || hidden <= 0)))
    {
      throw InvalidArgument("the row's attention needs q and k rows (a whole number of q heads "
                            "a KV head), the values, the output and, with x, the norm weight, "
                            "its output and a positive hidden size");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    const std::size_t table_row = static_cast<std::size_t>(layer) * table_.stride();
    RowPrep r{};
    r.x = x;
    r.norm_weight = static_cast<const std::uint16_t *>(norm_weight);
    r.normed = static_cast<std::uint16_t *>(normed);
    r.hidden = hidden;
    r.eps = eps;
    r.qk = static_cast<const std::uint16_t *>(qk);
    r.qk_out = static_cast<std::uint16_t *>(qk_out);
    r.q_heads = q_heads;
    r.kv_heads = kv_heads_;
    r.head_dim = head_dim_;
    r.table = rope.data();
    r.table_positions = rope.positions();
    r.values = static_cast<const std::uint16_t *>(values);
    r.pages = table_.addresses() + table_row;
    r.page_tokens = page_tokens_;
    r.positions = capacity_tokens();
    AttentionArgs a{};
    a.q = r.qk;
    a.out = static_cast<std::uint16_t *>(out);
    a.seq_q = 1;
    a.seq_k = seq_k;
    a.heads = q_heads;
    a.kv_heads = kv_heads_;
    a.head_dim = head_dim_;
    a.workspace = &workspace_;
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    kv.layout = Layout::kPaged;
    kv.pages = r.pages;
    kv.may_be_at[kFP16] = true;
    if (!decode_fast_applies(kv, a))
    {
      throw InvalidArgument("the row's attention takes 32-token pages, head_dim 64 or 128, at "
                            "most 16 q heads a KV head and 16-byte aligned rows");
    }
    DecodeLayers one{};
    one.split = true;
    one.layers = 1;
    one.row = &r;
    launch_decode_layers(kv, a, one, stream);
  }

  StepStore KVPages::step_store(int layer, const void *keys, const void *values,
                                const int *position)
  {
    require_layer(layer);
    if (!seals_ || !open_pages_)
    {
      throw LogicError("a store with its position on the device needs a sealing cache with "
                       "positions reserved");
    }
    sync_tables(runtime_stream());
    StepStore st{};
    st.keys = static_cast<const std::uint16_t *>(keys);
    st.values = static_cast<const std::uint16_t *>(values);
    st.position = position;
    st.open = open_page(layer, current_open_[layer]);
    const std::size_t row = static_cast<std::size_t>(layer) * table_.stride();
    st.addresses = table_.addresses() + row;
    st.tiers = table_.tiers() + row;
    st.kv_heads = kv_heads_;
    attend_open_[layer] = current_open_[layer];
    return st;
  }

  void KVPages::attention_step(int layer, const void *q, const void *k_bias, const RopeTable *rope,
                               void *out, const int *live_seq_k, int max_seq_k, int heads,
                               int kv_heads, int head_dim, const void *keys, const void *values,
                               float *keep, const StepStore *seal)
  {
    require_layer(layer);
    if (static_cast<std::size_t>(kv_heads) * head_dim != kv_width_)
    {
      throw InvalidArgument("kv_heads * head_dim is " + std::to_string(kv_heads * head_dim) +
                            "; this cache holds " + std::to_string(kv_width_) + " per token");
    }
    if (!seals_ || !open_pages_ || max_seq_k <= 0 || max_seq_k > capacity_tokens())
    {
      throw LogicError("a decode with its position on the device needs a sealing cache with its "
                       "positions, up to the most the run attends, reserved");
    }
    if (k_bias != nullptr &&
        (rope == nullptr || rope->head_dim() != head_dim || rope->positions() < max_seq_k))
    {
      throw InvalidArgument("a key bias needs a RoPE table for head_dim " +
                            std::to_string(head_dim) + " covering " + std::to_string(max_seq_k) +
                            " positions");
    }
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
    AttentionArgs a{};
    a.q = static_cast<const std::uint16_t *>(q);
    a.out = static_cast<std::uint16_t *>(out);
    a.k_bias = static_cast<const std::uint16_t *>(k_bias);
    a.rope = k_bias != nullptr ? rope->data() : nullptr;
    a.rope_positions = k_bias != nullptr ? rope->positions() : 0;
    a.rope_angles = k_bias != nullptr ? rope->angles() : nullptr;
    a.seq_q = 1;
    a.seq_k = max_seq_k;
    a.heads = heads;
    a.kv_heads = kv_heads;
    a.head_dim = head_dim;
    a.workspace = &workspace_;
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    kv.layout = Layout::kCausal;
    const std::size_t row = static_cast<std::size_t>(layer) * table_.stride();
    kv.pages = pages_ > 0 ? table_.addresses() + row : nullptr;
    kv.tiers = pages_ > 0 ? table_.tiers() + row : nullptr;
    kv.open = open_page(layer, current_open_[layer]);
    kv.chunk_k = static_cast<const std::uint16_t *>(keys);
    kv.chunk_v = static_cast<const std::uint16_t *>(values);
    kv.start = max_seq_k - 1;
    std::copy(may_be_at_.begin(), may_be_at_.end(), kv.may_be_at);
    if (!decode_fast_applies(kv, a))
    {
      throw InvalidArgument("a decode with its position on the device takes one query per head, "
                            "32-token pages, head_dim 64 or 128 and at most 16 query heads per KV "
                            "head, 16-byte aligned");
    }
    DecodeLayers ls{};
    ls.split = true;
    ls.layers = 1;
    ls.live_seq_k = live_seq_k;
    ls.seal = seal;
    if (keep != nullptr)
    {
      const int pages = (max_seq_k + page_tokens_ - 1) / page_tokens_;
      const std::size_t per_layer = decode_kept_floats(heads, kv_heads, max_seq_k);
      const std::size_t ml_floats = per_layer - static_cast<std::size_t>(heads) * pages * 2;
      ls.keep_ml = keep + layer * ml_floats;
      ls.keep_stats =
          keep + layers_ * ml_floats + static_cast<std::size_t>(layer) * heads * pages * 2;
    }
    launch_decode_layers(kv, a, ls, stream);
  }

  void KVPages::fold_step(float *keep, const int *live_seq_k, int max_seq_k, int heads,
                          int kv_heads, int head_dim, int score_every, float *scores,
                          long long scores_stride, float alpha)
  {
    if (keep == nullptr || live_seq_k == nullptr || score_every < 1)
    {
      throw InvalidArgument("a step's fold takes the kept statistics, the device's seq_k and a "
                            "cadence of at least 1");
    }
    DecodeFold f{};
    f.layers = layers_;
    f.heads = heads;
    f.kv_heads = kv_heads;
    f.head_dim = head_dim;
    f.seq_k = max_seq_k;
    f.kept = keep;
    f.scores = scores;
    f.scores_stride = scores_stride;
    f.alpha = alpha;
    f.live_seq_k = live_seq_k;
    f.score_every = score_every;
    launch_decode_fold(f, runtime_stream());
  }

  void KVPages::stored_on_device(int end)
  {
    if (end < 0 || end > capacity_tokens())
    {
      throw OutOfRange("positions up to " + std::to_string(end) + " are not all reserved");
    }
    for (int layer = 0; layer < layers_; ++layer)
    {
      sealed_[layer] = std::max(sealed_[layer], end / page_tokens_);
      attend_open_[layer] = current_open_[layer];
    }
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
    const hipStream_t stream = runtime_stream();
    sync_tables(stream);
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
    KVSource kv{};
    kv.page_tokens = page_tokens_;
    kv.pages = pages_ > 0 ? table_.addresses() : nullptr;
    if (seals_)
    {
      kv.layout = Layout::kCausal;
      kv.tiers = pages_ > 0 ? table_.tiers() : nullptr;
      kv.open = open_page(first_layer, attend_open_[first_layer]);
      kv.chunk_k = static_cast<const std::uint16_t *>(keys);
      kv.chunk_v = static_cast<const std::uint16_t *>(values);
      kv.start = seq_k - 1;
      std::copy(may_be_at_.begin(), may_be_at_.end(), kv.may_be_at);
    }
    else
    {
      kv.layout = Layout::kPaged;
      kv.may_be_at[kFP16] = true;
    }
    if (!decode_fast_applies(kv, a))
    {
      throw InvalidArgument("attention over several layers in one launch takes one query per "
                            "head, 32-token pages, head_dim 64 or 128 and at most 16 query heads "
                            "per KV head, 16-byte aligned; got head_dim " +
                            std::to_string(head_dim) + ", " + std::to_string(heads) + "/" +
                            std::to_string(kv_heads) + " heads, " + std::to_string(page_tokens_) +
                            "-token pages");
    }
    DecodeLayers ls{};
    ls.split = true;
    ls.first_layer = first_layer;
    ls.layers = layers;
    ls.table_stride = table_.stride();
    ls.open_table = seals_ ? open_table(stream) : nullptr;
    ls.q_stride = q_stride;
    ls.chunk_stride = kv_stride;
    ls.out_stride = out_stride;
    ls.mass_stride = mass_stride;
    ls.scores_stride = scores_stride;
    launch_decode_layers(kv, a, ls, stream);
  }

} // namespace mi
