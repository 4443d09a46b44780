// Host-side block manager (see block_manager.hpp).
#include "block_manager.hpp"

#include <algorithm>
#include <cstring>

#include "common.hpp"

namespace krill {

// FNV-1a 64 over schema(3) || dtype tag || utf8(model) || 0xFF || utf8(media)
// || 0xFF || tokens as 8-byte little-endian Int (PrefixCache.swift:511-532).
uint64_t prefix_key(const char *model_id, const char *media_hash, int32_t dtype_tag,
                    const int64_t *tokens, int64_t n) {
  uint64_t h = 14695981039346656037ull;
  auto mix = [&h](uint8_t b) {
    h ^= b;
    h *= 1099511628211ull;
  };
  mix(3);
  mix(static_cast<uint8_t>(dtype_tag));
  for (const char *p = model_id ? model_id : ""; *p; ++p) mix(static_cast<uint8_t>(*p));
  mix(0xFF);
  for (const char *p = media_hash ? media_hash : ""; *p; ++p) mix(static_cast<uint8_t>(*p));
  mix(0xFF);
  for (int64_t i = 0; i < n; ++i) {
    uint64_t t = static_cast<uint64_t>(tokens[i]);
    for (int j = 0; j < 8; ++j) mix(static_cast<uint8_t>(t >> (8 * j)));
  }
  return h;
}

static uint64_t splitmix64(uint64_t &s) {
  uint64_t z = (s += 0x9e3779b97f4a7c15ull);
  z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
  z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
  return z ^ (z >> 31);
}

BlockManager::BlockManager(const BlockManagerConfig &cfg) : cfg_(cfg) {
  refcnt_.assign(static_cast<size_t>(cfg_.num_blocks), 0);
  free_.resize(static_cast<size_t>(cfg_.num_blocks));
  // back() is handed out first: ascending ids by default.
  for (int32_t i = 0; i < cfg_.num_blocks; ++i) free_[static_cast<size_t>(i)] = cfg_.num_blocks - 1 - i;
  if (cfg_.free_list_seed != 0) {
    uint64_t s = cfg_.free_list_seed;
    for (size_t i = free_.size(); i > 1; --i) {
      size_t j = static_cast<size_t>(splitmix64(s) % i);
      std::swap(free_[i - 1], free_[j]);
    }
  }
}

int64_t BlockManager::memory_bytes(int64_t n) const {
  // int8 payload for K and V, plus scale and zero for K and V in fp16
  // (QuantizedKVCache.swift:33-42; G groups per row in affine mode).
  int64_t kv = 2 * n * cfg_.num_kv_heads * cfg_.head_dim;
  int64_t meta = 4 * n * cfg_.num_kv_heads * cfg_.groups * 2;
  return kv + meta;
}

int32_t BlockManager::check_seq(int32_t seq, bool mutable_required) const {
  if (seq < 0 || static_cast<size_t>(seq) >= seqs_.size() || !seqs_[static_cast<size_t>(seq)].alive)
    return fail(KRILL_E_INVAL, "invalid sequence handle %d", seq);
  if (mutable_required && seqs_[static_cast<size_t>(seq)].frozen)
    return fail(KRILL_E_STATE, "sequence %d belongs to a prefix entry and is read-only", seq);
  return KRILL_OK;
}

int32_t BlockManager::new_seq_id() {
  if (!free_seq_ids_.empty()) {
    int32_t id = free_seq_ids_.back();
    free_seq_ids_.pop_back();
    return id;
  }
  // Room for every id to come back, so that returning one never allocates.
  free_seq_ids_.reserve(seqs_.size() + 1);
  seqs_.emplace_back();
  return static_cast<int32_t>(seqs_.size() - 1);
}

void BlockManager::release_block(int32_t b) {
  if (--refcnt_[static_cast<size_t>(b)] == 0) free_.push_back(b);
}

void BlockManager::release_seq_blocks(Seq &s, size_t keep) {
  for (size_t i = keep; i < s.blocks.size(); ++i)
    if (s.blocks[i] != kDropped) release_block(s.blocks[i]);
  s.blocks.resize(keep);
}

bool BlockManager::entry_frees_blocks(const Entry &e) const {
  const Seq &s = seqs_[static_cast<size_t>(e.seq)];
  for (int32_t b : s.blocks)
    if (b != kDropped && refcnt_[static_cast<size_t>(b)] == 1) return true;
  return false;
}

void BlockManager::drop_entry(std::list<Entry>::iterator it, bool count_eviction, bool keep_key) {
  Seq &s = seqs_[static_cast<size_t>(it->seq)];
  size_t before = free_.size();
  release_seq_blocks(s, 0);
  s.alive = false;
  s.frozen = false;
  s.len = 0;
  free_seq_ids_.push_back(it->seq);
  if (count_eviction) {
    ++evicted_entries_;
    evicted_blocks_ += static_cast<int64_t>(free_.size() - before);
  }
  if (!keep_key) entry_by_key_.erase(it->key);
  entries_.erase(it);
}

// Evict least-recently-used prefix entries that own at least one block no
// live sequence references, until at most `target_used` blocks are in use
// or no such entry is left.
void BlockManager::evict_until_below(int32_t target_used) {
  auto used = [this] { return cfg_.num_blocks - static_cast<int32_t>(free_.size()); };
  auto it = entries_.begin();
  while (used() > target_used && it != entries_.end()) {
    if (entry_frees_blocks(*it)) {
      auto victim = it++;
      drop_entry(victim, true);
    } else {
      ++it;
    }
  }
}

int32_t BlockManager::alloc_block(int32_t *out) {
  int32_t threshold = static_cast<int32_t>(cfg_.watermark * static_cast<float>(cfg_.num_blocks));
  int32_t used = cfg_.num_blocks - static_cast<int32_t>(free_.size());
  if (used + 1 > threshold) evict_until_below(threshold - 1);
  if (free_.empty()) evict_until_below(cfg_.num_blocks - 1);
  if (free_.empty())
    return fail(KRILL_E_NOMEM, "block pool exhausted (%d blocks, no evictable prefix entry)",
                cfg_.num_blocks);
  int32_t b = free_.back();
  free_.pop_back();
  refcnt_[static_cast<size_t>(b)] = 1;
  *out = b;
  return KRILL_OK;
}

int32_t BlockManager::seq_create(int32_t *out) {
  std::lock_guard<std::mutex> g(mu_);
  if (!out) return fail(KRILL_E_INVAL, "seq_out is NULL");
  int32_t id = new_seq_id();
  Seq &s = seqs_[static_cast<size_t>(id)];
  s = Seq{};
  s.alive = true;
  ++live_seqs_;
  *out = id;
  return KRILL_OK;
}

int32_t BlockManager::seq_fork(int32_t src, int32_t n_tokens, int32_t *out) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(src, false)) return rc;
  if (!out) return fail(KRILL_E_INVAL, "seq_out is NULL");
  const int32_t src_len = seqs_[static_cast<size_t>(src)].len;
  const int32_t src_start = seqs_[static_cast<size_t>(src)].start;
  if (n_tokens < 0 || n_tokens > src_len)
    return fail(KRILL_E_RANGE, "fork of %d tokens from a sequence of %d", n_tokens, src_len);
  if (n_tokens < src_start)
    return fail(KRILL_E_RANGE, "fork of %d tokens below the sliding window (first retained token %d)", n_tokens,
                src_start);
  const Seq &p = seqs_[static_cast<size_t>(src)];
  const size_t nb = static_cast<size_t>((n_tokens + cfg_.block_tokens - 1) / cfg_.block_tokens);
  std::vector<int32_t> blocks(p.blocks.begin(), p.blocks.begin() + static_cast<std::ptrdiff_t>(nb));
  const int32_t id = new_seq_id();  // may grow seqs_ (p is not used after it)
  Seq &s = seqs_[static_cast<size_t>(id)];
  s = Seq{};
  s.alive = true;
  s.len = n_tokens;
  s.start = src_start;
  s.blocks = std::move(blocks);
  for (int32_t b : s.blocks)
    if (b != kDropped) ++refcnt_[static_cast<size_t>(b)];
  ++live_seqs_;
  *out = id;
  return KRILL_OK;
}

int32_t BlockManager::seq_free(int32_t seq) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, true)) return rc;
  Seq &s = seqs_[static_cast<size_t>(seq)];
  release_seq_blocks(s, 0);
  s.alive = false;
  s.len = 0;
  free_seq_ids_.push_back(seq);
  --live_seqs_;
  return KRILL_OK;
}

int32_t BlockManager::seq_reset(int32_t seq) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, true)) return rc;
  Seq &s = seqs_[static_cast<size_t>(seq)];
  release_seq_blocks(s, 0);
  s.len = 0;
  s.start = 0;
  return KRILL_OK;
}

int32_t BlockManager::seq_length(int32_t seq, int32_t *out) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, false)) return rc;
  if (!out) return fail(KRILL_E_INVAL, "len_out is NULL");
  *out = seqs_[static_cast<size_t>(seq)].len;
  return KRILL_OK;
}

int32_t BlockManager::seq_memory_bytes(int32_t seq, int64_t *out) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, false)) return rc;
  if (!out) return fail(KRILL_E_INVAL, "bytes_out is NULL");
  const Seq &s = seqs_[static_cast<size_t>(seq)];
  *out = memory_bytes(s.len - s.start);  // retained tokens
  return KRILL_OK;
}

int32_t BlockManager::seq_truncate(int32_t seq, int32_t n) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, true)) return rc;
  Seq &s = seqs_[static_cast<size_t>(seq)];
  // QuantizedKVCache.truncate: no-op unless 0 <= n < length (:137-138).
  if (n >= s.len || n < 0) return KRILL_OK;
  // RotatingKVCache.canTruncate: only the retained tail can go (RotatingKVCache.swift:123-127)
  if (n < s.start)
    return fail(KRILL_E_RANGE, "truncate to %d below the sliding window (first retained token %d)", n, s.start);
  size_t keep = static_cast<size_t>((n + cfg_.block_tokens - 1) / cfg_.block_tokens);
  release_seq_blocks(s, keep);
  s.len = n;
  return KRILL_OK;
}

int32_t BlockManager::reserve_append(int32_t seq, int32_t L, int32_t *slots_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, true)) return rc;
  if (L < 0) return fail(KRILL_E_INVAL, "append of %d tokens", L);
  if (L > 0 && !slots_out) return fail(KRILL_E_INVAL, "slot_mapping_out is NULL");
  Seq &s = seqs_[static_cast<size_t>(seq)];
  if (L == 0) return KRILL_OK;
  if (static_cast<int64_t>(s.len) + L > INT32_MAX / 2)
    return fail(KRILL_E_RANGE, "sequence would exceed %d tokens", INT32_MAX / 2);
  const int32_t bt = cfg_.block_tokens;
  // Sliding window: keep window - 1 tokens before the append
  // (RotatingKVCache.trimForAppend, RotatingKVCache.swift:70-75) and drop
  // every block that holds none of the retained ones.  The blocks go back to
  // the pool before the allocations below (they may be what makes them
  // succeed); a failed append takes them back.
  const int32_t old_start = s.start;
  const size_t need = static_cast<size_t>((s.len + L + bt - 1) / bt);
  std::vector<std::pair<int32_t, int32_t>> trimmed;  // (table index, block id)
  std::vector<int32_t> fresh;  // allocated here, released on failure
  // Host memory first (a failed allocation then changes nothing).
  trimmed.reserve(s.blocks.size());
  fresh.reserve(need - std::min(need, s.blocks.size()) + 1);
  s.blocks.reserve(need);
  pending_.reserve(pending_.size() + 1);
  if (cfg_.window > 0 && s.len - s.start > cfg_.window - 1) {
    s.start = s.len - (cfg_.window - 1);
    for (int32_t i = 0; i < s.start / bt; ++i) {
      int32_t &blk = s.blocks[static_cast<size_t>(i)];
      if (blk != kDropped) {
        trimmed.emplace_back(i, blk);
        release_block(blk);
        blk = kDropped;
      }
    }
  }

  int32_t cow_idx = -1, cow_old = -1;
  auto rollback = [&](int32_t rc) {
    for (int32_t b : fresh) release_block(b);
    if (cow_idx >= 0) {
      s.blocks[static_cast<size_t>(cow_idx)] = cow_old;
      pending_.pop_back();
    }
    s.blocks.resize(static_cast<size_t>((s.len + bt - 1) / bt));
    // Re-take the trimmed blocks: a block whose last reference the trim
    // dropped sits on the free stack (nothing was written to it: no kernel
    // runs for a failed append).
    for (const auto &tb : trimmed) {
      const int32_t b = tb.second;
      if (refcnt_[static_cast<size_t>(b)] == 0) {
        auto pos = std::find(free_.begin(), free_.end(), b);
        if (pos != free_.end()) free_.erase(pos);
      }
      ++refcnt_[static_cast<size_t>(b)];
      s.blocks[static_cast<size_t>(tb.first)] = b;
    }
    s.start = old_start;
    return rc;
  };

  // Copy-on-write: the partially filled tail block is shared.
  if (s.len % bt != 0) {
    int32_t idx = s.len / bt;
    int32_t tail = s.blocks[static_cast<size_t>(idx)];
    if (refcnt_[static_cast<size_t>(tail)] > 1) {
      int32_t nb;
      if (int32_t rc = alloc_block(&nb)) return rollback(rc);
      fresh.push_back(nb);
      pending_.push_back({tail, nb});
      s.blocks[static_cast<size_t>(idx)] = nb;
      cow_idx = idx;
      cow_old = tail;
    }
  }
  while (s.blocks.size() < need) {
    int32_t nb;
    if (int32_t rc = alloc_block(&nb)) return rollback(rc);
    fresh.push_back(nb);
    s.blocks.push_back(nb);
  }
  if (cow_idx >= 0) {
    release_block(cow_old);  // the sharer keeps its reference
    ++cow_;
  }
  for (int32_t i = 0; i < L; ++i) {
    int32_t p = s.len + i;
    slots_out[i] = s.blocks[static_cast<size_t>(p / bt)] * bt + p % bt;
  }
  s.len += L;
  appended_ += L;
  return KRILL_OK;
}

int32_t BlockManager::block_table(int32_t seq, int32_t *out, int32_t cap, int32_t *n_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (int32_t rc = check_seq(seq, false)) return rc;
  const Seq &s = seqs_[static_cast<size_t>(seq)];
  int32_t n = static_cast<int32_t>(s.blocks.size());
  if (n_out) *n_out = n;
  if (n > cap) return fail(KRILL_E_RANGE, "block table of %d entries exceeds capacity %d", n, cap);
  if (n > 0 && !out) return fail(KRILL_E_INVAL, "out is NULL");
  std::copy(s.blocks.begin(), s.blocks.end(), out);
  return KRILL_OK;
}

int32_t BlockManager::batch_tables(const int32_t *seqs, int32_t B, int32_t max_blocks,
                                   int32_t *tables_out, int32_t *lens_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (B < 0 || max_blocks < 0) return fail(KRILL_E_INVAL, "negative batch or table width");
  if (B > 0 && (!seqs || !lens_out || (max_blocks > 0 && !tables_out)))
    return fail(KRILL_E_INVAL, "NULL batch argument");
  for (int32_t b = 0; b < B; ++b) {
    if (int32_t rc = check_seq(seqs[b], false)) return rc;
    const Seq &s = seqs_[static_cast<size_t>(seqs[b])];
    if (static_cast<int32_t>(s.blocks.size()) > max_blocks)
      return fail(KRILL_E_RANGE, "sequence %d needs %zu blocks > max_blocks %d", seqs[b],
                  s.blocks.size(), max_blocks);
    int32_t *row = tables_out + static_cast<int64_t>(b) * max_blocks;
    std::fill(row, row + max_blocks, 0);
    std::copy(s.blocks.begin(), s.blocks.end(), row);
    lens_out[b] = s.len;
  }
  return KRILL_OK;
}

int32_t BlockManager::batch_starts(const int32_t *seqs, int32_t B, int32_t *starts_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (B < 0) return fail(KRILL_E_INVAL, "negative batch");
  if (B > 0 && (!seqs || !starts_out)) return fail(KRILL_E_INVAL, "NULL batch argument");
  for (int32_t b = 0; b < B; ++b) {
    if (int32_t rc = check_seq(seqs[b], false)) return rc;
    starts_out[b] = seqs_[static_cast<size_t>(seqs[b])].start;
  }
  return KRILL_OK;
}

int32_t BlockManager::set_window(int32_t window) {
  std::lock_guard<std::mutex> g(mu_);
  if (window < 0 || window == 1) return fail(KRILL_E_INVAL, "sliding window of %d tokens (0 or >= 2)", window);
  if (window == 0)
    for (const Seq &s : seqs_)
      if (s.alive && s.start > 0) return fail(KRILL_E_STATE, "a sequence already dropped tokens to the window");
  cfg_.window = window;
  return KRILL_OK;
}

int32_t BlockManager::prefix_store(int32_t seq, const char *model_id, const char *media_hash,
                                   const int64_t *tokens, int32_t n, int32_t *stored_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (stored_out) *stored_out = 0;
  if (int32_t rc = check_seq(seq, false)) return rc;
  if (seqs_[static_cast<size_t>(seq)].start > 0)
    return fail(KRILL_E_UNSUPPORTED, "prefix entry of a sequence that dropped tokens to the sliding window");
  if (n < 0 || (n > 0 && !tokens)) return fail(KRILL_E_INVAL, "bad token array");
  if (n > seqs_[static_cast<size_t>(seq)].len)
    return fail(KRILL_E_RANGE, "store of %d tokens from a sequence of %d", n,
                seqs_[static_cast<size_t>(seq)].len);
  // storeQuantized guards (PrefixCache.swift:375-383).
  if (n < cfg_.min_prefix_len) return KRILL_OK;
  if (cfg_.max_entry_bytes > 0 && memory_bytes(n) * cfg_.num_layers > cfg_.max_entry_bytes)
    return KRILL_OK;
  if (cfg_.max_entries <= 0) return KRILL_OK;
  const uint64_t key = prefix_key(model_id, media_hash, cfg_.dtype_tag, tokens, n);
  // Everything that allocates happens first, so that a failed host
  // allocation changes nothing: the entry's block list and list node, the
  // sequence slot, and the entry's key slot (an existing entry with the same
  // key hands its slot over).
  const size_t nb = static_cast<size_t>((n + cfg_.block_tokens - 1) / cfg_.block_tokens);
  const Seq &src = seqs_[static_cast<size_t>(seq)];
  std::vector<int32_t> blocks(src.blocks.begin(), src.blocks.begin() + static_cast<std::ptrdiff_t>(nb));
  std::list<Entry> node;
  node.push_back(Entry{key, model_id ? model_id : "", media_hash ? media_hash : "",
                       std::vector<int64_t>(tokens, tokens + n), -1});
  if (free_seq_ids_.empty()) {  // new_seq_id below may grow seqs_
    free_seq_ids_.reserve(seqs_.size() + 1);
    seqs_.reserve(seqs_.size() + 1);
  }
  auto slot = entry_by_key_.find(key);
  const bool replace = slot != entry_by_key_.end();
  if (!replace) slot = entry_by_key_.emplace(key, entries_.end()).first;
  // The blocks are referenced before any entry is dropped: the source may
  // itself be an entry (a handle from krill_prefix_lookup) that the key
  // match or the capacity eviction below removes.
  for (int32_t b : blocks) ++refcnt_[static_cast<size_t>(b)];  // no dropped block: start == 0
  if (replace) drop_entry(slot->second, false, true);
  // storeInMemory: evict LRU while at capacity (PrefixCache.swift:540-551).
  while (!entries_.empty() && static_cast<int32_t>(entries_.size()) >= cfg_.max_entries)
    drop_entry(entries_.begin(), true);
  // Frozen fork holding the first n tokens.
  const int32_t id = new_seq_id();
  Seq &s = seqs_[static_cast<size_t>(id)];
  s = Seq{};
  s.alive = true;
  s.frozen = true;
  s.len = n;
  s.blocks = std::move(blocks);
  node.front().seq = id;
  entries_.splice(entries_.end(), node);
  slot->second = std::prev(entries_.end());
  if (stored_out) *stored_out = 1;
  return KRILL_OK;
}

int32_t BlockManager::prefix_lookup(const char *model_id, const char *media_hash,
                                    const int64_t *tokens, int32_t n, int32_t *prefix_len_out,
                                    int32_t *entry_seq_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (!prefix_len_out || !entry_seq_out) return fail(KRILL_E_INVAL, "NULL output");
  *prefix_len_out = 0;
  *entry_seq_out = -1;
  if (n < 0 || (n > 0 && !tokens)) return fail(KRILL_E_INVAL, "bad token array");
  if (n < cfg_.min_prefix_len) return KRILL_OK;
  const int32_t step = std::max(1, cfg_.min_prefix_len / 2);
  for (int32_t check = n; check >= cfg_.min_prefix_len; check -= step) {
    const int32_t seq = probe_locked(model_id, media_hash, tokens, check);
    if (seq < 0) continue;
    *prefix_len_out = check;
    *entry_seq_out = seq;
    return KRILL_OK;
  }
  return KRILL_OK;
}

int32_t BlockManager::probe_locked(const char *model_id, const char *media_hash, const int64_t *tokens,
                                   int32_t n) {
  const uint64_t key = prefix_key(model_id, media_hash, cfg_.dtype_tag, tokens, n);
  auto it = entry_by_key_.find(key);
  if (it == entry_by_key_.end()) return -1;
  const Entry &e = *it->second;
  // Keys are hashes; an entry only hits when its tokens are the probe's.
  if (static_cast<int32_t>(e.tokens.size()) != n || !std::equal(e.tokens.begin(), e.tokens.end(), tokens))
    return -1;
  entries_.splice(entries_.end(), entries_, it->second);  // touch (MRU)
  return e.seq;
}

int32_t BlockManager::prefix_probe(const char *model_id, const char *media_hash, const int64_t *tokens, int32_t n,
                                   int32_t *entry_seq_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (!entry_seq_out) return fail(KRILL_E_INVAL, "NULL output");
  *entry_seq_out = -1;
  if (n < 0 || (n > 0 && !tokens)) return fail(KRILL_E_INVAL, "bad token array");
  if (n < cfg_.min_prefix_len) return KRILL_OK;
  *entry_seq_out = probe_locked(model_id, media_hash, tokens, n);
  return KRILL_OK;
}

int32_t BlockManager::prefix_lookup_longest(const char *model_id, const char *media_hash,
                                            const int64_t *tokens, int32_t n,
                                            int32_t *prefix_len_out, int32_t *entry_seq_out) {
  std::lock_guard<std::mutex> g(mu_);
  if (!prefix_len_out || !entry_seq_out) return fail(KRILL_E_INVAL, "NULL output");
  *prefix_len_out = 0;
  *entry_seq_out = -1;
  if (n < 0 || (n > 0 && !tokens)) return fail(KRILL_E_INVAL, "bad token array");
  if (n < cfg_.min_prefix_len) return KRILL_OK;
  const std::string model = model_id ? model_id : "", media = media_hash ? media_hash : "";
  int32_t best = 0;
  auto best_it = entries_.end();
  for (auto it = entries_.end(); it != entries_.begin();) {  // most recent first
    --it;
    if (it->model != model || it->media != media || it->tokens.empty()) continue;
    int32_t m = std::min<int32_t>(n, static_cast<int32_t>(it->tokens.size())), lcp = 0;
    while (lcp < m && it->tokens[static_cast<size_t>(lcp)] == tokens[lcp]) ++lcp;
    if (lcp >= cfg_.min_prefix_len && lcp > best) {
      best = lcp;
      best_it = it;
    }
  }
  if (best_it == entries_.end()) return KRILL_OK;
  *prefix_len_out = best;
  *entry_seq_out = best_it->seq;
  entries_.splice(entries_.end(), entries_, best_it);
  return KRILL_OK;
}

int32_t BlockManager::prefix_clear() {
  std::lock_guard<std::mutex> g(mu_);
  while (!entries_.empty()) drop_entry(entries_.begin(), false);
  return KRILL_OK;
}

int32_t BlockManager::prefix_count(int32_t *out) {
  std::lock_guard<std::mutex> g(mu_);
  if (!out) return fail(KRILL_E_INVAL, "count_out is NULL");
  *out = static_cast<int32_t>(entries_.size());
  return KRILL_OK;
}

std::vector<CopyPair> BlockManager::take_pending() {
  std::lock_guard<std::mutex> g(mu_);
  std::vector<CopyPair> out;
  out.swap(pending_);
  return out;
}

bool BlockManager::has_pending() {
  std::lock_guard<std::mutex> g(mu_);
  return !pending_.empty();
}

int32_t BlockManager::refcounts(int32_t *out, int32_t cap) {
  std::lock_guard<std::mutex> g(mu_);
  if (cap < 0 || (cap > 0 && !out)) return fail(KRILL_E_INVAL, "bad output buffer");
  const int32_t n = std::min(cap, cfg_.num_blocks);
  std::copy(refcnt_.begin(), refcnt_.begin() + n, out);
  return KRILL_OK;
}

BlockManagerStats BlockManager::stats() {
  std::lock_guard<std::mutex> g(mu_);
  BlockManagerStats st{};
  st.num_blocks = cfg_.num_blocks;
  st.blocks_free = static_cast<int32_t>(free_.size());
  st.blocks_used = cfg_.num_blocks - st.blocks_free;
  for (int32_t r : refcnt_)
    if (r > 1) ++st.blocks_shared;
  st.live_seqs = live_seqs_;
  st.prefix_entries = static_cast<int32_t>(entries_.size());
  st.appended_tokens = appended_;
  st.cow_copies = cow_;
  st.evicted_entries = evicted_entries_;
  st.evicted_blocks = evicted_blocks_;
  st.pending_copies = static_cast<int64_t>(pending_.size());
  return st;
}

}  // namespace krill
