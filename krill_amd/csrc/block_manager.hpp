// Host-side block manager of the paged int8 KV pool: fixed-size 64-token
// blocks, per-sequence block tables, refcounted sharing, copy-on-write and
// LRU eviction of prefix entries.  Pure C++ (no HIP): it only hands out block
// ids and records block copies; the device side consumes them.
//
// It replaces the per-sequence state of QuantizedKVCache
// (Sources/KrillCache/QuantizedKVCache.swift:17-146) and the int8 half of
// PrefixCache (Sources/KrillCache/PrefixCache.swift:161-308, :369-400,
// :511-551) with one shared pool.
#pragma once

#include <cstdint>
#include <list>
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

namespace krill {

struct CopyPair {
  int32_t src;
  int32_t dst;
};

struct BlockManagerConfig {
  int32_t num_blocks = 0;
  int32_t block_tokens = 64;
  int32_t num_layers = 1;
  int32_t num_kv_heads = 1;
  int32_t head_dim = 64;
  int32_t groups = 1;             // scale/zero pairs per (token, head)
  int32_t dtype_tag = 2;          // prefix-key dtype tag (2 = int8, PrefixCache.swift:488)
  float watermark = 0.9f;         // occupancy that triggers entry eviction
  int32_t max_entries = 8;        // PrefixCache maxMemoryEntries default (PrefixCache.swift:100)
  int32_t min_prefix_len = 8;     // PrefixCache minPrefixLength default (PrefixCache.swift:101)
  int64_t max_entry_bytes = -1;   // <= 0: no cap
  uint64_t free_list_seed = 0;
  int32_t window = 0;             // sliding window in tokens (0: none)
};

struct BlockManagerStats {
  int32_t num_blocks, blocks_used, blocks_free, blocks_shared, live_seqs, prefix_entries;
  int64_t appended_tokens, cow_copies, evicted_entries, evicted_blocks, pending_copies;
};

uint64_t prefix_key(const char *model_id, const char *media_hash, int32_t dtype_tag,
                    const int64_t *tokens, int64_t n);

class BlockManager {
 public:
  explicit BlockManager(const BlockManagerConfig &cfg);

  int32_t seq_create(int32_t *out);
  int32_t seq_fork(int32_t src, int32_t n_tokens, int32_t *out);
  int32_t seq_free(int32_t seq);
  int32_t seq_reset(int32_t seq);
  int32_t seq_length(int32_t seq, int32_t *out);
  int32_t seq_memory_bytes(int32_t seq, int64_t *out);
  int32_t seq_truncate(int32_t seq, int32_t n);
  int32_t reserve_append(int32_t seq, int32_t L, int32_t *slots_out);
  int32_t block_table(int32_t seq, int32_t *out, int32_t cap, int32_t *n_out);
  int32_t batch_tables(const int32_t *seqs, int32_t B, int32_t max_blocks, int32_t *tables_out,
                       int32_t *lens_out);
  // First retained token of each sequence (0 without a window).
  int32_t batch_starts(const int32_t *seqs, int32_t B, int32_t *starts_out);
  // Sliding window of every sequence from the next append on (0: none).
  int32_t set_window(int32_t window);

  int32_t prefix_store(int32_t seq, const char *model_id, const char *media_hash,
                       const int64_t *tokens, int32_t n, int32_t *stored_out);
  int32_t prefix_lookup(const char *model_id, const char *media_hash, const int64_t *tokens,
                        int32_t n, int32_t *prefix_len_out, int32_t *entry_seq_out);
  // One exact length: the entry keyed by tokens[0..n) (touched on a hit).
  int32_t prefix_probe(const char *model_id, const char *media_hash, const int64_t *tokens, int32_t n,
                       int32_t *entry_seq_out);
  int32_t prefix_lookup_longest(const char *model_id, const char *media_hash,
                                const int64_t *tokens, int32_t n, int32_t *prefix_len_out,
                                int32_t *entry_seq_out);
  int32_t prefix_clear();
  int32_t prefix_count(int32_t *out);

  // Queued copy-on-write copies, removed from the queue.
  std::vector<CopyPair> take_pending();
  bool has_pending();
  BlockManagerStats stats();
  int32_t refcounts(int32_t *out, int32_t cap);

  // Per-layer bytes of `n` cached tokens (QuantizedKVCache.memorySizeBytes).
  int64_t memory_bytes(int64_t n) const;

 private:
  // Table entry of a block dropped from a sliding window.
  static constexpr int32_t kDropped = -1;
  struct Seq {
    std::vector<int32_t> blocks;  // absolute block index -> block id (kDropped below the window)
    int32_t len = 0;
    int32_t start = 0;  // first retained token
    bool alive = false;
    bool frozen = false;  // owned by a prefix entry
  };
  struct Entry {
    uint64_t key;
    std::string model, media;
    std::vector<int64_t> tokens;
    int32_t seq;
  };

  int32_t check_seq(int32_t seq, bool mutable_required) const;
  // Entry sequence keyed by tokens[0..n) with exactly those tokens, touched
  // (most recently used); -1 when there is none.  Caller holds mu_.
  int32_t probe_locked(const char *model_id, const char *media_hash, const int64_t *tokens, int32_t n);
  int32_t new_seq_id();
  int32_t alloc_block(int32_t *out);
  void release_block(int32_t b);
  void release_seq_blocks(Seq &s, size_t keep);
  bool entry_frees_blocks(const Entry &e) const;
  void drop_entry(std::list<Entry>::iterator it, bool count_eviction, bool keep_key = false);
  void evict_until_below(int32_t target_used);

  BlockManagerConfig cfg_;
  std::mutex mu_;
  std::vector<int32_t> refcnt_;
  std::vector<int32_t> free_;  // stack; back() is handed out next
  std::vector<Seq> seqs_;
  std::vector<int32_t> free_seq_ids_;
  std::list<Entry> entries_;  // front = least recently used
  std::unordered_map<uint64_t, std::list<Entry>::iterator> entry_by_key_;
  std::vector<CopyPair> pending_;
  int64_t appended_ = 0, cow_ = 0, evicted_entries_ = 0, evicted_blocks_ = 0;
  int32_t live_seqs_ = 0;
};

}  // namespace krill
