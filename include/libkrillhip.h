/*
 * libkrillhip.h -- C ABI of the MI355X (gfx950) int8 paged KV-cache library.
 *
 * Drop-in for Krill's int8 KV hot path.  Each entry point names the reference
 * interface it replaces (paths relative to the srvsngh99/Krill source tree):
 *
 *   pool / sequences   QuantizedKVCache state   Sources/KrillCache/QuantizedKVCache.swift:17-146
 *                      makeQuantizedKVCaches     Sources/KrillCache/QuantizedKVCache.swift:207-210
 *   prefix entries     PrefixCache int8 API      Sources/KrillCache/PrefixCache.swift:161-308,:369-400,:511-551
 *   kernels            KrillKernels registry     Sources/KrillKernels/KernelRegistry.swift:13-162
 *
 * Conventions
 *   - Every call returns int32_t: KRILL_OK (0) or a negative KRILL_E_* code.
 *     The library never aborts; krill_last_error() gives a per-thread message.
 *   - Pointers named `dev_*` or documented as device pointers are HIP device
 *     memory; everything else is host memory.  Kernels are asynchronous on the
 *     given stream (NULL = the pool's stream).  Block-manager calls are host
 *     only, thread-safe (one mutex per pool) and never synchronise the device.
 *   - Tensor layouts follow the reference: new K/V and queries are
 *     [B][H][L][D] (QuantizedKVCache.update input, QuantizedKVCache.swift:46),
 *     snapshots are [B][H][S][D] u8 + [B][H][S][G] f16 (QuantizedKVSnapshot,
 *     QuantizedKVCache.swift:150-157; G = 1 in the reference's row mode).
 *   - Attention takes queries as fp16 (relative rounding 2^-11; scores and
 *     softmax in fp32).  bf16 queries keep their whole range: a query row
 *     whose largest |q| is 65504 or more is scaled by an exact power of two
 *     before the fp16 rounding and its scores by the inverse, so it neither
 *     overflows nor changes the rows beside it; elements of such a row below
 *     2^-40 of its largest |q| round to zero.  A row holding inf or NaN
 *     gives NaN output.
 */
#ifndef LIBKRILLHIP_H
#define LIBKRILLHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KRILL_ABI_VERSION 1

/* status codes */
#define KRILL_OK 0
#define KRILL_E_INVAL (-1)       /* bad argument */
#define KRILL_E_NOMEM (-2)       /* block pool exhausted after eviction, or device OOM */
#define KRILL_E_RANGE (-3)       /* length / index outside the valid range */
#define KRILL_E_HIP (-4)         /* a HIP runtime call failed (message in krill_last_error) */
#define KRILL_E_STATE (-5)       /* operation not allowed in this state (frozen / freed handle) */
#define KRILL_E_UNSUPPORTED (-6) /* shape or mode this build does not handle */

/* storage (quantizer) modes */
#define KRILL_QUANT_REF_ROW 0 /* reference rows: per (token, head) min/max over D, truncating cast,
                                 fp16 scale + fp16 zero (QuantizedKVCache.swift:181-197) */
#define KRILL_QUANT_AFFINE_G64 1 /* affine 8-bit in groups of 64, fp16 scale + fp16 bias
                                    (MLX affine quantize semantics, CheckpointQuantizer.swift:255-260) */

/* element types */
#define KRILL_DTYPE_F16 0
#define KRILL_DTYPE_BF16 1
#define KRILL_DTYPE_F32 2

/* pool flags */
#define KRILL_POOL_HOST_ONLY 1u /* block manager only: no device memory, kernels refused */

/* pool options (krill_pool_set_option) */
#define KRILL_OPT_SPLIT_BLOCKS 1 /* attention work unit in 64-token blocks: per wave on the VALU path
                                    (1..64, consecutive blocks of the batch's concatenated block lists),
                                    per split of one sequence on the MFMA path; 0 = automatic */
#define KRILL_OPT_ATTN_PATH 2    /* 0 auto (VALU <= 8 query rows per KV head, else MFMA), 1 VALU, 2 MFMA;
                                    "VALU" names the decode kernel (one token per lane for the softmax; its
                                    scores and P.V use the matrix cores at head_dim 128 with 3-8 rows and at
                                    head_dim 512), "MFMA" the row-tiled kernel of verify and prefill */
#define KRILL_OPT_WINDOW 3       /* sliding window in tokens (0 none, else >= 2): before each append a
                                    sequence keeps its last window - 1 tokens and its blocks that hold none
                                    of them go back to the pool (RotatingKVCache.trimForAppend,
                                    RotatingKVCache.swift:70-75); for the pool of the sliding layers */
#define KRILL_OPT_PREFIX_SPLIT 4 /* shared-prefix cascade: shared-prefix blocks per workgroup of its prefix
                                    pass (1..64); 0 = automatic */

typedef struct krill_pool *krill_pool_t;
typedef void *krill_stream_t; /* hipStream_t */

typedef struct krill_pool_desc {
  int32_t num_layers;
  int32_t num_kv_heads;
  int32_t head_dim;      /* 64, 128, 256 or 512 (Gemma 4 full-attention layers) */
  int32_t block_tokens;  /* must be 64 */
  int32_t num_blocks;    /* physical blocks per layer */
  int32_t quant_mode;    /* KRILL_QUANT_* */
  int32_t in_dtype;      /* dtype of K/V/Q handed to the kernels: KRILL_DTYPE_BF16 or _F16 */
  uint32_t flags;        /* KRILL_POOL_* */
  float evict_watermark; /* occupancy that triggers LRU eviction of prefix entries; 0 -> 0.9 */
  int32_t max_prefix_entries; /* in-memory entry cap (PrefixCache maxMemoryEntries); 0 -> 8 */
  int32_t min_prefix_len;     /* PrefixCache minPrefixLength; 0 -> 8 */
  int64_t max_entry_bytes;    /* per-entry KV byte cap (PrefixCache maxEntryBytes); <= 0 -> none */
  uint64_t free_list_seed;    /* 0: blocks handed out in ascending order; else a seeded shuffle */
} krill_pool_desc;

typedef struct krill_pool_stats {
  int32_t num_blocks;
  int32_t blocks_used;   /* refcount > 0 */
  int32_t blocks_free;
  int32_t blocks_shared; /* refcount > 1 */
  int32_t live_seqs;     /* caller-owned sequences */
  int32_t prefix_entries;
  int64_t appended_tokens;
  int64_t cow_copies;
  int64_t evicted_entries;
  int64_t evicted_blocks;
  int64_t pending_copies; /* COW block copies queued, not yet issued to a stream */
  int64_t device_bytes;   /* bytes of the KV slab */
  int64_t block_bytes;    /* bytes of one (layer, block) across all KV heads */
} krill_pool_stats;

typedef struct krill_snapshot {
  void *keys;         /* u8  [B][H][S][D] device */
  void *values;       /* u8  [B][H][S][D] device */
  void *key_scales;   /* f16 [B][H][S][G] device */
  void *key_zeros;    /* f16 [B][H][S][G] device (bias in affine mode) */
  void *value_scales; /* f16 [B][H][S][G] device */
  void *value_zeros;  /* f16 [B][H][S][G] device */
} krill_snapshot;

/* ---------------------------------------------------------------- misc */

/* Last error message of the calling thread ("" if none). */
const char *krill_last_error(void);
int32_t krill_abi_version(void);
/* Diagnostics, no counterpart in the reference: per-wave timestamps of the
 * last decode-attention launch, from a library built with `make stamps`
 * (libkrillhip_stamps.so; the product build returns KRILL_E_UNSUPPORTED).
 * Copies up to max_waves rows of 6 words: realtime clock (100 MHz) at the
 * wave's start, when its first block is in registers, and at its end; 0;
 * HW_ID | XCC_ID << 32; blocks | segments << 32.  Returns the rows copied. */
int32_t krill_diag_wave_stamps(uint64_t *out, int32_t max_waves);

/* ---------------------------------------------------------------- pool */

/* Replaces makeQuantizedKVCaches(numLayers:) (QuantizedKVCache.swift:207-210):
 * one pool holds every layer's cache for every sequence. */
int32_t krill_pool_create(const krill_pool_desc *desc, krill_stream_t stream, krill_pool_t *out);
int32_t krill_pool_destroy(krill_pool_t pool);
int32_t krill_pool_get_stats(krill_pool_t pool, krill_pool_stats *out);
int32_t krill_pool_set_stream(krill_pool_t pool, krill_stream_t stream);
int32_t krill_pool_set_option(krill_pool_t pool, int32_t option, int64_t value);
/* Issue queued copy-on-write block copies on `stream` (kernels do this
 * themselves before they touch the pool).  Copies are never issued into a
 * stream that is capturing a HIP graph: there this call, and any kernel
 * entry point while copies are queued, fails with KRILL_E_STATE and leaves
 * the copies queued.  Callers that replay graphs flush eagerly after each
 * step's krill_seq_reserve_append calls. */
int32_t krill_pool_flush(krill_pool_t pool, krill_stream_t stream);

/* Introspection (tests, debugging): copy the per-block reference counts of
 * the first min(cap, num_blocks) blocks.  No counterpart in the reference
 * (it has no block pool). */
int32_t krill_pool_refcounts(krill_pool_t pool, int32_t *out, int32_t cap);

/* ----------------------------------------------------------- sequences */

/* QuantizedKVCache.init (QuantizedKVCache.swift:25) */
int32_t krill_seq_create(krill_pool_t pool, int32_t *seq_out);
/* New sequence sharing the first n_tokens of `src` (blocks refcounted, no
 * copy).  Replaces restoreQuantized(_:) + truncate(to:) of a prefix hit
 * (QuantizedKVCache.swift:122-145, InferenceEngine.swift:1395-1417). */
int32_t krill_seq_fork(krill_pool_t pool, int32_t src, int32_t n_tokens, int32_t *seq_out);
/* reset() (QuantizedKVCache.swift:92-99) = truncate to 0; free drops the handle. */
int32_t krill_seq_free(krill_pool_t pool, int32_t seq);
int32_t krill_seq_reset(krill_pool_t pool, int32_t seq);
/* sequenceLength (QuantizedKVCache.swift:28-30) */
int32_t krill_seq_length(krill_pool_t pool, int32_t seq, int32_t *len_out);
/* memorySizeBytes, per layer (QuantizedKVCache.swift:33-42) */
int32_t krill_seq_memory_bytes(krill_pool_t pool, int32_t seq, int64_t *bytes_out);
/* truncate(to:) (QuantizedKVCache.swift:135-145): no-op when n >= length or n < 0. */
int32_t krill_seq_truncate(krill_pool_t pool, int32_t seq, int32_t n);
/* The bookkeeping half of update(keys:values:) (QuantizedKVCache.swift:49-61):
 * reserve L slots at the end, copy-on-write the tail block if it is shared,
 * LRU-evict prefix entries once occupancy passes the watermark.  Writes L
 * physical slot ids (block * 64 + offset) to slot_mapping_out (host).
 * KRILL_E_NOMEM leaves the sequence unchanged. */
int32_t krill_seq_reserve_append(krill_pool_t pool, int32_t seq, int32_t L, int32_t *slot_mapping_out);
/* Physical block ids of a sequence (host). */
int32_t krill_seq_block_table(krill_pool_t pool, int32_t seq, int32_t *out, int32_t cap, int32_t *n_out);
/* Host block tables [B][max_blocks] (unused entries 0) and lengths [B] for a
 * batch; replaces the per-epoch left-padded stack (BatchedDecode.swift:96-151)
 * as the thing the batched forward consumes. */
int32_t krill_batch_tables(krill_pool_t pool, const int32_t *seqs, int32_t B, int32_t max_blocks,
                           int32_t *tables_out, int32_t *lens_out);

/* ------------------------------------------------------ prefix entries */

/* storeQuantized (PrefixCache.swift:369-400): keep the first n tokens of
 * `seq` as an LRU entry (a frozen fork).  stored_out = 0 when skipped
 * (n < min_prefix_len or over max_entry_bytes), 1 when stored. */
int32_t krill_prefix_store(krill_pool_t pool, int32_t seq, const char *model_id, const char *media_hash,
                           const int64_t *tokens, int32_t n, int32_t *stored_out);
/* lookupQuantized (PrefixCache.swift:161-170 via scan :273-308): exact entry
 * for tokens[0..checkLen) with checkLen stepping down by max(1, min/2).
 * Miss: *prefix_len_out = 0, *entry_seq_out = -1. */
int32_t krill_prefix_lookup(krill_pool_t pool, const char *model_id, const char *media_hash,
                            const int64_t *tokens, int32_t n, int32_t *prefix_len_out, int32_t *entry_seq_out);
/* One step of that scan at exactly n tokens: the in-memory entry keyed by
 * tokens[0..n), LRU-touched on a hit (memoryCache[key] + touchEntryLocked,
 * PrefixCache.swift:294-298).  For callers that interleave their own tier
 * between the lengths (the disk tier, :300-304).  Miss (or n below
 * min_prefix_len): *entry_seq_out = -1. */
int32_t krill_prefix_probe(krill_pool_t pool, const char *model_id, const char *media_hash, const int64_t *tokens,
                           int32_t n, int32_t *entry_seq_out);
/* lookupLongestPrefixQuantized (PrefixCache.swift:235-263): entry with the
 * longest common prefix >= min_prefix_len (ties: most recently used). */
int32_t krill_prefix_lookup_longest(krill_pool_t pool, const char *model_id, const char *media_hash,
                                    const int64_t *tokens, int32_t n, int32_t *prefix_len_out,
                                    int32_t *entry_seq_out);
int32_t krill_prefix_clear(krill_pool_t pool);
int32_t krill_prefix_count(krill_pool_t pool, int32_t *count_out);
/* cacheKey (PrefixCache.swift:511-532): FNV-1a 64 of schema 3 || dtype tag ||
 * model || 0xFF || media || 0xFF || tokens (8-byte little-endian). */
int32_t krill_prefix_key(const char *model_id, const char *media_hash, int32_t dtype_tag,
                         const int64_t *tokens, int64_t n, uint64_t *key_out);

/* ------------------------------------------------------------- kernels */

/* Fused quantize + paged append: the arithmetic half of update(keys:values:)
 * (QuantizedKVCache.swift:49-61 with quantizePerHead :181-197, or the affine
 * group-64 quantizer).  dev_k/dev_v: [B][Hkv][L][D] in the pool's in_dtype;
 * dev_slot_mapping: [B][L] int32 (from krill_seq_reserve_append; < 0 skips). */
int32_t krill_quantize_append(krill_pool_t pool, int32_t layer, const void *dev_k, const void *dev_v,
                              const int32_t *dev_slot_mapping, int32_t B, int32_t L, krill_stream_t stream);
/* Same with element strides (b, h, l) of K and V (d contiguous), e.g. a
 * projection output [B][L][Hkv][D]: (L*Hkv*D, D, Hkv*D). */
int32_t krill_quantize_append_strided(krill_pool_t pool, int32_t layer, const void *dev_k,
                                      const void *dev_v, int64_t stride_b, int64_t stride_h,
                                      int64_t stride_l, const int32_t *dev_slot_mapping, int32_t B,
                                      int32_t L, krill_stream_t stream);
/* RoPE fused into the append: krill_quantize_append_strided with every K row
 * rotated first, the applyRoPEPerRow (Attention.swift:13-20) that precedes
 * update() (Attention.swift:85-86 with the cache update after it): MLX RoPE,
 * traditional = false, over all D dims (element i < D/2 pairs with i + D/2).
 * Row (b, l) turns by position dev_positions[b*L + l] with the fp32 table
 * dev_cos_sin[max_pos][D] (D/2 cosines of the pair angles, then their sines):
 *   k'[i] = k[i]*c_i - k[i+D/2]*s_i,  k'[i+D/2] = k[i]*s_i + k[i+D/2]*c_i
 * in fp32, each product and sum rounded once, then rounded to in_dtype -- the
 * tensor the unrotated call would be handed -- and quantized; V as is.  Rows
 * whose position lies outside [0, max_pos) are not written, like rows with a
 * negative slot. */
int32_t krill_quantize_append_rope(krill_pool_t pool, int32_t layer, const void *dev_k, const void *dev_v,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_l,
                                   const int32_t *dev_slot_mapping, const int32_t *dev_positions,
                                   const float *dev_cos_sin, int32_t max_pos, int32_t B, int32_t L,
                                   krill_stream_t stream);

/* Paged -> contiguous snapshot.  left_pad = 0: quantizedSnapshot()
 * (QuantizedKVCache.swift:106-115), tokens at [0, len), zeros after;
 * left_pad = 1: stackCachesLeftPaddedQuantized (BatchedDecode.swift:96-151),
 * tokens at [S_out - len, S_out), u8/f16 zeros before. */
int32_t krill_gather(krill_pool_t pool, int32_t layer, const int32_t *dev_block_tables,
                     const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks, int32_t S_out,
                     int32_t left_pad, const krill_snapshot *out, krill_stream_t stream);
/* Paged -> dequantized fp16 K/V [B][H][S_out][D]: snapshot()
 * (QuantizedKVCache.swift:82-89, dequantize :200-204). */
int32_t krill_gather_dequant(krill_pool_t pool, int32_t layer, const int32_t *dev_block_tables,
                             const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks, int32_t S_out,
                             int32_t left_pad, void *dev_k_out, void *dev_v_out, krill_stream_t stream);
/* Contiguous snapshot -> paged: restoreQuantized(_:) (QuantizedKVCache.swift
 * :122-129) and the int8 scatterBack slice (ContinuousBatcher.swift:743-801).
 * Row b copies snapshot tokens [dev_src_start[b], +L) to dev_slot_mapping[b][0..L). */
int32_t krill_scatter(krill_pool_t pool, int32_t layer, const krill_snapshot *in, int32_t B, int32_t S_in,
                      const int32_t *dev_src_start, const int32_t *dev_slot_mapping, int32_t L,
                      krill_stream_t stream);
/* Copy whole blocks in every layer: dev_src_dst = n pairs (src, dst). */
int32_t krill_copy_blocks(krill_pool_t pool, const int32_t *dev_src_dst, int32_t n, krill_stream_t stream);

/* Workspace bytes for krill_decode_attention / krill_verify_attention. */
int32_t krill_attention_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t Lq,
                                       int32_t max_seq_len, size_t *bytes_out);
/* Paged int8 decode attention, o = softmax(scale q K^T) V over each
 * sequence's cached tokens (MLXFast.scaledDotProductAttention at
 * Gemma4Model.swift:516-517 / Attention.swift:95-98 with the left-pad mask of
 * BatchedDecode.swift:277-287).  dev_q: [B][Hq][1][D] in_dtype;
 * dev_seq_lens include the token appended this step; out: [B][Hq][1][D]
 * in out_dtype (F32, F16 or BF16).  max_seq_len: host bound on seq_lens
 * (blocks of a longer sequence beyond it are not read).  Two launches on
 * `stream`: the attention kernel and the merge of partial results. */
int32_t krill_decode_attention(krill_pool_t pool, int32_t layer, const void *dev_q,
                               const int32_t *dev_block_tables, const int32_t *dev_seq_lens, int32_t B,
                               int32_t max_blocks, int32_t max_seq_len, int32_t Hq, float scale,
                               void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                               krill_stream_t stream);
/* Decode step with the append fused: krill_quantize_append_strided of each
 * sequence's newest token followed by krill_decode_attention, in one
 * attention launch (plus the merge).  dev_k_new / dev_v_new: rows [b][h][D]
 * in in_dtype at element strides (stride_b, stride_h), d contiguous (e.g.
 * (Hkv*D, D) for [B][Hkv][1][D]).  The token is written at position
 * seq_lens[b] - 1 of the sequence's table, i.e. the slot
 * krill_seq_reserve_append handed out this step; the pool bytes and the
 * output equal those of the two separate calls.  A sequence of length 0, or
 * whose last position lies beyond max_seq_len or the table width, gets no
 * token written.  Replaces the update + SDPA pair of a decode step
 * (QuantizedKVCache.swift:49-74 followed by Attention.swift:95-98). */
int32_t krill_decode_append_attention(krill_pool_t pool, int32_t layer, const void *dev_q,
                                      const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                      int64_t stride_h, const int32_t *dev_block_tables,
                                      const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks,
                                      int32_t max_seq_len, int32_t Hq, float scale, void *dev_out,
                                      int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                      krill_stream_t stream);
/* krill_decode_append_attention without a workspace argument: the split-K
 * partials go to a static device array of 32 MiB (KRILL_NOALLOC_SCRATCH_BYTES)
 * that each GPU holds from library load to process end.  No counterpart in
 * the reference: this entry point is for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, hosts
 * that forbid allocation); it calls no hipMalloc/hipFree.  Same arguments,
 * kernels, output and pool bytes as krill_decode_append_attention.  A step
 * whose workspace (krill_attention_workspace_size, Lq = 1) exceeds the
 * array fails with KRILL_E_RANGE before any launch.  Every call on one GPU
 * shares that GPU's array and leaves its partials there (nothing in it
 * needs to start at zero): calls that overlap on one GPU -- on different
 * streams, or from several pools or threads -- race, so keep them on one
 * stream or ordered by events.  Under graph capture, queued copy-on-write
 * copies must be flushed eagerly first (krill_pool_flush). */
#define KRILL_NOALLOC_SCRATCH_BYTES (32u << 20)
int32_t krill_decode_append_attention_noalloc(krill_pool_t pool, int32_t layer, const void *dev_q,
                                              const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                              int64_t stride_h, const int32_t *dev_block_tables,
                                              const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks,
                                              int32_t max_seq_len, int32_t Hq, float scale, void *dev_out,
                                              int32_t out_dtype, krill_stream_t stream);
/* The decode step with RoPE as well: krill_decode_append_attention for
 * unrotated queries and new K rows, each turned first by its token's
 * position seq_lens[b] - 1 exactly as krill_quantize_append_rope turns K
 * (table dev_cos_sin[max_pos][D], max_pos >= max_seq_len): the
 * applyRoPEPerRow of queries and keys (Attention.swift:13-20), then
 * update() and SDPA.  The output and the pool bytes equal those of
 * krill_quantize_append_rope at the reserved slots followed by
 * krill_decode_attention on the rotated queries. */
int32_t krill_decode_append_attention_rope(krill_pool_t pool, int32_t layer, const void *dev_q,
                                           const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                           int64_t stride_h, const int32_t *dev_block_tables,
                                           const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks,
                                           int32_t max_seq_len, int32_t Hq, float scale, const float *dev_cos_sin,
                                           int32_t max_pos, void *dev_out, int32_t out_dtype, void *dev_ws,
                                           size_t ws_bytes, krill_stream_t stream);
/* Decode attention for sequences that share a prefix (forked from one
 * prefix entry: krill_seq_fork / krill_prefix_lookup, PrefixCache.swift
 * :161-170 with InferenceEngine.swift:1395-1420): sequence b's keys are the
 * prefix_blocks * 64 tokens of the blocks dev_prefix_table[0..prefix_blocks)
 * followed by its own dev_suffix_lens[b] tokens in the blocks
 * dev_suffix_tables[b][..] (its table from column prefix_blocks on).  Same
 * output as krill_decode_attention over the whole tables (within floating-
 * point reassociation): the prefix is attended once for all B sequences'
 * queries (as one sequence whose query positions are the B sequences, on the
 * MFMA path when B * Hq/Hkv > 8 rows per KV head), each suffix on its own,
 * and the partial softmaxes merged.  Three launches on `stream`. */
int32_t krill_shared_prefix_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t prefix_blocks,
                                           int32_t max_suffix_len, size_t *bytes_out);
int32_t krill_decode_attention_shared_prefix(krill_pool_t pool, int32_t layer, const void *dev_q,
                                             const int32_t *dev_prefix_table, int32_t prefix_blocks,
                                             const int32_t *dev_suffix_tables, const int32_t *dev_suffix_lens,
                                             int32_t B, int32_t max_blocks, int32_t max_suffix_len, int32_t Hq,
                                             float scale, void *dev_out, int32_t out_dtype, void *dev_ws,
                                             size_t ws_bytes, krill_stream_t stream);
/* The same with the step's append fused, as krill_decode_append_attention
 * does for the single-pass decode: sequence b's new token (rows at
 * dev_k_new / dev_v_new + b * stride_b + h * stride_h) is quantized into its
 * suffix at position dev_suffix_lens[b] - 1 (slot reserved beforehand) and
 * attended over in the same launches; byte for byte the same cache and
 * output as krill_quantize_append followed by
 * krill_decode_attention_shared_prefix. */
int32_t krill_decode_append_attention_shared_prefix(krill_pool_t pool, int32_t layer, const void *dev_q,
                                                    const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                                    int64_t stride_h, const int32_t *dev_prefix_table,
                                                    int32_t prefix_blocks, const int32_t *dev_suffix_tables,
                                                    const int32_t *dev_suffix_lens, int32_t B, int32_t max_blocks,
                                                    int32_t max_suffix_len, int32_t Hq, float scale, void *dev_out,
                                                    int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                                    krill_stream_t stream);
/* First retained token of each sequence (0 unless the pool's window dropped
 * tokens): RotatingKVCache's totalSeen - retainedLength
 * (RotatingKVCache.swift:57-66); the sequence's length stays the total
 * appended (sequenceLength).  Host arrays. */
int32_t krill_batch_starts(krill_pool_t pool, const int32_t *seqs, int32_t B, int32_t *starts_out);
/* Sliding-window attention (RotatingKVCache.update + the sliding mask of
 * createSlidingWindowCausalMask, LlamaModel.swift:216-230): query row j of
 * sequence b (position p = lens[b] - Lq + j) sees keys k with
 * max(starts[b], p - window + 1) <= k <= p.  Tables are the pool's (block
 * entries below the window are -1 and never read) with the starts of
 * krill_batch_starts (dev_starts NULL: 0, for a pool that keeps every
 * block).  Reads only the blocks from the one holding each sequence's first
 * visible key.  Lq = 1 is decode (the retained window, no mask, as the
 * reference), Lq > 1 a chunked prefill; VALU / MFMA as the other calls. */
int32_t krill_window_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t Lq, int32_t max_blocks,
                                    int32_t max_seq_len, int32_t window, size_t *bytes_out);
int32_t krill_attention_windowed(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                                 const int32_t *dev_block_tables, const int32_t *dev_seq_lens,
                                 const int32_t *dev_starts, int32_t window, int32_t B, int32_t max_blocks,
                                 int32_t max_seq_len, int32_t Hq, float scale, void *dev_out, int32_t out_dtype,
                                 void *dev_ws, size_t ws_bytes, krill_stream_t stream);
/* The sliding layers' decode step in one launch: each sequence's newest
 * token (K/V rows [b][h][D] at element strides stride_b, stride_h) is
 * written at position seq_lens[b] - 1 (the slot krill_seq_reserve_append
 * handed out, after its window trim) and every query attends its window, as
 * krill_quantize_append at that slot followed by krill_attention_windowed
 * with Lq = 1 -- the update() of RotatingKVCache (RotatingKVCache.swift:40-173)
 * and SDPA of a decode step.  With dev_cos_sin (fp32 [max_pos][D], max_pos >=
 * max_seq_len) the queries and new K rows are first turned by the token's
 * absolute position, as krill_decode_append_attention_rope does (the
 * rotating model's applyRoPEPerRow, Attention.swift:13-20); NULL: no RoPE.
 * The decode kernel only: at most 8 query rows per KV head, head_dim <= 256
 * with RoPE (KRILL_E_UNSUPPORTED otherwise).  Workspace:
 * krill_window_workspace_size with Lq = 1. */
int32_t krill_decode_append_attention_windowed(krill_pool_t pool, int32_t layer, const void *dev_q,
                                               const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                               int64_t stride_h, const int32_t *dev_block_tables,
                                               const int32_t *dev_seq_lens, const int32_t *dev_starts,
                                               int32_t window, int32_t B, int32_t max_blocks, int32_t max_seq_len,
                                               int32_t Hq, float scale, const float *dev_cos_sin, int32_t max_pos,
                                               void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                               krill_stream_t stream);
/* Speculative-verify / chunked-prefill attention: Lq new query rows per
 * sequence, already appended, causal inside the window (row j sees tokens
 * [0, len - Lq + j]; BatchedDecode.swift:299-312, LlamaModel.swift:186-202).
 * dev_q / dev_out: [B][Hq][Lq][D]. */
int32_t krill_verify_attention(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                               const int32_t *dev_block_tables, const int32_t *dev_seq_lens, int32_t B,
                               int32_t max_blocks, int32_t max_seq_len, int32_t Hq, float scale,
                               void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                               krill_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* LIBKRILLHIP_H */
