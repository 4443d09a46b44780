// C ABI of libkrillhip (declared in include/libkrillhip.h): argument checks,
// device memory ownership, stream plumbing and error reporting around the
// host block manager and the gfx950 kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstring>
#include <memory>
#include <mutex>
#include <new>

#include "block_manager.hpp"
#include "common.hpp"
#include "kdev.hpp"
#include "launch.hpp"
#include "scratch.hpp"

using krill::fail;

struct krill_pool {
  krill_pool_desc desc{};
  std::unique_ptr<krill::BlockManager> bm;
  krill::PoolGeometry geom{};
  hipStream_t stream = nullptr;
  int device = 0;
  bool host_only = false;
  int32_t opt_split_blocks = 0;
  int32_t opt_path = 0;
  int32_t opt_prefix_split = 0;
  std::mutex flush_mu;
};

namespace krill {
hipError_t launch_copy_pairs(const PoolGeometry &g, const CopyPair *pairs, int32_t n, hipStream_t st);
}

namespace {

constexpr int32_t kMaxHeadDim = 512;

int32_t hip_fail(hipError_t e, const char *what) {
  return fail(KRILL_E_HIP, "%s: %s (%d)", what, hipGetErrorString(e), static_cast<int>(e));
}

// Keeps the pool's device current for the duration of a call.
class DeviceGuard {
 public:
  explicit DeviceGuard(int dev) {
    if (hipGetDevice(&prev_) == hipSuccess && prev_ != dev) {
      if (hipSetDevice(dev) == hipSuccess) switched_ = true;
    }
  }
  ~DeviceGuard() {
    if (switched_) (void)hipSetDevice(prev_);
  }

 private:
  int prev_ = 0;
  bool switched_ = false;
};

int32_t check_pool(krill_pool_t p) {
  if (!p) return fail(KRILL_E_INVAL, "pool is NULL");
  return KRILL_OK;
}

int32_t check_device_pool(krill_pool_t p, int32_t layer) {
  if (int32_t rc = check_pool(p)) return rc;
  if (p->host_only) return fail(KRILL_E_STATE, "pool was created host-only; kernels need device memory");
  if (layer < 0 || layer >= p->desc.num_layers)
    return fail(KRILL_E_RANGE, "layer %d outside [0, %d)", layer, p->desc.num_layers);
  return KRILL_OK;
}

hipStream_t pick_stream(krill_pool_t p, krill_stream_t s) { return s ? static_cast<hipStream_t>(s) : p->stream; }

// Issue queued copy-on-write copies before anything touches the pool.
// Copies are never issued into a stream that is capturing a HIP graph: the
// graph would carry this step's (source, destination) pairs by value and
// repeat them on every replay, copying the shared block over the tokens
// appended to the private copy since, while copies queued between replays
// would never run.  Such a call fails with KRILL_E_STATE and leaves the
// copies queued; the caller flushes eagerly (krill_pool_flush) before it
// captures or replays.
int32_t flush_pending(krill_pool_t p, hipStream_t st) {
  if (p->host_only) {
    (void)p->bm->take_pending();
    return KRILL_OK;
  }
  std::lock_guard<std::mutex> g(p->flush_mu);
  if (!p->bm->has_pending()) return KRILL_OK;
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  const hipError_t ce = hipStreamIsCapturing(st, &cs);
  if (ce != hipSuccess) {
    (void)hipGetLastError();
    return fail(KRILL_E_STATE, "copy-on-write block copies are queued and the stream's capture state is unknown "
                "(%s): call krill_pool_flush on an idle stream first", hipGetErrorString(ce));
  }
  if (cs != hipStreamCaptureStatusNone)
    return fail(KRILL_E_STATE, "copy-on-write block copies are queued while the stream captures a graph: call "
                "krill_pool_flush eagerly after krill_seq_reserve_append, before capturing and before each replay");
  std::vector<krill::CopyPair> pairs = p->bm->take_pending();
  if (pairs.empty()) return KRILL_OK;
  hipError_t e = krill::launch_copy_pairs(p->geom, pairs.data(), static_cast<int32_t>(pairs.size()), st);
  if (e != hipSuccess) return hip_fail(e, "copy-on-write block copy");
  return KRILL_OK;
}

}  // namespace

extern "C" {

const char *krill_last_error(void) { return krill::g_last_error; }

int32_t krill_abi_version(void) { return KRILL_ABI_VERSION; }

int32_t krill_diag_wave_stamps(uint64_t *out, int32_t max_waves) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (!out || max_waves < 0) return fail(KRILL_E_INVAL, "out is NULL or max_waves < 0");
    const int32_t n = krill::wave_stamps(reinterpret_cast<unsigned long long *>(out), max_waves);
    if (n == -1) return fail(KRILL_E_UNSUPPORTED, "this build records no wave stamps (make stamps)");
    if (n < 0) return fail(KRILL_E_HIP, "copy of the wave stamps failed");
    return n;
  });
}

int32_t krill_pool_create(const krill_pool_desc *desc, krill_stream_t stream, krill_pool_t *out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (!desc || !out) return fail(KRILL_E_INVAL, "desc/out is NULL");
    *out = nullptr;
    const krill_pool_desc &d = *desc;
    if (d.num_layers < 1 || d.num_kv_heads < 1 || d.num_blocks < 1)
      return fail(KRILL_E_INVAL, "num_layers, num_kv_heads and num_blocks must be >= 1");
    if (d.head_dim != 64 && d.head_dim != 128 && d.head_dim != 256 && d.head_dim != kMaxHeadDim)
      return fail(KRILL_E_UNSUPPORTED, "head_dim %d (supported: 64, 128, 256, 512)", d.head_dim);
    if (d.block_tokens != 64) return fail(KRILL_E_UNSUPPORTED, "block_tokens %d (supported: 64)", d.block_tokens);
    if (d.quant_mode != KRILL_QUANT_REF_ROW && d.quant_mode != KRILL_QUANT_AFFINE_G64)
      return fail(KRILL_E_INVAL, "quant_mode %d", d.quant_mode);
    if (d.in_dtype != KRILL_DTYPE_F16 && d.in_dtype != KRILL_DTYPE_BF16)
      return fail(KRILL_E_INVAL, "in_dtype %d (bf16 or f16)", d.in_dtype);
    if (d.evict_watermark < 0.0f || d.evict_watermark > 1.0f || std::isnan(d.evict_watermark))
      return fail(KRILL_E_INVAL, "evict_watermark %f outside [0, 1]", static_cast<double>(d.evict_watermark));

    std::unique_ptr<krill_pool> p(new (std::nothrow) krill_pool());
    if (!p) return fail(KRILL_E_NOMEM, "host allocation failed");
    p->desc = d;
    if (p->desc.evict_watermark == 0.0f) p->desc.evict_watermark = 0.9f;
    if (p->desc.max_prefix_entries == 0) p->desc.max_prefix_entries = 8;
    if (p->desc.min_prefix_len == 0) p->desc.min_prefix_len = 8;
    p->host_only = (d.flags & KRILL_POOL_HOST_ONLY) != 0;
    p->stream = static_cast<hipStream_t>(stream);

    krill::PoolGeometry &g = p->geom;
    g.num_layers = d.num_layers;
    g.num_blocks = d.num_blocks;
    g.Hkv = d.num_kv_heads;
    g.D = d.head_dim;
    g.G = d.quant_mode == KRILL_QUANT_AFFINE_G64 ? d.head_dim / 64 : 1;
    g.mode = d.quant_mode == KRILL_QUANT_AFFINE_G64 ? krill::MODE_AFFINE : krill::MODE_REF;
    g.in_dtype = d.in_dtype == KRILL_DTYPE_BF16 ? krill::DT_BF16 : krill::DT_F16;
    g.head_bytes = krill::head_region_bytes(g.D, g.G);
    g.block_stride = static_cast<int64_t>(g.Hkv) * g.head_bytes;
    g.layer_stride = static_cast<int64_t>(g.num_blocks) * g.block_stride;
    const int64_t total = g.layer_stride * g.num_layers;

    if (!p->host_only) {
      hipError_t e = hipGetDevice(&p->device);
      if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
      e = hipDeviceGetAttribute(&g.num_cus, hipDeviceAttributeMultiprocessorCount, p->device);
      if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute(multiprocessor count)");
      // this device's copy of the static scratch (krill_decode_append_attention_noalloc)
      e = krill::scratch_init(p->device);
      if (e != hipSuccess) return hip_fail(e, "address of the static scratch");
      void *mem = nullptr;
      e = hipMalloc(&mem, static_cast<size_t>(total));
      if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(KRILL_E_NOMEM, "hipMalloc of %lld bytes for the KV pool failed: %s", static_cast<long long>(total),
                    hipGetErrorString(e));
      }
      g.base = static_cast<uint8_t *>(mem);
      e = hipMemset(mem, 0, static_cast<size_t>(total));
      if (e != hipSuccess) {
        (void)hipFree(mem);
        return hip_fail(e, "hipMemset of the KV pool");
      }
    }

    krill::BlockManagerConfig c;
    c.num_blocks = d.num_blocks;
    c.block_tokens = d.block_tokens;
    c.num_layers = d.num_layers;
    c.num_kv_heads = d.num_kv_heads;
    c.head_dim = d.head_dim;
    c.groups = g.G;
    c.watermark = p->desc.evict_watermark;
    c.max_entries = p->desc.max_prefix_entries;
    c.min_prefix_len = p->desc.min_prefix_len;
    c.max_entry_bytes = p->desc.max_entry_bytes;
    c.free_list_seed = p->desc.free_list_seed;
    p->bm.reset(new (std::nothrow) krill::BlockManager(c));
    if (!p->bm) {
      if (g.base) (void)hipFree(g.base);
      return fail(KRILL_E_NOMEM, "host allocation failed");
    }
    *out = p.release();
    return KRILL_OK;
  });
}

int32_t krill_pool_destroy(krill_pool_t pool) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (!pool) return KRILL_OK;
    int32_t rc = KRILL_OK;
    if (pool->geom.base) {
      DeviceGuard dg(pool->device);
      hipError_t e = hipDeviceSynchronize();
      if (e != hipSuccess) rc = hip_fail(e, "hipDeviceSynchronize before freeing the pool");
      e = hipFree(pool->geom.base);
      if (e != hipSuccess && rc == KRILL_OK) rc = hip_fail(e, "hipFree of the KV pool");
    }
    delete pool;
    return rc;
  });
}

int32_t krill_pool_get_stats(krill_pool_t pool, krill_pool_stats *out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    if (!out) return fail(KRILL_E_INVAL, "out is NULL");
    krill::BlockManagerStats s = pool->bm->stats();
    std::memset(out, 0, sizeof(*out));
    out->num_blocks = s.num_blocks;
    out->blocks_used = s.blocks_used;
    out->blocks_free = s.blocks_free;
    out->blocks_shared = s.blocks_shared;
    out->live_seqs = s.live_seqs;
    out->prefix_entries = s.prefix_entries;
    out->appended_tokens = s.appended_tokens;
    out->cow_copies = s.cow_copies;
    out->evicted_entries = s.evicted_entries;
    out->evicted_blocks = s.evicted_blocks;
    out->pending_copies = s.pending_copies;
    out->device_bytes = pool->host_only ? 0 : pool->geom.layer_stride * pool->geom.num_layers;
    out->block_bytes = pool->geom.block_stride;
    return KRILL_OK;
  });
}

int32_t krill_pool_refcounts(krill_pool_t pool, int32_t *out, int32_t cap) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->refcounts(out, cap);
  });
}

int32_t krill_pool_set_stream(krill_pool_t pool, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    pool->stream = static_cast<hipStream_t>(stream);
    return KRILL_OK;
  });
}

int32_t krill_pool_set_option(krill_pool_t pool, int32_t option, int64_t value) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    switch (option) {
      case KRILL_OPT_SPLIT_BLOCKS:
        if (value < 0 || value > (1 << 20)) return fail(KRILL_E_INVAL, "split blocks %lld", static_cast<long long>(value));
        pool->opt_split_blocks = static_cast<int32_t>(value);
        return KRILL_OK;
      case KRILL_OPT_ATTN_PATH:
        if (value < 0 || value > 2) return fail(KRILL_E_INVAL, "attention path %lld", static_cast<long long>(value));
        pool->opt_path = static_cast<int32_t>(value);
        return KRILL_OK;
      case KRILL_OPT_WINDOW:
        if (value < 0 || value > INT32_MAX / 4) return fail(KRILL_E_INVAL, "window %lld", static_cast<long long>(value));
        return pool->bm->set_window(static_cast<int32_t>(value));
      case KRILL_OPT_PREFIX_SPLIT:
        if (value < 0 || value > 64) return fail(KRILL_E_INVAL, "prefix split %lld", static_cast<long long>(value));
        pool->opt_prefix_split = static_cast<int32_t>(value);
        return KRILL_OK;

      default:
        return fail(KRILL_E_INVAL, "unknown option %d", option);
    }
  });
}

int32_t krill_pool_flush(krill_pool_t pool, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    DeviceGuard dg(pool->device);
    return flush_pending(pool, pick_stream(pool, stream));
  });
}

// ------------------------------------------------------------- sequences

int32_t krill_seq_create(krill_pool_t pool, int32_t *seq_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_create(seq_out);
  });
}
int32_t krill_seq_fork(krill_pool_t pool, int32_t src, int32_t n_tokens, int32_t *seq_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_fork(src, n_tokens, seq_out);
  });
}
int32_t krill_seq_free(krill_pool_t pool, int32_t seq) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_free(seq);
  });
}
int32_t krill_seq_reset(krill_pool_t pool, int32_t seq) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_reset(seq);
  });
}
int32_t krill_seq_length(krill_pool_t pool, int32_t seq, int32_t *len_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_length(seq, len_out);
  });
}
int32_t krill_seq_memory_bytes(krill_pool_t pool, int32_t seq, int64_t *bytes_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_memory_bytes(seq, bytes_out);
  });
}
int32_t krill_seq_truncate(krill_pool_t pool, int32_t seq, int32_t n) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->seq_truncate(seq, n);
  });
}
int32_t krill_seq_reserve_append(krill_pool_t pool, int32_t seq, int32_t L, int32_t *slot_mapping_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->reserve_append(seq, L, slot_mapping_out);
  });
}
int32_t krill_seq_block_table(krill_pool_t pool, int32_t seq, int32_t *out, int32_t cap, int32_t *n_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->block_table(seq, out, cap, n_out);
  });
}
int32_t krill_batch_tables(krill_pool_t pool, const int32_t *seqs, int32_t B, int32_t max_blocks,
                           int32_t *tables_out, int32_t *lens_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->batch_tables(seqs, B, max_blocks, tables_out, lens_out);
  });
}

int32_t krill_batch_starts(krill_pool_t pool, const int32_t *seqs, int32_t B, int32_t *starts_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->batch_starts(seqs, B, starts_out);
  });
}

// -------------------------------------------------------- prefix entries

int32_t krill_prefix_store(krill_pool_t pool, int32_t seq, const char *model_id, const char *media_hash,
                           const int64_t *tokens, int32_t n, int32_t *stored_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_store(seq, model_id, media_hash, tokens, n, stored_out);
  });
}
int32_t krill_prefix_lookup(krill_pool_t pool, const char *model_id, const char *media_hash,
                            const int64_t *tokens, int32_t n, int32_t *prefix_len_out, int32_t *entry_seq_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_lookup(model_id, media_hash, tokens, n, prefix_len_out, entry_seq_out);
  });
}
int32_t krill_prefix_probe(krill_pool_t pool, const char *model_id, const char *media_hash, const int64_t *tokens,
                           int32_t n, int32_t *entry_seq_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_probe(model_id, media_hash, tokens, n, entry_seq_out);
  });
}
int32_t krill_prefix_lookup_longest(krill_pool_t pool, const char *model_id, const char *media_hash,
                                    const int64_t *tokens, int32_t n, int32_t *prefix_len_out,
                                    int32_t *entry_seq_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_lookup_longest(model_id, media_hash, tokens, n, prefix_len_out, entry_seq_out);
  });
}
int32_t krill_prefix_clear(krill_pool_t pool) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_clear();
  });
}
int32_t krill_prefix_count(krill_pool_t pool, int32_t *count_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    return pool->bm->prefix_count(count_out);
  });
}
int32_t krill_prefix_key(const char *model_id, const char *media_hash, int32_t dtype_tag, const int64_t *tokens,
                         int64_t n, uint64_t *key_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (!key_out) return fail(KRILL_E_INVAL, "key_out is NULL");
    if (n < 0 || (n > 0 && !tokens)) return fail(KRILL_E_INVAL, "bad token array");
    if (dtype_tag < 0 || dtype_tag > 255) return fail(KRILL_E_INVAL, "dtype tag %d", dtype_tag);
    *key_out = krill::prefix_key(model_id, media_hash, dtype_tag, tokens, n);
    return KRILL_OK;
  });
}

// ---------------------------------------------------------------- kernels

int32_t krill_quantize_append_strided(krill_pool_t pool, int32_t layer, const void *dev_k, const void *dev_v,
                                      int64_t stride_b, int64_t stride_h, int64_t stride_l,
                                      const int32_t *dev_slot_mapping, int32_t B, int32_t L,
                                      krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B < 0 || L < 0) return fail(KRILL_E_INVAL, "negative B or L");
    if (B == 0 || L == 0) return KRILL_OK;
    if (!dev_k || !dev_v || !dev_slot_mapping) return fail(KRILL_E_INVAL, "NULL device pointer");
    if (stride_b < 0 || stride_h < 0 || stride_l < 0) return fail(KRILL_E_INVAL, "negative stride");
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_quantize_append(pool->geom, layer, dev_k, dev_v, stride_b, stride_h, stride_l,
                                                 dev_slot_mapping, B, L, st);
    if (e != hipSuccess) return hip_fail(e, "quantize-append launch");
    return KRILL_OK;
  });
}

int32_t krill_quantize_append_rope(krill_pool_t pool, int32_t layer, const void *dev_k, const void *dev_v,
                                   int64_t stride_b, int64_t stride_h, int64_t stride_l,
                                   const int32_t *dev_slot_mapping, const int32_t *dev_positions,
                                   const float *dev_cos_sin, int32_t max_pos, int32_t B, int32_t L,
                                   krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B < 0 || L < 0) return fail(KRILL_E_INVAL, "negative B or L");
    if (B == 0 || L == 0) return KRILL_OK;
    if (!dev_k || !dev_v || !dev_slot_mapping || !dev_positions || !dev_cos_sin)
      return fail(KRILL_E_INVAL, "NULL device pointer");
    if (stride_b < 0 || stride_h < 0 || stride_l < 0) return fail(KRILL_E_INVAL, "negative stride");
    if (max_pos < 1) return fail(KRILL_E_INVAL, "max_pos %d: the table needs at least one position", max_pos);
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_quantize_append(pool->geom, layer, dev_k, dev_v, stride_b, stride_h, stride_l,
                                                 dev_slot_mapping, B, L, st, dev_positions, dev_cos_sin, max_pos);
    if (e != hipSuccess) return hip_fail(e, "RoPE quantize-append launch");
    return KRILL_OK;
  });
}

int32_t krill_quantize_append(krill_pool_t pool, int32_t layer, const void *dev_k, const void *dev_v,
                              const int32_t *dev_slot_mapping, int32_t B, int32_t L, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    if (!pool) return fail(KRILL_E_INVAL, "pool is NULL");
    const int64_t D = pool->desc.head_dim, H = pool->desc.num_kv_heads;
    return krill_quantize_append_strided(pool, layer, dev_k, dev_v, H * L * D, L * D, D, dev_slot_mapping, B, L,
                                         stream);
  });
}

int32_t krill_gather(krill_pool_t pool, int32_t layer, const int32_t *dev_block_tables, const int32_t *dev_seq_lens,
                     int32_t B, int32_t max_blocks, int32_t S_out, int32_t left_pad, const krill_snapshot *out,
                     krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B < 0 || S_out < 0 || max_blocks < 0) return fail(KRILL_E_INVAL, "negative B, S_out or max_blocks");
    if (B == 0 || S_out == 0) return KRILL_OK;
    if (!out || !out->keys || !out->values || !out->key_scales || !out->key_zeros || !out->value_scales ||
        !out->value_zeros || !dev_block_tables || !dev_seq_lens)
      return fail(KRILL_E_INVAL, "NULL pointer");
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_gather(pool->geom, layer, dev_block_tables, dev_seq_lens, B, max_blocks, S_out,
                                        left_pad ? 1 : 0, out->keys, out->values, out->key_scales, out->key_zeros,
                                        out->value_scales, out->value_zeros, st);
    if (e != hipSuccess) return hip_fail(e, "gather launch");
    return KRILL_OK;
  });
}

int32_t krill_gather_dequant(krill_pool_t pool, int32_t layer, const int32_t *dev_block_tables,
                             const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks, int32_t S_out,
                             int32_t left_pad, void *dev_k_out, void *dev_v_out, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B < 0 || S_out < 0 || max_blocks < 0) return fail(KRILL_E_INVAL, "negative B, S_out or max_blocks");
    if (B == 0 || S_out == 0) return KRILL_OK;
    if (!dev_k_out || !dev_v_out || !dev_block_tables || !dev_seq_lens) return fail(KRILL_E_INVAL, "NULL pointer");
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_gather_dequant(pool->geom, layer, dev_block_tables, dev_seq_lens, B, max_blocks,
                                                S_out, left_pad ? 1 : 0, dev_k_out, dev_v_out, st);
    if (e != hipSuccess) return hip_fail(e, "dequantizing gather launch");
    return KRILL_OK;
  });
}

int32_t krill_scatter(krill_pool_t pool, int32_t layer, const krill_snapshot *in, int32_t B, int32_t S_in,
                      const int32_t *dev_src_start, const int32_t *dev_slot_mapping, int32_t L,
                      krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B < 0 || S_in < 0 || L < 0) return fail(KRILL_E_INVAL, "negative B, S_in or L");
    if (B == 0 || L == 0) return KRILL_OK;
    if (!in || !in->keys || !in->values || !in->key_scales || !in->key_zeros || !in->value_scales ||
        !in->value_zeros || !dev_src_start || !dev_slot_mapping)
      return fail(KRILL_E_INVAL, "NULL pointer");
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_scatter(pool->geom, layer, in->keys, in->values, in->key_scales, in->key_zeros,
                                         in->value_scales, in->value_zeros, B, S_in, dev_src_start, dev_slot_mapping,
                                         L, st);
    if (e != hipSuccess) return hip_fail(e, "scatter launch");
    return KRILL_OK;
  });
}

int32_t krill_copy_blocks(krill_pool_t pool, const int32_t *dev_src_dst, int32_t n, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, 0)) return rc;
    if (n < 0) return fail(KRILL_E_INVAL, "negative pair count");
    if (n == 0) return KRILL_OK;
    if (!dev_src_dst) return fail(KRILL_E_INVAL, "NULL pointer");
    DeviceGuard dg(pool->device);
    hipStream_t st = pick_stream(pool, stream);
    if (int32_t rc = flush_pending(pool, st)) return rc;
    hipError_t e = krill::launch_copy_blocks(pool->geom, dev_src_dst, n, st);
    if (e != hipSuccess) return hip_fail(e, "block copy launch");
    return KRILL_OK;
  });
}

int32_t krill_attention_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t Lq, int32_t max_seq_len,
                                       size_t *bytes_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    if (!bytes_out) return fail(KRILL_E_INVAL, "bytes_out is NULL");
    krill::AttnPlan plan;
    int32_t pr = krill::plan_attention(pool->geom, B, Hq, Lq, max_seq_len, pool->opt_split_blocks, pool->opt_path,
                                       &plan);
    if (pr == -2) return fail(KRILL_E_UNSUPPORTED, "VALU path handles at most 8 query rows per KV head");
    if (pr != 0) return fail(KRILL_E_INVAL, "Hq %d not a multiple of %d KV heads, or bad B/Lq/length", Hq,
                             pool->geom.Hkv);
    *bytes_out = plan.ws_bytes;
    return KRILL_OK;
  });
}

struct NewTokens {  // decode step with the append fused (all null/zero: none)
  const void *k = nullptr, *v = nullptr;
  int64_t sb = 0, sh = 0;
  const float *rope_cs = nullptr;  // RoPE of the queries and the new K rows (null: none)
  int32_t rope_max_pos = 0;
};

static int32_t run_attention(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                             const int32_t *dev_block_tables, const int32_t *dev_seq_lens, int32_t B,
                             int32_t max_blocks, int32_t max_seq_len, int32_t Hq, float scale, void *dev_out,
                             int32_t out_dtype, void *dev_ws, size_t ws_bytes, krill_stream_t stream,
                             const NewTokens &nt = NewTokens(), bool static_scratch = false) {
  if (int32_t rc = check_device_pool(pool, layer)) return rc;
  if (B < 0 || max_blocks < 0 || max_seq_len < 0) return fail(KRILL_E_INVAL, "negative B, max_blocks or length");
  if (B == 0) return KRILL_OK;
  if (!dev_q || !dev_block_tables || !dev_seq_lens || !dev_out) return fail(KRILL_E_INVAL, "NULL device pointer");
  if (out_dtype != KRILL_DTYPE_F32 && out_dtype != KRILL_DTYPE_F16 && out_dtype != KRILL_DTYPE_BF16)
    return fail(KRILL_E_INVAL, "out_dtype %d", out_dtype);
  if (!std::isfinite(scale)) return fail(KRILL_E_INVAL, "scale is not finite");
  if ((int64_t)max_blocks * 64 < (int64_t)max_seq_len)
    return fail(KRILL_E_RANGE, "max_seq_len %d exceeds the %d-block table width", max_seq_len, max_blocks);
  krill::AttnPlan plan;
  int32_t pr = krill::plan_attention(pool->geom, B, Hq, Lq, max_seq_len, pool->opt_split_blocks, pool->opt_path,
                                     &plan);
  if (pr == -2) return fail(KRILL_E_UNSUPPORTED, "VALU path handles at most 8 query rows per KV head");
  if (pr != 0) return fail(KRILL_E_INVAL, "Hq %d not a multiple of %d KV heads, or bad B/Lq/length", Hq,
                           pool->geom.Hkv);
  if (static_scratch && plan.ws_bytes > ws_bytes)
    return fail(KRILL_E_RANGE,
                "this step needs %zu bytes of workspace, more than the %zu-byte static scratch "
                "(krill_decode_append_attention takes a workspace of any size)",
                plan.ws_bytes, ws_bytes);
  if (ws_bytes < plan.ws_bytes || (plan.ws_bytes > 0 && !dev_ws))
    return fail(KRILL_E_INVAL, "workspace of %zu bytes < %zu required", ws_bytes, plan.ws_bytes);
  krill::AttnLaunch a;
  a.q = dev_q;
  a.tables = dev_block_tables;
  a.lens = dev_seq_lens;
  a.B = B;
  a.max_blocks = max_blocks;
  a.max_seq_len = max_seq_len;
  a.Hq = Hq;
  a.Lq = Lq;
  a.scale = scale;
  a.out = dev_out;
  a.out_dtype = out_dtype == KRILL_DTYPE_F32 ? krill::DT_F32 : out_dtype == KRILL_DTYPE_F16 ? krill::DT_F16 : krill::DT_BF16;
  a.ws = dev_ws;
  a.ws_bytes = ws_bytes;
  a.split_blocks = plan.split_blocks;
  a.path = pool->opt_path;
  a.k_new = nt.k;
  a.v_new = nt.v;
  a.kn_sb = nt.sb;
  a.kn_sh = nt.sh;
  a.rope_cs = nt.rope_cs;
  a.rope_max_pos = nt.rope_max_pos;
  DeviceGuard dg(pool->device);
  hipStream_t st = pick_stream(pool, stream);
  if (int32_t rc = flush_pending(pool, st)) return rc;
  hipError_t e = krill::launch_attention(pool->geom, layer, a, plan, st);
  if (e != hipSuccess) return hip_fail(e, "attention launch");
  return KRILL_OK;
}

int32_t krill_decode_attention(krill_pool_t pool, int32_t layer, const void *dev_q, const int32_t *dev_block_tables,
                               const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks, int32_t max_seq_len,
                               int32_t Hq, float scale, void *dev_out, int32_t out_dtype, void *dev_ws,
                               size_t ws_bytes, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    return run_attention(pool, layer, dev_q, 1, dev_block_tables, dev_seq_lens, B, max_blocks, max_seq_len, Hq, scale,
                         dev_out, out_dtype, dev_ws, ws_bytes, stream);
  });
}

int32_t krill_decode_append_attention(krill_pool_t pool, int32_t layer, const void *dev_q, const void *dev_k_new,
                                      const void *dev_v_new, int64_t stride_b, int64_t stride_h,
                                      const int32_t *dev_block_tables, const int32_t *dev_seq_lens, int32_t B,
                                      int32_t max_blocks, int32_t max_seq_len, int32_t Hq, float scale,
                                      void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                      krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (B > 0 && (!dev_k_new || !dev_v_new)) return fail(KRILL_E_INVAL, "NULL new K/V pointer");
    if (stride_b < 0 || stride_h < 0) return fail(KRILL_E_INVAL, "negative stride");
    NewTokens nt;
    nt.k = dev_k_new;
    nt.v = dev_v_new;
    nt.sb = stride_b;
    nt.sh = stride_h;
    return run_attention(pool, layer, dev_q, 1, dev_block_tables, dev_seq_lens, B, max_blocks, max_seq_len, Hq, scale,
                         dev_out, out_dtype, dev_ws, ws_bytes, stream, nt);
  });
}

int32_t krill_decode_append_attention_noalloc(krill_pool_t pool, int32_t layer, const void *dev_q,
                                              const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                              int64_t stride_h, const int32_t *dev_block_tables,
                                              const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks,
                                              int32_t max_seq_len, int32_t Hq, float scale, void *dev_out,
                                              int32_t out_dtype, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_device_pool(pool, layer)) return rc;
    if (B > 0 && (!dev_k_new || !dev_v_new)) return fail(KRILL_E_INVAL, "NULL new K/V pointer");
    if (stride_b < 0 || stride_h < 0) return fail(KRILL_E_INVAL, "negative stride");
    // the device address of this GPU's scratch array, resolved when the pool
    // was created on it (never the array's host-side name)
    void *scratch = krill::scratch_ptr(pool->device);
    if (!scratch) return fail(KRILL_E_STATE, "static scratch of device %d not resolved", pool->device);
    NewTokens nt;
    nt.k = dev_k_new;
    nt.v = dev_v_new;
    nt.sb = stride_b;
    nt.sh = stride_h;
    return run_attention(pool, layer, dev_q, 1, dev_block_tables, dev_seq_lens, B, max_blocks, max_seq_len, Hq, scale,
                         dev_out, out_dtype, scratch, krill::kScratchBytes, stream, nt, true);
  });
}

int32_t krill_decode_append_attention_rope(krill_pool_t pool, int32_t layer, const void *dev_q,
                                           const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                           int64_t stride_h, const int32_t *dev_block_tables,
                                           const int32_t *dev_seq_lens, int32_t B, int32_t max_blocks,
                                           int32_t max_seq_len, int32_t Hq, float scale, const float *dev_cos_sin,
                                           int32_t max_pos, void *dev_out, int32_t out_dtype, void *dev_ws,
                                           size_t ws_bytes, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (B > 0 && (!dev_k_new || !dev_v_new || !dev_cos_sin)) return fail(KRILL_E_INVAL, "NULL new K/V or table pointer");
    if (stride_b < 0 || stride_h < 0) return fail(KRILL_E_INVAL, "negative stride");
    if (max_pos < 1 || max_pos < max_seq_len)
      return fail(KRILL_E_INVAL, "RoPE table of %d positions does not cover max_seq_len %d", max_pos, max_seq_len);
    NewTokens nt;
    nt.k = dev_k_new;
    nt.v = dev_v_new;
    nt.sb = stride_b;
    nt.sh = stride_h;
    nt.rope_cs = dev_cos_sin;
    nt.rope_max_pos = max_pos;
    return run_attention(pool, layer, dev_q, 1, dev_block_tables, dev_seq_lens, B, max_blocks, max_seq_len, Hq, scale,
                         dev_out, out_dtype, dev_ws, ws_bytes, stream, nt);
  });
}

// Plans of the shared-prefix cascade's two passes and the workspace split.
static int32_t plan_shared_prefix(krill_pool_t pool, int32_t B, int32_t Hq, int32_t prefix_blocks,
                                  int32_t max_suffix_len, krill::AttnPlan *pp, krill::AttnPlan *sp,
                                  size_t *suffix_off, size_t *total) {
  if (B < 0 || prefix_blocks < 1 || max_suffix_len < 0) return fail(KRILL_E_INVAL, "bad B, prefix_blocks or length");
  if ((int64_t)prefix_blocks * 64 > INT32_MAX / 2) return fail(KRILL_E_RANGE, "prefix of %d blocks", prefix_blocks);
  const int32_t psplit = pool->opt_prefix_split > 0 ? pool->opt_prefix_split : pool->opt_split_blocks;
  int32_t r = krill::plan_attention(pool->geom, 1, Hq, std::max(B, 1), prefix_blocks * 64, psplit, 0, pp);
  if (r == 0)
    r = krill::plan_attention(pool->geom, B, Hq, 1, max_suffix_len, pool->opt_split_blocks, pool->opt_path, sp);
  if (r == -2) return fail(KRILL_E_UNSUPPORTED, "VALU path handles at most 8 query rows per KV head");
  if (r != 0) return fail(KRILL_E_INVAL, "Hq %d not a multiple of %d KV heads, or bad B/length", Hq, pool->geom.Hkv);
  *suffix_off = (pp->ws_bytes + 255) & ~(size_t)255;
  *total = *suffix_off + sp->ws_bytes;
  return KRILL_OK;
}

int32_t krill_shared_prefix_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t prefix_blocks,
                                           int32_t max_suffix_len, size_t *bytes_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    if (!bytes_out) return fail(KRILL_E_INVAL, "bytes_out is NULL");
    krill::AttnPlan pp, sp;
    size_t off = 0, total = 0;
    if (int32_t rc = plan_shared_prefix(pool, B, Hq, prefix_blocks, max_suffix_len, &pp, &sp, &off, &total)) return rc;
    *bytes_out = total;
    return KRILL_OK;
  });
}

static int32_t run_shared_prefix(krill_pool_t pool, int32_t layer, const void *dev_q,
                                 const int32_t *dev_prefix_table, int32_t prefix_blocks,
                                 const int32_t *dev_suffix_tables, const int32_t *dev_suffix_lens, int32_t B,
                                 int32_t max_blocks, int32_t max_suffix_len, int32_t Hq, float scale, void *dev_out,
                                 int32_t out_dtype, void *dev_ws, size_t ws_bytes, krill_stream_t stream,
                                 const NewTokens &nt) {
  if (int32_t rc = check_device_pool(pool, layer)) return rc;
  if (B < 0 || max_blocks < 0 || max_suffix_len < 0) return fail(KRILL_E_INVAL, "negative B, max_blocks or length");
  if (B == 0) return KRILL_OK;
  if (!dev_q || !dev_prefix_table || !dev_suffix_tables || !dev_suffix_lens || !dev_out)
    return fail(KRILL_E_INVAL, "NULL device pointer");
  if (out_dtype != KRILL_DTYPE_F32 && out_dtype != KRILL_DTYPE_F16 && out_dtype != KRILL_DTYPE_BF16)
    return fail(KRILL_E_INVAL, "out_dtype %d", out_dtype);
  if (!std::isfinite(scale)) return fail(KRILL_E_INVAL, "scale is not finite");
  if ((int64_t)max_blocks * 64 < (int64_t)max_suffix_len)
    return fail(KRILL_E_RANGE, "max_suffix_len %d exceeds the %d-block table width", max_suffix_len, max_blocks);
  krill::AttnPlan pp, sp;
  size_t off = 0, total = 0;
  if (int32_t rc = plan_shared_prefix(pool, B, Hq, prefix_blocks, max_suffix_len, &pp, &sp, &off, &total)) return rc;
  if (ws_bytes < total || !dev_ws) return fail(KRILL_E_INVAL, "workspace of %zu bytes < %zu required", ws_bytes, total);
  const int32_t od = out_dtype == KRILL_DTYPE_F32 ? krill::DT_F32 : out_dtype == KRILL_DTYPE_F16 ? krill::DT_F16
                                                                                                : krill::DT_BF16;
  const int64_t D = pool->geom.D;
  // prefix pass: one sequence (the prefix blocks), the B sequences as its query positions
  krill::AttnLaunch pa;
  pa.q = dev_q;
  pa.tables = dev_prefix_table;
  pa.lens = dev_suffix_lens;  // not read: len_const
  pa.B = 1;
  pa.max_blocks = prefix_blocks;
  pa.max_seq_len = prefix_blocks * 64;
  pa.Hq = Hq;
  pa.Lq = B;
  pa.scale = scale;
  pa.out = dev_out;
  pa.out_dtype = od;
  pa.ws = dev_ws;
  pa.ws_bytes = off;
  pa.split_blocks = pp.split_blocks;
  pa.path = 0;
  pa.q_strided = 1;  // q is [B][Hq][1][D]: query position j = sequence j
  pa.q_sb = 0;
  pa.q_sh = D;
  pa.q_sj = (int64_t)Hq * D;
  pa.len_const = prefix_blocks * 64;
  pa.causal = 0;
  pa.partial_only = 1;
  // suffix pass: each sequence's own blocks
  krill::AttnLaunch sa;
  sa.q = dev_q;
  sa.tables = dev_suffix_tables;
  sa.lens = dev_suffix_lens;
  sa.B = B;
  sa.max_blocks = max_blocks;
  sa.max_seq_len = max_suffix_len;
  sa.Hq = Hq;
  sa.Lq = 1;
  sa.scale = scale;
  sa.out = dev_out;
  sa.out_dtype = od;
  sa.ws = static_cast<uint8_t *>(dev_ws) + off;
  sa.ws_bytes = ws_bytes - off;
  sa.split_blocks = sp.split_blocks;
  sa.path = pool->opt_path;
  sa.partial_only = 1;
  sa.k_new = nt.k;  // the newest token sits in the suffix blocks
  sa.v_new = nt.v;
  sa.kn_sb = nt.sb;
  sa.kn_sh = nt.sh;
  DeviceGuard dg(pool->device);
  hipStream_t st = pick_stream(pool, stream);
  if (int32_t rc = flush_pending(pool, st)) return rc;
  hipError_t e = krill::launch_attention_shared_prefix(pool->geom, layer, pa, pp, sa, sp, st);
  if (e != hipSuccess) return hip_fail(e, "shared-prefix attention launch");
  return KRILL_OK;
}

int32_t krill_decode_attention_shared_prefix(krill_pool_t pool, int32_t layer, const void *dev_q,
                                             const int32_t *dev_prefix_table, int32_t prefix_blocks,
                                             const int32_t *dev_suffix_tables, const int32_t *dev_suffix_lens,
                                             int32_t B, int32_t max_blocks, int32_t max_suffix_len, int32_t Hq,
                                             float scale, void *dev_out, int32_t out_dtype, void *dev_ws,
                                             size_t ws_bytes, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    return run_shared_prefix(pool, layer, dev_q, dev_prefix_table, prefix_blocks, dev_suffix_tables, dev_suffix_lens, B,
                             max_blocks, max_suffix_len, Hq, scale, dev_out, out_dtype, dev_ws, ws_bytes, stream,
                             NewTokens());
  });
}

int32_t krill_decode_append_attention_shared_prefix(krill_pool_t pool, int32_t layer, const void *dev_q,
                                                    const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                                    int64_t stride_h, const int32_t *dev_prefix_table,
                                                    int32_t prefix_blocks, const int32_t *dev_suffix_tables,
                                                    const int32_t *dev_suffix_lens, int32_t B, int32_t max_blocks,
                                                    int32_t max_suffix_len, int32_t Hq, float scale, void *dev_out,
                                                    int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                                    krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (B > 0 && (!dev_k_new || !dev_v_new)) return fail(KRILL_E_INVAL, "NULL new K/V pointer");
    if (stride_b < 0 || stride_h < 0) return fail(KRILL_E_INVAL, "negative new-row stride");
    NewTokens nt;
    nt.k = dev_k_new;
    nt.v = dev_v_new;
    nt.sb = stride_b;
    nt.sh = stride_h;
    return run_shared_prefix(pool, layer, dev_q, dev_prefix_table, prefix_blocks, dev_suffix_tables, dev_suffix_lens, B,
                             max_blocks, max_suffix_len, Hq, scale, dev_out, out_dtype, dev_ws, ws_bytes, stream, nt);
  });
}

// Plan of a sliding-window call: the lengths the kernels see (from the block
// holding each sequence's first visible key) are at most Lq + window + 62.
static int32_t plan_windowed(krill_pool_t pool, int32_t B, int32_t Hq, int32_t Lq, int32_t max_blocks,
                             int32_t max_seq_len, int32_t window, krill::AttnPlan *plan, size_t *total) {
  if (B < 0 || Lq < 1 || max_blocks < 0 || max_seq_len < 0) return fail(KRILL_E_INVAL, "bad B, Lq, width or length");
  if (window < 2) return fail(KRILL_E_INVAL, "sliding window of %d tokens (>= 2)", window);
  const int64_t vmax = std::min<int64_t>(max_seq_len, (int64_t)Lq + window + 62);
  int32_t r = krill::plan_attention(pool->geom, B, Hq, Lq, (int32_t)vmax, pool->opt_split_blocks, pool->opt_path,
                                    plan);
  if (r == -2) return fail(KRILL_E_UNSUPPORTED, "VALU path handles at most 8 query rows per KV head");
  if (r != 0) return fail(KRILL_E_INVAL, "Hq %d not a multiple of %d KV heads, or bad B/Lq/length", Hq, pool->geom.Hkv);
  *total = plan->ws_bytes;
  return KRILL_OK;
}

int32_t krill_window_workspace_size(krill_pool_t pool, int32_t B, int32_t Hq, int32_t Lq, int32_t max_blocks,
                                    int32_t max_seq_len, int32_t window, size_t *bytes_out) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (int32_t rc = check_pool(pool)) return rc;
    if (!bytes_out) return fail(KRILL_E_INVAL, "bytes_out is NULL");
    krill::AttnPlan plan;
    size_t total = 0;
    if (int32_t rc = plan_windowed(pool, B, Hq, Lq, max_blocks, max_seq_len, window, &plan, &total)) return rc;
    *bytes_out = total;
    return KRILL_OK;
  });
}

static int32_t run_windowed(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                            const int32_t *dev_block_tables, const int32_t *dev_seq_lens, const int32_t *dev_starts,
                            int32_t window, int32_t B, int32_t max_blocks, int32_t max_seq_len, int32_t Hq,
                            float scale, void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                            krill_stream_t stream, const NewTokens &nt) {
  if (int32_t rc = check_device_pool(pool, layer)) return rc;
  if (B < 0 || max_blocks < 0 || max_seq_len < 0) return fail(KRILL_E_INVAL, "negative B, max_blocks or length");
  if (B == 0) return KRILL_OK;
  if (!dev_q || !dev_block_tables || !dev_seq_lens || !dev_out) return fail(KRILL_E_INVAL, "NULL device pointer");
  if (out_dtype != KRILL_DTYPE_F32 && out_dtype != KRILL_DTYPE_F16 && out_dtype != KRILL_DTYPE_BF16)
    return fail(KRILL_E_INVAL, "out_dtype %d", out_dtype);
  if (!std::isfinite(scale)) return fail(KRILL_E_INVAL, "scale is not finite");
  if ((int64_t)max_blocks * 64 < (int64_t)max_seq_len)
    return fail(KRILL_E_RANGE, "max_seq_len %d exceeds the %d-block table width", max_seq_len, max_blocks);
  if (B > 65535) return fail(KRILL_E_RANGE, "batch of %d sequences (at most 65535)", B);
  krill::AttnPlan plan;
  size_t total = 0;
  if (int32_t rc = plan_windowed(pool, B, Hq, Lq, max_blocks, max_seq_len, window, &plan, &total)) return rc;
  if (nt.k && plan.use_mfma)
    return fail(KRILL_E_UNSUPPORTED, "the fused windowed step runs on the decode kernel: at most 8 query rows per "
                "KV head (call krill_quantize_append, then krill_attention_windowed)");
  if (nt.rope_cs && pool->geom.D > 256)
    return fail(KRILL_E_UNSUPPORTED, "windowed RoPE step at head_dim %d (at most 256)", pool->geom.D);
  const int64_t view = std::min<int64_t>(max_seq_len, (int64_t)Lq + window + 62);
  if (!plan.use_mfma && pool->geom.D <= 256) {
    // the decode kernel's per-sequence workgroups: at most 64 blocks per wave
    const int32_t lim = krill::valu_window_limit(pool->geom, plan.NR, nt.rope_cs != nullptr);
    if (view > lim)
      return fail(KRILL_E_UNSUPPORTED, "window of %d tokens: the windowed decode kernel reads at most %d tokens per "
                  "sequence with %d query rows per KV head (KRILL_OPT_ATTN_PATH 2 runs the MFMA kernel instead)",
                  window, lim, plan.NR);
  }
  if (ws_bytes < total || (total > 0 && !dev_ws))
    return fail(KRILL_E_INVAL, "workspace of %zu bytes < %zu required", ws_bytes, total);
  krill::AttnLaunch a;
  a.q = dev_q;
  a.tables = dev_block_tables;
  a.lens = dev_seq_lens;
  a.B = B;
  a.max_blocks = max_blocks;
  a.max_seq_len = (int32_t)view;
  a.Hq = Hq;
  a.Lq = Lq;
  a.scale = scale;
  a.out = dev_out;
  a.out_dtype = out_dtype == KRILL_DTYPE_F32 ? krill::DT_F32 : out_dtype == KRILL_DTYPE_F16 ? krill::DT_F16
                                                                                          : krill::DT_BF16;
  a.ws = dev_ws;
  a.ws_bytes = ws_bytes;
  a.split_blocks = plan.split_blocks;
  a.path = pool->opt_path;
  a.k_new = nt.k;
  a.v_new = nt.v;
  a.kn_sb = nt.sb;
  a.kn_sh = nt.sh;
  a.rope_cs = nt.rope_cs;
  a.rope_max_pos = nt.rope_max_pos;
  DeviceGuard dg(pool->device);
  hipStream_t st = pick_stream(pool, stream);
  if (int32_t rc = flush_pending(pool, st)) return rc;
  hipError_t e = krill::launch_attention_windowed(pool->geom, layer, a, plan, dev_starts, window, st);
  if (e != hipSuccess) return hip_fail(e, "windowed attention launch");
  return KRILL_OK;
}

int32_t krill_attention_windowed(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                                 const int32_t *dev_block_tables, const int32_t *dev_seq_lens,
                                 const int32_t *dev_starts, int32_t window, int32_t B, int32_t max_blocks,
                                 int32_t max_seq_len, int32_t Hq, float scale, void *dev_out, int32_t out_dtype,
                                 void *dev_ws, size_t ws_bytes, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    return run_windowed(pool, layer, dev_q, Lq, dev_block_tables, dev_seq_lens, dev_starts, window, B, max_blocks,
                        max_seq_len, Hq, scale, dev_out, out_dtype, dev_ws, ws_bytes, stream, NewTokens{});
  });
}

int32_t krill_decode_append_attention_windowed(krill_pool_t pool, int32_t layer, const void *dev_q,
                                               const void *dev_k_new, const void *dev_v_new, int64_t stride_b,
                                               int64_t stride_h, const int32_t *dev_block_tables,
                                               const int32_t *dev_seq_lens, const int32_t *dev_starts,
                                               int32_t window, int32_t B, int32_t max_blocks, int32_t max_seq_len,
                                               int32_t Hq, float scale, const float *dev_cos_sin, int32_t max_pos,
                                               void *dev_out, int32_t out_dtype, void *dev_ws, size_t ws_bytes,
                                               krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (B > 0 && (!dev_k_new || !dev_v_new)) return fail(KRILL_E_INVAL, "NULL new K/V pointer");
    if (stride_b < 0 || stride_h < 0) return fail(KRILL_E_INVAL, "negative stride");
    if (dev_cos_sin && (max_pos < 1 || max_pos < max_seq_len))
      return fail(KRILL_E_INVAL, "RoPE table of %d positions does not cover max_seq_len %d", max_pos, max_seq_len);
    NewTokens nt;
    nt.k = dev_k_new;
    nt.v = dev_v_new;
    nt.sb = stride_b;
    nt.sh = stride_h;
    nt.rope_cs = dev_cos_sin;
    nt.rope_max_pos = dev_cos_sin ? max_pos : 0;
    return run_windowed(pool, layer, dev_q, 1, dev_block_tables, dev_seq_lens, dev_starts, window, B, max_blocks,
                        max_seq_len, Hq, scale, dev_out, out_dtype, dev_ws, ws_bytes, stream, nt);
  });
}

int32_t krill_verify_attention(krill_pool_t pool, int32_t layer, const void *dev_q, int32_t Lq,
                               const int32_t *dev_block_tables, const int32_t *dev_seq_lens, int32_t B,
                               int32_t max_blocks, int32_t max_seq_len, int32_t Hq, float scale, void *dev_out,
                               int32_t out_dtype, void *dev_ws, size_t ws_bytes, krill_stream_t stream) {
  return krill::guarded([&]() -> int32_t {
    krill::clear_error();
    if (Lq < 1) return fail(KRILL_E_INVAL, "Lq %d", Lq);
    return run_attention(pool, layer, dev_q, Lq, dev_block_tables, dev_seq_lens, B, max_blocks, max_seq_len, Hq, scale,
                         dev_out, out_dtype, dev_ws, ws_bytes, stream);
  });
}

}  // extern "C"
