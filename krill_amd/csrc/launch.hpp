// Host-side launch entry points of the gfx950 kernels (called by capi.cpp).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krill {

struct PoolGeometry {
  uint8_t *base = nullptr;    // device slab
  int64_t layer_stride = 0;   // bytes per layer
  int64_t block_stride = 0;   // bytes per block (all heads)
  int32_t head_bytes = 0;     // bytes per (block, head)
  int32_t num_layers = 0, num_blocks = 0, Hkv = 0, D = 0, G = 1;
  int32_t mode = 0;           // MODE_REF / MODE_AFFINE
  int32_t in_dtype = 1;       // DT_F16 / DT_BF16
  int32_t num_cus = 0;        // compute units of the pool's device (0: host-only pool)
};

struct AttnLaunch {
  const void *q;  // [B][Hq][Lq][D] in_dtype
  const int32_t *tables;
  const int32_t *lens;
  int32_t B, max_blocks, max_seq_len, Hq, Lq;
  float scale;
  void *out;
  int32_t out_dtype;
  void *ws;
  size_t ws_bytes;
  int32_t split_blocks;  // 0 = automatic
  int32_t path;          // 0 auto, 1 VALU, 2 MFMA
  // decode step with the append fused: each sequence's newest token (K/V
  // rows [b][h][D] at element strides kn_sb, kn_sh) is written at position
  // len - 1 before it is read; null for attention over the cache as it is
  const void *k_new = nullptr, *v_new = nullptr;
  int64_t kn_sb = 0, kn_sh = 0;
  // RoPE of the queries and the newest K rows (null: none), table [max_pos][D]
  const float *rope_cs = nullptr;
  int32_t rope_max_pos = 0;
  // views used by the shared-prefix cascade: q at element strides (q_strided),
  // every sequence of length len_const (>= 0; lens unused), no causal window,
  // partials only (no output, no merge launch)
  int32_t q_strided = 0;
  int64_t q_sb = 0, q_sh = 0, q_sj = 0;
  int32_t len_const = -1;
  int32_t causal = 1;
  int32_t partial_only = 0;
  // sliding window (window > 0): first retained key per sequence (null: 0)
  const int32_t *win_start = nullptr;
  int32_t window = 0;
};

// Splits/rows plan shared by the workspace query and the launch.
struct AttnPlan {
  int32_t NR;             // query rows per KV head = (Hq/Hkv) * Lq
  int32_t use_mfma;       // 1 when the MFMA kernel runs
  int32_t split_blocks;   // option value: blocks per wave (<= 64), 0 automatic
  int32_t waves;          // workgroups per (KV head, row group): the flat block split
  int32_t nb_cap;         // blocks per sequence covered (from max_seq_len)
  int64_t slots;          // partial results the workspace holds
  int32_t row_groups;     // row groups per KV head (1 on the VALU path)
  int32_t rows_per_group; // query rows per wave: NR (VALU), 16 * nrt (MFMA)
  int32_t nrt;            // MFMA: 16-row tiles per wave (register budget bound)
  int32_t group_waves;    // MFMA: row groups per workgroup, one wave each, sharing one LDS ring (1 on the VALU path)
  int32_t token_split;    // MFMA: 2 = one row group per workgroup, its two waves split each block's tokens; else 1
  size_t ws_bytes;
};

int32_t plan_attention(const PoolGeometry &g, int32_t B, int32_t Hq, int32_t Lq, int32_t max_seq_len,
                       int32_t split_blocks, int32_t path, AttnPlan *plan);

// rope_pos non-null: K rows rotated first (MLX RoPE, traditional = false)
// at positions rope_pos[b][l] from the fp32 table rope_cs[rope_max_pos][D].
hipError_t launch_quantize_append(const PoolGeometry &g, int32_t layer, const void *k, const void *v,
                                  int64_t sb, int64_t sh, int64_t sl, const int32_t *slots, int32_t B,
                                  int32_t L, hipStream_t st, const int32_t *rope_pos = nullptr,
                                  const float *rope_cs = nullptr, int32_t rope_max_pos = 0);
hipError_t launch_gather(const PoolGeometry &g, int32_t layer, const int32_t *tables, const int32_t *lens,
                         int32_t B, int32_t max_blocks, int32_t S_out, int32_t left_pad, void *keys,
                         void *values, void *ks, void *kz, void *vs, void *vz, hipStream_t st);
hipError_t launch_gather_dequant(const PoolGeometry &g, int32_t layer, const int32_t *tables,
                                 const int32_t *lens, int32_t B, int32_t max_blocks, int32_t S_out,
                                 int32_t left_pad, void *k_out, void *v_out, hipStream_t st);
hipError_t launch_scatter(const PoolGeometry &g, int32_t layer, const void *keys, const void *values,
                          const void *ks, const void *kz, const void *vs, const void *vz, int32_t B,
                          int32_t S_in, const int32_t *src_start, const int32_t *slots, int32_t L,
                          hipStream_t st);
hipError_t launch_copy_blocks(const PoolGeometry &g, const int32_t *src_dst, int32_t n, hipStream_t st);
hipError_t launch_attention(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st);
// Shared-prefix cascade: the prefix pass (pa: one virtual sequence of the
// prefix blocks, the B sequences as its query positions, non-causal, partials
// only), the suffix pass (sa: decode over each sequence's own blocks,
// partials only) and the merge of both into sa.out.
// Sliding-window attention: the kernels' window variants read each sequence
// from the block holding its first visible key (tables: the pool's, entries
// below the window dropped and never read) and mask keys below
// max(starts[b], position - window + 1).
hipError_t launch_attention_windowed(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                                     const int32_t *starts, int32_t window, hipStream_t st);
hipError_t launch_attention_shared_prefix(const PoolGeometry &g, int32_t layer, const AttnLaunch &pa,
                                         const AttnPlan &pp, const AttnLaunch &sa, const AttnPlan &sp,
                                         hipStream_t st);

// Resident waves per compute unit of the VALU decode kernel for (D, NR,
// mode), from the runtime's occupancy query on a device pool, else the
// register-budget design point.
int32_t valu_waves_per_cu(const PoolGeometry &g, int32_t NR);
// Longest windowed view (tokens) of the decode kernel's per-sequence
// workgroups (head_dim <= 256; 0 elsewhere).
int32_t valu_window_limit(const PoolGeometry &g, int32_t NR, bool rope);
// Resident workgroups per compute unit of the MFMA kernel for (D, nrt,
// group_waves, token_split, mode) (bound by its LDS ring or its registers), from the
// occupancy query on a device pool.
int32_t mfma_groups_per_cu(const PoolGeometry &g, int32_t nrt, int32_t group_waves, int32_t token_split);

// Per-wave timestamps of the last decode launch (diagnostic build only).
int32_t wave_stamps(unsigned long long *host, int32_t max_waves);

// Per-configuration kernels, defined in the attention translation units.
hipError_t launch_attn_valu(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st);
hipError_t launch_attn_mfma(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st);
hipError_t launch_attn_merge(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                             hipStream_t st);

}  // namespace krill
