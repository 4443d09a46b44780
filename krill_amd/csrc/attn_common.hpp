// Arguments and workspace layout shared by the paged attention kernels
// (VALU and MFMA paths).
#pragma once

#include "kdev.hpp"
#include "launch.hpp"

namespace krill {

// Workspace: `slots` partial results of RR query rows each (RR = rows per
// row group: all NR rows on the VALU path, 16 * nrt on the MFMA path),
// 256-byte aligned pieces:
//   o      float [slots][RR][D]   unnormalised partial outputs
//   ml     float [slots][RR][2]   (running max m in log2 units, sum l)
// slot = (hk * row_groups + rg) * (waves + B) + wave + b: the flat block
// order of each (KV head, row group) split over `waves` waves, one slot per
// (wave, sequence it touches).
struct WsLayout {
  size_t o, ml, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

inline WsLayout ws_layout(int64_t slots, int64_t NR, int64_t D) {
  WsLayout w;
  w.o = 0;
  w.ml = align256(w.o + (size_t)(slots * NR * D) * sizeof(float));
  w.total = align256(w.ml + (size_t)(slots * NR * 2) * sizeof(float));
  return w;
}

struct AttnArgs {
  LayerView lv;
  const uint16_t *q;  // [B][Hq][Lq][D] in q_dtype
  int32_t q_dtype;
  const int32_t *tables;
  const int32_t *lens;
  int32_t B, max_blocks;
  int32_t nb_cap;  // blocks per sequence the plan covers (from max_seq_len)
  int32_t Hkv, R, Lq, Hq, NR;
  float scale_log2;  // softmax scale * log2(e)
  int32_t split_blocks;
  int32_t row_groups, rows_per_group;  // query rows per wave (all NR on the VALU path)
  int32_t group_waves;  // row groups per workgroup (MFMA path; 1 on the VALU path)
  int32_t waves;  // workgroups per (KV head, row group)
  float *ws_o;
  float *ws_ml;
  void *out;  // [B][Hq][Lq][D]
  int32_t out_dtype;
  const uint16_t *k_new, *v_new;  // fused append of the newest token (null: none)
  int64_t kn_sb, kn_sh;           // their element strides (batch, head)
  // RoPE (null: none): queries and the newest K rows turn by their positions
  // (query row j of sequence b: lens[b] - Lq + j) with the fp32 table
  // rope_cs[rope_max_pos][D]
  const float *rope_cs;
  int32_t rope_max_pos;
  // element strides of q (batch, head, query position); default: [B][Hq][Lq][D]
  int64_t q_sb, q_sh, q_sj;
  int32_t len_const;     // >= 0: every sequence holds this many tokens (lens not read)
  int32_t causal;        // 1: query row j sees keys [0, len - Lq + j]; 0: every key
  int32_t partial_only;  // 1: every segment leaves a partial, none writes the output
  // sliding window (window > 0): query row j of sequence b sees keys
  // [max(win_start[b], len - Lq + j - window + 1), len - Lq + j]
  // (win_start null: 0)
  const int32_t *win_start;
  int32_t window;
};

inline AttnArgs make_attn_args(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p) {
  AttnArgs r;
  r.lv.base = g.base + (int64_t)layer * g.layer_stride;
  r.lv.block_stride = g.block_stride;
  r.lv.head_bytes = g.head_bytes;
  r.lv.num_blocks = g.num_blocks;
  r.q = static_cast<const uint16_t *>(a.q);
  r.q_dtype = g.in_dtype;
  r.tables = a.tables;
  r.lens = a.lens;
  r.B = a.B;
  r.max_blocks = a.max_blocks;
  r.nb_cap = p.nb_cap;
  r.Hkv = g.Hkv;
  r.R = a.Hq / g.Hkv;
  r.Lq = a.Lq;
  r.Hq = a.Hq;
  r.NR = p.NR;
  r.scale_log2 = a.scale * 1.4426950408889634f;
  r.split_blocks = p.split_blocks;
  r.row_groups = p.row_groups;
  r.rows_per_group = p.rows_per_group;
  r.group_waves = p.group_waves;
  r.waves = p.waves;
  const WsLayout w = ws_layout(p.slots, p.rows_per_group, g.D);
  uint8_t *base = static_cast<uint8_t *>(a.ws);
  r.ws_o = reinterpret_cast<float *>(base + w.o);
  r.ws_ml = reinterpret_cast<float *>(base + w.ml);
  r.out = a.out;
  r.out_dtype = a.out_dtype;
  r.k_new = static_cast<const uint16_t *>(a.k_new);
  r.v_new = static_cast<const uint16_t *>(a.v_new);
  r.kn_sb = a.kn_sb;
  r.kn_sh = a.kn_sh;
  r.rope_cs = a.rope_cs;
  r.rope_max_pos = a.rope_max_pos;
  if (a.q_strided) {
    r.q_sb = a.q_sb;
    r.q_sh = a.q_sh;
    r.q_sj = a.q_sj;
  } else {
    r.q_sj = g.D;
    r.q_sh = (int64_t)a.Lq * g.D;
    r.q_sb = (int64_t)a.Hq * a.Lq * g.D;
  }
  r.len_const = a.len_const;
  r.causal = a.causal;
  r.partial_only = a.partial_only;
  r.win_start = a.win_start;
  r.window = a.window;
  return r;
}

// Blocks of a sequence of length `len` that the kernels may touch: bounded by
// the table width and by the plan's per-sequence cap (from the host's
// max_seq_len), so a length beyond either bound can never index past the
// table or the workspace.
__device__ __forceinline__ int seq_blocks(const AttnArgs &a, int len) {
  int nb = len > 0 ? (len + 63) >> 6 : 0;
  nb = nb < a.max_blocks ? nb : a.max_blocks;
  return nb < a.nb_cap ? nb : a.nb_cap;
}

__device__ __forceinline__ float load_q(const uint16_t *p, int dt) {
  return dt == DT_BF16 ? bf16_bits_to_f32(*p) : f16_bits_to_f32(*p);
}

// RoPE table row of position `pos` (clamped into the table: positions come
// from device lengths the host bounds by max_seq_len <= rope_max_pos).
__device__ __forceinline__ const float *rope_row(const AttnArgs &a, int pos, int D) {
  pos = pos < 0 ? 0 : (pos >= a.rope_max_pos ? a.rope_max_pos - 1 : pos);
  return a.rope_cs + (int64_t)pos * D;
}

// RoPE of one row held as E = D/64 elements per lane (d = lane*E + e, dtype
// bits): MLX RoPE, traditional = false -- the partner of d is d +- D/2, in
// lane ^ 32 -- in fp32, each product and sum rounded once, then rounded to
// the dtype.  All 64 lanes must be active.
template <int D, int DT>
__device__ __forceinline__ void rope_row_lanes(uint16_t (&x)[D / 64], const float *crow) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const bool hi = lane >= 32;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    const float xv = elem_to_f32<DT>(x[e]);
    const float o = __shfl_xor(xv, 32, 64);
    const int i = (lane & 31) * E + e;
    const float c = crow[i], sn = crow[D / 2 + i];
    const float r = hi ? o * sn + xv * c : xv * c - o * sn;
    x[e] = DT == DT_BF16 ? f32_to_bf16_bits(r) : f32_to_f16_bits(r);
  }
}
// The same for a pair of dtype elements per word: lo holds elements (d, d+1),
// hi their partners (d + D/2, d + D/2 + 1); c2 / s2 the pair's cos / sin.
template <int DT>
__device__ __forceinline__ void rope_pair_words(uint32_t &lo, uint32_t &hi, float2 c2, float2 s2) {
  const float a0 = elem_to_f32<DT>((uint16_t)(lo & 0xffffu)), a1 = elem_to_f32<DT>((uint16_t)(lo >> 16));
  const float b0 = elem_to_f32<DT>((uint16_t)(hi & 0xffffu)), b1 = elem_to_f32<DT>((uint16_t)(hi >> 16));
  const float r0 = a0 * c2.x - b0 * s2.x, r1 = a1 * c2.y - b1 * s2.y;
  const float t0 = a0 * s2.x + b0 * c2.x, t1 = a1 * s2.y + b1 * c2.y;
  auto bits = [](float f) -> uint32_t { return DT == DT_BF16 ? f32_to_bf16_bits(f) : f32_to_f16_bits(f); };
  lo = bits(r0) | (bits(r1) << 16);
  hi = bits(t0) | (bits(t1) << 16);
}

// Tokens held by sequence b.
__device__ __forceinline__ int len_of(const AttnArgs &a, int b) { return a.len_const >= 0 ? a.len_const : a.lens[b]; }
// Sliding window: the kernels see each sequence from the block holding its
// first visible key, fb = max(start, len - Lq - window + 1, 0) / 64: length
// len - 64 fb, table entries from column fb, first retained key start - 64 fb.
__device__ __forceinline__ int win_first_block(const AttnArgs &a, int b, int len) {
  const int st = a.win_start ? a.win_start[b] : 0;
  const int lo = max(max(st, len - a.Lq - a.window + 1), 0);
  return min(lo >> 6, a.max_blocks);
}
// Length of sequence b as the kernels see it.
template <bool WIN>
__device__ __forceinline__ int seq_len_view(const AttnArgs &a, int b) {
  const int len = len_of(a, b);
  if constexpr (WIN) return len - 64 * win_first_block(a, b, len);
  return len;
}
__device__ __forceinline__ int seq_len_any(const AttnArgs &a, int b) {
  return a.window > 0 ? seq_len_view<true>(a, b) : len_of(a, b);
}
// Table column of the first block the kernels see and the first retained key
// relative to it (window only).
template <bool WIN>
__device__ __forceinline__ int table_offset(const AttnArgs &a, int b) {
  if constexpr (WIN) return win_first_block(a, b, len_of(a, b));
  return 0;
}
__device__ __forceinline__ int win_view_start(const AttnArgs &a, int b) {
  return (a.win_start ? a.win_start[b] : 0) - 64 * win_first_block(a, b, len_of(a, b));
}
// Query vector (head hq, position j) of sequence b.
__device__ __forceinline__ const uint16_t *q_row(const AttnArgs &a, int b, int hq, int j) {
  return a.q + (int64_t)b * a.q_sb + (int64_t)hq * a.q_sh + (int64_t)j * a.q_sj;
}
// Keys [0, lim) seen by query position j of a sequence of length len.
__device__ __forceinline__ int key_limit(const AttnArgs &a, int len, int j) {
  return a.causal ? len - a.Lq + j + 1 : len;
}

// Output / partial-result addressing.  Rows are r = j*R + h (query position
// j, head h inside the KV group).
__device__ __forceinline__ int64_t out_row_base(const AttnArgs &a, int b, int hk, int r, int D) {
  const int hq = hk * a.R + r % a.R, j = r / a.R;
  return (((int64_t)b * a.Hq + hq) * a.Lq + j) * D;
}

// Inclusive prefix sum over the 64 lanes of a wave.
__device__ __forceinline__ int wave_incl_scan(int v) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int t = __shfl_up(v, d, 64);
    if (lane >= d) v += t;
  }
  return v;
}

__device__ __forceinline__ int wave_allsum_int(int v) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) v += __shfl_xor(v, d, 64);
  return v;
}

// Blocks of a sequence of length len that row group rg reads: with several
// row groups (long query windows) a group stops at the block holding the
// last key its last row sees (causal window); a single group reads them all.
// The row groups of one workgroup (group_waves of them, sharing its LDS
// ring) read the same blocks: those of the workgroup's last row group.
__device__ __forceinline__ int seq_blocks_rg(const AttnArgs &a, int len, int rg) {
  const int nb = seq_blocks(a, len);
  if (a.row_groups <= 1 || !a.causal) return nb;
  const int gw = a.group_waves;
  const int rg_last = min(a.row_groups, (rg / gw + 1) * gw) - 1;
  const int rlast = min(a.NR, (rg_last + 1) * a.rows_per_group) - 1;
  const int lim = len - a.Lq + rlast / a.R + 1;
  const int nv = lim > 0 ? (lim + 63) >> 6 : 0;
  return nb < nv ? nb : nv;
}

// Flat block order of a (KV head, row group): the blocks of sequences 0, 1,
// .., B-1 one after another (T blocks).  Returns T and sets start_out /
// nb_out to the flat index of sequence b's first block and its block count.
// Uniform across the wave; one round of lens loads.
__device__ __forceinline__ int flat_total_and_start(const AttnArgs &a, int b, int rg, int &start_out, int &nb_out) {
  const int lane = threadIdx.x & 63;
  int carry = 0;
  for (int c0 = 0; c0 < a.B; c0 += 64) {
    const int bb = c0 + lane;
    const int nbv = bb < a.B ? seq_blocks_rg(a, seq_len_any(a, bb), rg) : 0;
    const int incl = wave_incl_scan(nbv) + carry;
    if (b >= c0 && b < c0 + 64) {
      start_out = __builtin_amdgcn_readlane(incl - nbv, b - c0);
      nb_out = __builtin_amdgcn_readlane(nbv, b - c0);
    }
    carry = __builtin_amdgcn_readlane(incl, 63);
  }
  return carry;
}
// The wave holding flat block i (T > 0 blocks over W waves).
__device__ __forceinline__ int flat_wave_of(int64_t i, int T, int W) { return (int)(i * W / T); }

}  // namespace krill
