// Arguments and workspace layout shared by the paged attention kernels
// (VALU and MFMA paths).
#pragma once

#include "kdev.hpp"
#include "launch.hpp"

namespace krill {

// Workspace carve-up, 256-byte aligned pieces:
//   o      float [B][Hkv][max_splits][NR][D]   unnormalised split outputs
//   ml     float [B][Hkv][max_splits][NR][2]   (running max m in log2 units, sum l)
//   q16    fp16  [B][Hkv][NR][D]               queries rounded to fp16 (VALU path)
//   qsum   float [B][Hkv][NR][G]               per scale group sums of q16
struct WsLayout {
  size_t o, ml, q16, qsum, total;
};

inline size_t align256(size_t x) { return (x + 255) & ~(size_t)255; }

inline WsLayout ws_layout(int64_t B, int64_t Hkv, int64_t max_splits, int64_t NR, int64_t D, int64_t G) {
  WsLayout w;
  w.o = 0;
  w.ml = align256(w.o + (size_t)(B * Hkv * max_splits * NR * D) * sizeof(float));
  w.q16 = align256(w.ml + (size_t)(B * Hkv * max_splits * NR * 2) * sizeof(float));
  w.qsum = align256(w.q16 + (size_t)(B * Hkv * NR * D) * sizeof(uint16_t));
  w.total = align256(w.qsum + (size_t)(B * Hkv * NR * G) * sizeof(float));
  return w;
}

struct AttnArgs {
  LayerView lv;
  const uint16_t *q;  // [B][Hq][Lq][D] in q_dtype
  int32_t q_dtype;
  const int32_t *tables;
  const int32_t *lens;
  int32_t max_blocks;
  int32_t Hkv, R, Lq, Hq, NR;
  float scale_log2;  // softmax scale * log2(e)
  int32_t split_blocks, max_splits;
  float *ws_o;
  float *ws_ml;
  uint16_t *q16;
  float *qsum;
  void *out;  // [B][Hq][Lq][D]
  int32_t out_dtype;
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
  r.max_blocks = a.max_blocks;
  r.Hkv = g.Hkv;
  r.R = a.Hq / g.Hkv;
  r.Lq = a.Lq;
  r.Hq = a.Hq;
  r.NR = p.NR;
  r.scale_log2 = a.scale * 1.4426950408889634f;
  r.split_blocks = p.split_blocks;
  r.max_splits = p.max_splits;
  const WsLayout w = ws_layout(a.B, g.Hkv, p.max_splits, p.NR, g.D, g.G);
  uint8_t *base = static_cast<uint8_t *>(a.ws);
  r.ws_o = reinterpret_cast<float *>(base + w.o);
  r.ws_ml = reinterpret_cast<float *>(base + w.ml);
  r.q16 = reinterpret_cast<uint16_t *>(base + w.q16);
  r.qsum = reinterpret_cast<float *>(base + w.qsum);
  r.out = a.out;
  r.out_dtype = a.out_dtype;
  return r;
}

// Blocks of sequence b that the kernels may touch: bounded by the table width
// and by the split grid sized from the host's max_seq_len, so a length beyond
// either bound can never index past the table or the workspace.
__device__ __forceinline__ int seq_blocks(const AttnArgs &a, int len) {
  int nb = (len + 63) >> 6;
  nb = nb < a.max_blocks ? nb : a.max_blocks;
  const int cap = a.max_splits * a.split_blocks;
  return nb < cap ? nb : cap;
}

__device__ __forceinline__ float load_q(const uint16_t *p, int dt) {
  return dt == DT_BF16 ? bf16_bits_to_f32(*p) : f16_bits_to_f32(*p);
}

// Output / partial-result addressing.  Rows are r = j*R + h (query position
// j, head h inside the KV group).
__device__ __forceinline__ int64_t out_row_base(const AttnArgs &a, int b, int hk, int r, int D) {
  const int hq = hk * a.R + r % a.R, j = r / a.R;
  return (((int64_t)b * a.Hq + hq) * a.Lq + j) * D;
}
__device__ __forceinline__ int64_t part_index(const AttnArgs &a, int b, int hk, int split, int r) {
  return (((int64_t)b * a.Hkv + hk) * a.max_splits + split) * a.NR + r;
}

}  // namespace krill
