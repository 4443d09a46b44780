// gfx950 kernels that write and read the paged int8 pool: fused
// quantize-append, gather (paged -> contiguous / left-padded snapshot),
// dequantizing gather, scatter (snapshot -> paged), block copy (COW), and
// the split-K merge of the attention kernels.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>

#include "attn_common.hpp"
#include "block_manager.hpp"
#include "kdev.hpp"
#include "launch.hpp"

namespace krill {

static inline LayerView layer_view(const PoolGeometry &g, int32_t layer) {
  LayerView lv;
  lv.base = g.base + (int64_t)layer * g.layer_stride;
  lv.block_stride = g.block_stride;
  lv.head_bytes = g.head_bytes;
  lv.num_blocks = g.num_blocks;
  return lv;
}

// ---------------------------------------------------------------------------
// Fused quantize + paged append (quantize_row / store_row: the reference's
// row quantizer or the affine group-64 one).  One wave64 per (row, K|V);
// each lane owns D/64 consecutive elements.
//
// RoPE (rope.pos set): K rows are rotated first, as MLX RoPE with
// traditional = false over all D dims (element i < D/2 pairs with i + D/2),
// at position pos[b * L + l] from the fp32 table cs[pos][D] (cos of angle i,
// then sin of angle i):
//   k'[i] = k[i] c_i - k[i + D/2] s_i,   k'[i + D/2] = k[i] s_i + k[i + D/2] c_i
// in fp32 (each product and sum rounded once), then rounded to the element
// dtype -- the bf16/f16 tensor the unfused path would hand to the quantizer.
// Rows whose position lies outside [0, max_pos) are not written (K nor V),
// like rows with a negative slot.
// ---------------------------------------------------------------------------
struct RopeArgs {
  const int32_t *pos;  // [B][L] token positions (null: no rotation)
  const float *cs;     // [max_pos][D]
  int32_t max_pos;
};

template <int D, int MODE, int DT, bool ROPE>
__global__ __launch_bounds__(256) void k_quantize_append(LayerView lv, const uint16_t *__restrict__ k,
                                                         const uint16_t *__restrict__ v, int64_t sb,
                                                         int64_t sh, int64_t sl,
                                                         const int32_t *__restrict__ slots, int32_t B,
                                                         int32_t L, int32_t Hkv, RopeArgs rope) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int64_t nrows = (int64_t)B * Hkv * L;
  if (wave >= 2 * nrows) return;
  const int kv = (int)(wave & 1);
  const int64_t row = wave >> 1;
  const int l = (int)(row % L);
  const int h = (int)((row / L) % Hkv);
  const int b = (int)(row / ((int64_t)L * Hkv));
  const int slot = slots[(int64_t)b * L + l];
  if (slot < 0) return;
  const int blk = slot >> 6, t = slot & 63;
  if (blk >= lv.num_blocks) return;
  const uint16_t *src = (kv ? v : k) + (int64_t)b * sb + (int64_t)h * sh + (int64_t)l * sl + lane * E;
  float x[E];
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = elem_to_f32<DT>(src[e]);
  if constexpr (ROPE) {
    const int p = rope.pos[(int64_t)b * L + l];
    if ((unsigned)p >= (unsigned)rope.max_pos) return;  // uniform per wave
    if (kv == 0) {
      // lane owns d = lane*E + e; its partner d +- D/2 sits in lane ^ 32
      const float *c = rope.cs + (int64_t)p * D;
      const bool hi = lane >= 32;
#pragma unroll
      for (int e = 0; e < E; ++e) {
        const int i = (lane & 31) * E + e;
        const float o = __shfl_xor(x[e], 32, 64);
        const float cv = c[i], sv = c[D / 2 + i];
        x[e] = round_dt<DT>(hi ? o * sv + x[e] * cv : x[e] * cv - o * sv);
      }
    }
  }
  uint8_t qb[E];
  float scale, zero;
  quantize_row<D, MODE, DT>(x, qb, scale, zero);
  store_row<D, MODE>(head_region(lv, blk, h), kv, t, lane, qb, scale, zero);
}

// Which of the 16 bytes of V piece `o` (byte offset inside the V region of
// a block) belong to tokens in the 64-bit token set `tm`: the piece holds
// positions p = 16 h .. 16 h + 15 of one d in token group tg, and position
// p = 16 h + x is token 32 tg + 8 h + 4 (x / 8) + x % 4 + 16 ((x / 4) % 2)
// (vtok, pool layout in kdev.hpp), so bytes 0-3, 4-7, 8-11 and 12-15 are
// tokens 32 tg + 8 h + {0..3, 16..19, 4..7, 20..23}.
template <int D>
__device__ __forceinline__ unsigned v_piece_mask(int o, uint64_t tm) {
  const int tg = o / (32 * D);
  const int h = ((o % (32 * D)) >> 10) & 1;  // (piece index / 64) % 2
  const uint64_t s = tm >> (32 * tg + 8 * h);
  return (unsigned)((s & 0xfu) | (((s >> 16) & 0xfu) << 4) | (((s >> 4) & 0xfu) << 8) | (((s >> 20) & 0xfu) << 12));
}

// Bulk append (prefill, chunked appends): one workgroup (256 threads) per
// (sequence, head, 64 consecutive rows).  Each thread quantizes one scale
// group of one row of K or V on its own (64 elements in affine mode, the
// whole row in the reference's row mode) with the same scalar steps as
// quantize_row (ref_safe_scale / ref_q, affine_w / affine_params / affine_q),
// so the bytes are the same as the per-row kernel's.  When the rows' slots
// are consecutive positions (the block manager hands them out that way) they
// fall into at most two blocks: K bytes (16-byte pieces per token) and the
// (scale, zero) words go straight to the pool, the transposed V rows to an
// LDS image of those blocks' V regions, whose new bytes are then written out
// in region order -- whole 16-byte pieces where every byte belongs to a new
// token, single bytes at the edges of the token range -- instead of one-byte
// scattered stores.  Other slot patterns (and slots < 0) store each group
// straight to its block.
template <int D, int MODE, int DT, bool ROPE>
__global__ __launch_bounds__(256) void k_quantize_append_blocks(LayerView lv, const uint16_t *__restrict__ k,
                                                                const uint16_t *__restrict__ v, int64_t sb,
                                                                int64_t sh, int64_t sl,
                                                                const int32_t *__restrict__ slots, int32_t L,
                                                                RopeArgs rope) {
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int GE = D / G;  // elements per scale group
  constexpr int VB = 64 * D;         // V bytes of a block (region offset v_offset(D))
  constexpr int ITEMS = 64 * G * 2;  // (row, group, K|V)
  __shared__ __attribute__((aligned(16))) uint8_t img[2][VB];
  const int tid = threadIdx.x, lane = tid & 63;
  const int h = blockIdx.y, b = blockIdx.z;
  const int l0 = blockIdx.x * 64;
  const int nrows = min(64, L - l0);
  const int32_t *srow = slots + (int64_t)b * L + l0;

  // the chunk's layout, computed by every wave (uniform)
  const int sv = lane < nrows ? srow[lane] : -1;
  const int pv = ROPE && lane < nrows ? rope.pos[(int64_t)b * L + l0 + lane] : 0;  // row's position
  const bool pos_ok = !ROPE || (unsigned)pv < (unsigned)rope.max_pos;
  const int prev = __shfl_up(sv, 1, 64);
  bool bad = lane < nrows && (sv < 0 || (sv >> 6) >= lv.num_blocks || !pos_ok);
  if (lane > 0 && lane < nrows && !bad && sv != prev + 1) bad = !((prev & 63) == 63 && (sv & 63) == 0);
  const bool brk = lane > 0 && lane < nrows && (sv >> 6) != (prev >> 6);
  const unsigned long long brks = __ballot(brk);
  const bool fast = __ballot(bad) == 0 && __popcll(brks) <= 1;
  const int slot0 = __builtin_amdgcn_readfirstlane(sv);
  const int nA = brks ? (int)__builtin_ctzll(brks) : nrows;  // rows in the first block
  const int blkA = slot0 >> 6, tA = slot0 & 63;
  const int blkB = brks ? __builtin_amdgcn_readlane(sv, nA) >> 6 : -1;

  // RoPE: the chunk's K rows rotated by the whole workgroup into LDS (four
  // pairs (i, i + D/2) per thread step, element dtype bits), then quantized
  // from there like unrotated rows from memory.
  __shared__ __attribute__((aligned(16))) uint16_t krot[ROPE ? 64 * D : 8];
  if constexpr (ROPE) {
    constexpr int QPR = D / 8;  // quads of pairs per row
#pragma unroll 1
    for (int q = tid; q < 64 * QPR; q += 256) {
      const int r = q / QPR, i4 = 4 * (q % QPR);
      const int p = __shfl(pv, r, 64);
      if (r >= nrows || (unsigned)p >= (unsigned)rope.max_pos) continue;
      const uint16_t *row = k + (int64_t)b * sb + (int64_t)h * sh + (int64_t)(l0 + r) * sl;
      const uint2 w1 = *reinterpret_cast<const uint2 *>(row + i4);
      const uint2 w2 = *reinterpret_cast<const uint2 *>(row + D / 2 + i4);
      const float4 c4 = *reinterpret_cast<const float4 *>(rope.cs + (int64_t)p * D + i4);
      const float4 s4 = *reinterpret_cast<const float4 *>(rope.cs + (int64_t)p * D + D / 2 + i4);
      const uint16_t a[4] = {(uint16_t)(w1.x & 0xffffu), (uint16_t)(w1.x >> 16), (uint16_t)(w1.y & 0xffffu),
                             (uint16_t)(w1.y >> 16)};
      const uint16_t c[4] = {(uint16_t)(w2.x & 0xffffu), (uint16_t)(w2.x >> 16), (uint16_t)(w2.y & 0xffffu),
                             (uint16_t)(w2.y >> 16)};
      const float cv[4] = {c4.x, c4.y, c4.z, c4.w}, sn[4] = {s4.x, s4.y, s4.z, s4.w};
      uint16_t o1[4], o2[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float x1 = elem_to_f32<DT>(a[j]), x2 = elem_to_f32<DT>(c[j]);
        const float y1 = x1 * cv[j] - x2 * sn[j], y2 = x1 * sn[j] + x2 * cv[j];
        o1[j] = DT == DT_BF16 ? f32_to_bf16_bits(y1) : f32_to_f16_bits(y1);
        o2[j] = DT == DT_BF16 ? f32_to_bf16_bits(y2) : f32_to_f16_bits(y2);
      }
      *reinterpret_cast<uint2 *>(krot + r * D + i4) =
          uint2{(uint32_t)o1[0] | ((uint32_t)o1[1] << 16), (uint32_t)o1[2] | ((uint32_t)o1[3] << 16)};
      *reinterpret_cast<uint2 *>(krot + r * D + D / 2 + i4) =
          uint2{(uint32_t)o2[0] | ((uint32_t)o2[1] << 16), (uint32_t)o2[2] | ((uint32_t)o2[3] << 16)};
    }
    __syncthreads();
  }

#pragma unroll 1
  for (int item = tid; item < ITEMS; item += 256) {
    const int kv = item / (64 * G), r = (item / G) % 64, g = item % G;
    // both reads before any lane leaves the iteration: a lane-crossing read
    // from a lane that is switched off returns 0, not that lane's value
    const int slot = __shfl(sv, r, 64);
    const int p = __shfl(pv, r, 64);
    if (r >= nrows || slot < 0 || (slot >> 6) >= lv.num_blocks) continue;
    if (ROPE && (unsigned)p >= (unsigned)rope.max_pos) continue;
    const int t = slot & 63;
    // K with RoPE: the group's rotated elements from the LDS copy (a branch
    // of its own, `kv` being the same for the whole wave: a pointer selected
    // between LDS and global memory would make every load a flat load)
    uint4 raw[GE / 8];
    if (ROPE && kv == 0) {
      const uint16_t *src = krot + r * D + g * GE;
#pragma unroll
      for (int c = 0; c < GE / 8; ++c) raw[c] = *reinterpret_cast<const uint4 *>(src + 8 * c);
    } else {
      const uint16_t *src = (kv ? v : k) + (int64_t)b * sb + (int64_t)h * sh + (int64_t)(l0 + r) * sl + g * GE;
#pragma unroll
      for (int c = 0; c < GE / 8; ++c) raw[c] = *reinterpret_cast<const uint4 *>(src + 8 * c);
    }
    auto elem = [&](int e) -> float {
      const uint4 w = raw[e >> 3];
      const uint32_t u = ((e & 7) >> 1) == 0 ? w.x : ((e & 7) >> 1) == 1 ? w.y : ((e & 7) >> 1) == 2 ? w.z : w.w;
      return elem_to_f32<DT>((uint16_t)((e & 1) ? (u >> 16) : (u & 0xffffu)));
    };
    uint32_t qw[GE / 4];
    float scale, zero;
    if constexpr (MODE == MODE_REF) {
      float mn = elem(0), mx = mn;
#pragma unroll
      for (int e = 1; e < GE; ++e) {
        mn = fminf(mn, elem(e));
        mx = fmaxf(mx, elem(e));
      }
      const float safe = ref_safe_scale<DT>(mn, mx);
      const float rs = __builtin_amdgcn_rcpf(safe);
#pragma unroll
      for (int c = 0; c < GE / 4; ++c) {
        uint32_t wv = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) wv |= (uint32_t)ref_q_r<DT>(elem(4 * c + e), mn, safe, rs) << (8 * e);
        qw[c] = wv;
      }
      scale = safe;
      zero = mn + 0.0f;  // a zero minimum is stored as +0 (min over +-0 depends on order)
    } else {
      // The group's elements rounded to fp16 (affine_w) are fp16 values: kept
      // as packed pairs (no second conversion for the quantize pass), their
      // minimum and maximum taken two at a time.
      half2_t wp[GE / 2];
#pragma unroll
      for (int c = 0; c < GE / 8; ++c) {
        const uint32_t u4[4] = {raw[c].x, raw[c].y, raw[c].z, raw[c].w};
#pragma unroll
        for (int j = 0; j < 4; ++j)
          wp[4 * c + j] = DT == DT_F16 ? u32_as_h2(u4[j])
                                       : half2_t{(_Float16)__builtin_bit_cast(float, u4[j] << 16),
                                                 (_Float16)__builtin_bit_cast(float, u4[j] & 0xffff0000u)};
      }
      half2_t mn2 = wp[0], mx2 = wp[0];
#pragma unroll
      for (int i = 1; i < GE / 2; ++i) {
        mn2 = __builtin_elementwise_min(mn2, wp[i]);
        mx2 = __builtin_elementwise_max(mx2, wp[i]);
      }
      const float wmin = fminf((float)mn2[0], (float)mn2[1]), wmax = fmaxf((float)mx2[0], (float)mx2[1]);
      // the packed values stay in registers for the second pass (the
      // compiler would otherwise redo both conversions per element there)
#pragma unroll
      for (int i = 0; i < GE / 2; ++i) asm volatile("; keep %0" : "+v"(wp[i]));
      affine_params(wmin, wmax, scale, zero);
      const float rs = __builtin_amdgcn_rcpf(scale);
#pragma unroll
      for (int c = 0; c < GE / 4; ++c) {
        const half2_t p0 = wp[2 * c], p1 = wp[2 * c + 1];
        const float w4[4] = {(float)p0[0], (float)p0[1], (float)p1[0], (float)p1[1]};
        qw[c] = affine_q4(w4, scale, zero, rs);
      }
    }
    uint8_t *reg = head_region(lv, slot >> 6, h);
    const int d0 = g * GE;
    if (kv == 0) {
#pragma unroll
      for (int c = 0; c < GE / 16; ++c)
        *reinterpret_cast<uint4 *>(reg + k_byte(t, d0 + 16 * c)) =
            uint4{qw[4 * c], qw[4 * c + 1], qw[4 * c + 2], qw[4 * c + 3]};
    } else {
      // V: into the LDS image of the block's V region or straight to the block.
      // Offsets are taken relative to the V region (v_byte - v_offset, in
      // [0, 64 D)): an LDS pointer moved below its array would wrap in the
      // 32-bit LDS address space.  The two destinations stay in separate
      // branches (`fast` is uniform): one pointer selected between them would
      // be a generic address, and every byte would go out as a flat store
      // through the vector-memory path instead of an LDS write.
      if (fast) {
        uint8_t *vimg = img[r < nA ? 0 : 1];
#pragma unroll
        for (int e = 0; e < GE; ++e) vimg[v_byte(D, t, d0 + e) - v_offset(D)] = (uint8_t)(qw[e >> 2] >> (8 * (e & 3)));
      } else {
        uint8_t *vdst = reg + v_offset(D);
#pragma unroll
        for (int e = 0; e < GE; ++e) vdst[v_byte(D, t, d0 + e) - v_offset(D)] = (uint8_t)(qw[e >> 2] >> (8 * (e & 3)));
      }
    }
    const uint32_t meta = (uint32_t)f32_to_f16_bits(scale) | ((uint32_t)f32_to_f16_bits(zero) << 16);
    *reinterpret_cast<uint32_t *>(reg + (kv ? vm_offset(D, G) : km_offset(D)) + ((t * G + g) << 2)) = meta;
  }
  if (!fast) return;  // uniform across the workgroup
  __syncthreads();

  // V write-out in region order: block A holds tokens [tA, tA + nA), block B [0, nrows - nA)
#pragma unroll 1
  for (int ib = 0; ib < (blkB >= 0 ? 2 : 1); ++ib) {
    const int tlo = ib == 0 ? tA : 0, thi = ib == 0 ? tA + nA : nrows - nA;
    // tokens [tlo, thi) as a bit set (thi <= 64)
    const uint64_t tm = (thi >= 64 ? ~0ull : ((1ull << thi) - 1ull)) & ~((1ull << tlo) - 1ull);
    uint8_t *reg = head_region(lv, ib == 0 ? blkA : blkB, h) + v_offset(D);
    const uint8_t *im = img[ib];
#pragma unroll 1
    for (int q = tid; q < VB / 16; q += 256) {
      const int o = q * 16;
      const unsigned mask = v_piece_mask<D>(o, tm);
      if (mask == 0xffffu) {
        *reinterpret_cast<uint4 *>(reg + o) = *reinterpret_cast<const uint4 *>(im + o);
      } else if (mask) {
#pragma unroll
        for (int x = 0; x < 16; ++x)
          if (mask & (1u << x)) reg[o + x] = im[o + x];
      }
    }
  }
}

// Append of each sequence's newest token, its position len - 1 located
// through the block table (the decode step: lens count the new token).  A
// token outside the blocks the attention reads (len = 0, or a block beyond
// the table width / max_seq_len) is not written; this is the rule the fused
// decode kernel follows too.  One wave64 per (sequence, head, K|V).
template <int D, int MODE, int DT>
__global__ __launch_bounds__(256) void k_append_newest(AttnArgs a) {
  constexpr int E = D / 64;
  const int lane = threadIdx.x & 63;
  const int64_t wave = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (wave >= 2 * (int64_t)a.B * a.Hkv) return;
  const int kv = (int)(wave & 1);
  const int h = (int)((wave >> 1) % a.Hkv);
  const int b = (int)((wave >> 1) / a.Hkv);
  const int len = a.lens[b];
  const int nb = seq_blocks(a, len);
  if (nb == 0 || ((len - 1) >> 6) != nb - 1) return;
  const int phys = a.tables[(int64_t)b * a.max_blocks + nb - 1];
  if ((unsigned)phys >= (unsigned)a.lv.num_blocks) return;
  const uint16_t *src = (kv ? a.v_new : a.k_new) + (int64_t)b * a.kn_sb + (int64_t)h * a.kn_sh + lane * E;
  uint16_t raw[E];
#pragma unroll
  for (int e = 0; e < E; ++e) raw[e] = src[e];
  if (a.rope_cs && kv == 0) rope_row_lanes<D, DT>(raw, rope_row(a, len - 1, D));
  float x[E];
#pragma unroll
  for (int e = 0; e < E; ++e) x[e] = elem_to_f32<DT>(raw[e]);
  uint8_t qb[E];
  float scale, zero;
  quantize_row<D, MODE, DT>(x, qb, scale, zero);
  store_row<D, MODE>(head_region(a.lv, phys, h), kv, (len - 1) & 63, lane, qb, scale, zero);
}

// ---------------------------------------------------------------------------
// Gather: paged -> [B][H][S_out][D] u8 + [B][H][S_out][G] f16 x4.
// left_pad = 1 reproduces stackCachesLeftPaddedQuantized
// (Sources/KrillEngine/BatchedDecode.swift:96-151): right-aligned rows,
// u8 0 / fp16 0 padding.  left_pad = 0 is quantizedSnapshot() with a zero tail.
// ---------------------------------------------------------------------------

// One workgroup per (token block, head, sequence): the block's K chunks go
// out as 16-byte pieces (token t, d 16c..16c+15: contiguous in the pool's
// chunk-major K and in the output row), V goes through LDS (the pool holds it
// transposed), metadata as (scale, zero) words.  Rows that no token of the
// block lands on are left to the zero workgroups (blockIdx.x >= nbx), which
// clear every output row outside the sequence's token range.  A block whose
// table entry is out of range (or beyond max_blocks) gives zero rows, as a
// row gather would.
template <int D, int G>
__global__ __launch_bounds__(256) void k_gather(LayerView lv, const int32_t *__restrict__ tables,
                                                const int32_t *__restrict__ lens, int32_t H, int32_t max_blocks,
                                                int32_t S_out, int32_t left_pad, int32_t nbx, uint8_t *keys,
                                                uint8_t *values, uint16_t *ks, uint16_t *kz, uint16_t *vs,
                                                uint16_t *vz) {
  constexpr int CH = D / 16;  // 16-byte pieces per row
  constexpr int VB = 64 * D;  // V bytes of one (block, head)
  __shared__ __attribute__((aligned(16))) uint8_t vl[VB];
  const int x = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int len = lens[b];
  const int off = left_pad ? S_out - len : 0;  // output row of token ti: ti + off
  const int t_lo = max(0, -off), t_hi = min(len, S_out - off);
  const int64_t row0 = ((int64_t)b * H + h) * S_out;  // first output row of (b, h)
  const uint4 zero4 = {0u, 0u, 0u, 0u};
  if (x >= nbx) {  // zero rows: output rows with no token
    const int s0 = (x - nbx) * 64;
    for (int p = tid; p < 64 * CH; p += 256) {
      const int s = s0 + p / CH, c = p % CH;
      const int ti = s - off;
      if (s < S_out && (ti < t_lo || ti >= t_hi)) {
        *reinterpret_cast<uint4 *>(keys + (row0 + s) * D + 16 * c) = zero4;
        *reinterpret_cast<uint4 *>(values + (row0 + s) * D + 16 * c) = zero4;
      }
    }
    for (int p = tid; p < 64 * G; p += 256) {
      const int s = s0 + p / G, g = p % G;
      const int ti = s - off;
      if (s < S_out && (ti < t_lo || ti >= t_hi)) {
        const int64_t m = (row0 + s) * G + g;
        ks[m] = kz[m] = vs[m] = vz[m] = 0;
      }
    }
    return;
  }
  if (t_hi <= t_lo) return;
  const int j = (t_lo >> 6) + x;  // token block of this workgroup
  const int ta = max(64 * j, t_lo), tb = min(64 * j + 64, t_hi);
  if (ta >= tb) return;
  const int blk = j < max_blocks ? tables[(int64_t)b * max_blocks + j] : -1;
  const bool valid = (unsigned)blk < (unsigned)lv.num_blocks;  // uniform over the workgroup
  const uint8_t *reg = valid ? head_region(lv, blk, h) : nullptr;
  if (valid) {  // V region into LDS, 16 bytes per thread and step
    for (int p = tid; p < VB / 16; p += 256)
      *reinterpret_cast<uint4 *>(vl + 16 * p) = *reinterpret_cast<const uint4 *>(reg + v_offset(D) + 16 * p);
  }
  __syncthreads();
  for (int p = tid; p < 64 * CH; p += 256) {
    const int t = p / CH, c = p % CH;
    const int ti = 64 * j + t;
    if (ti < ta || ti >= tb) continue;
    const int64_t o = (row0 + ti + off) * D + 16 * c;
    uint4 kq = zero4, vq = zero4;
    if (valid) {
      kq = *reinterpret_cast<const uint4 *>(reg + k_byte(t, 16 * c));
      uint32_t w[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) acc |= (uint32_t)vl[v_byte(D, t, 16 * c + 4 * q + e) - v_offset(D)] << (8 * e);
        w[q] = acc;
      }
      vq = uint4{w[0], w[1], w[2], w[3]};
    }
    *reinterpret_cast<uint4 *>(keys + o) = kq;
    *reinterpret_cast<uint4 *>(values + o) = vq;
  }
  for (int p = tid; p < 64 * G; p += 256) {
    const int t = p / G, g = p % G;
    const int ti = 64 * j + t;
    if (ti < ta || ti >= tb) continue;
    uint32_t km = 0, vm = 0;
    if (valid) {
      km = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + ((t * G + g) << 2));
      vm = *reinterpret_cast<const uint32_t *>(reg + vm_offset(D, G) + ((t * G + g) << 2));
    }
    const int64_t m = (row0 + ti + off) * G + g;
    ks[m] = (uint16_t)(km & 0xffffu);
    kz[m] = (uint16_t)(km >> 16);
    vs[m] = (uint16_t)(vm & 0xffffu);
    vz[m] = (uint16_t)(vm >> 16);
  }
}

// Dequantizing gather: fp16 K/V [B][H][S_out][D].
// MODE_REF: f16(f16(f16(q) * s) + z), the two roundings of
// QuantizedKVCache.dequantize (QuantizedKVCache.swift:200-204).
// MODE_AFFINE: f16(s*q + b) rounded once.
// Tiled as k_gather: one workgroup per (token block, head, sequence), 16 K
// or V bytes (one scale group) -> 16 fp16 per piece, V through LDS; zero
// workgroups clear the rows without a token.
template <int D, int G, int MODE>
__device__ __forceinline__ void dequant16(const uint8_t (&qb)[16], uint32_t meta, uint16_t *dst) {
  const float sc = f16_bits_to_f32((uint16_t)(meta & 0xffffu)), zr = f16_bits_to_f32((uint16_t)(meta >> 16));
  uint32_t w[8];
#pragma unroll
  for (int e = 0; e < 16; e += 2) {
    uint16_t o[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const float q = (float)qb[e + u];
      if constexpr (MODE == MODE_REF)
        o[u] = f32_to_f16_bits(f16_bits_to_f32(f32_to_f16_bits(q * sc)) + zr);
      else
        o[u] = f32_to_f16_bits(sc * q + zr);
    }
    w[e / 2] = (uint32_t)o[0] | ((uint32_t)o[1] << 16);
  }
  reinterpret_cast<uint4 *>(dst)[0] = uint4{w[0], w[1], w[2], w[3]};
  reinterpret_cast<uint4 *>(dst)[1] = uint4{w[4], w[5], w[6], w[7]};
}

template <int D, int G, int MODE>
__global__ __launch_bounds__(256) void k_gather_dequant(LayerView lv, const int32_t *__restrict__ tables,
                                                        const int32_t *__restrict__ lens, int32_t H,
                                                        int32_t max_blocks, int32_t S_out, int32_t left_pad,
                                                        int32_t nbx, uint16_t *k_out, uint16_t *v_out) {
  constexpr int CH = D / 16;
  constexpr int VB = 64 * D;
  constexpr int DG = D / G;  // dims per scale group (a multiple of 16)
  __shared__ __attribute__((aligned(16))) uint8_t vl[VB];
  const int x = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x;
  const int len = lens[b];
  const int off = left_pad ? S_out - len : 0;
  const int t_lo = max(0, -off), t_hi = min(len, S_out - off);
  const int64_t row0 = ((int64_t)b * H + h) * S_out;
  const uint4 zero4 = {0u, 0u, 0u, 0u};
  if (x >= nbx) {
    const int s0 = (x - nbx) * 64;
    for (int p = tid; p < 64 * CH; p += 256) {
      const int s = s0 + p / CH, c = p % CH;
      const int ti = s - off;
      if (s < S_out && (ti < t_lo || ti >= t_hi)) {
        uint4 *kd = reinterpret_cast<uint4 *>(k_out + (row0 + s) * D + 16 * c);
        uint4 *vd = reinterpret_cast<uint4 *>(v_out + (row0 + s) * D + 16 * c);
        kd[0] = kd[1] = vd[0] = vd[1] = zero4;
      }
    }
    return;
  }
  if (t_hi <= t_lo) return;
  const int j = (t_lo >> 6) + x;
  const int ta = max(64 * j, t_lo), tb = min(64 * j + 64, t_hi);
  if (ta >= tb) return;
  const int blk = j < max_blocks ? tables[(int64_t)b * max_blocks + j] : -1;
  const bool valid = (unsigned)blk < (unsigned)lv.num_blocks;
  const uint8_t *reg = valid ? head_region(lv, blk, h) : nullptr;
  if (valid) {
    for (int p = tid; p < VB / 16; p += 256)
      *reinterpret_cast<uint4 *>(vl + 16 * p) = *reinterpret_cast<const uint4 *>(reg + v_offset(D) + 16 * p);
  }
  __syncthreads();
  for (int p = tid; p < 64 * CH; p += 256) {
    const int t = p / CH, c = p % CH;
    const int ti = 64 * j + t;
    if (ti < ta || ti >= tb) continue;
    uint16_t *kd = k_out + (row0 + ti + off) * D + 16 * c;
    uint16_t *vd = v_out + (row0 + ti + off) * D + 16 * c;
    if (!valid) {
      reinterpret_cast<uint4 *>(kd)[0] = reinterpret_cast<uint4 *>(kd)[1] = zero4;
      reinterpret_cast<uint4 *>(vd)[0] = reinterpret_cast<uint4 *>(vd)[1] = zero4;
      continue;
    }
    const int g = (16 * c) / DG;
    const uint32_t km = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + ((t * G + g) << 2));
    const uint32_t vm = *reinterpret_cast<const uint32_t *>(reg + vm_offset(D, G) + ((t * G + g) << 2));
    const uint4 kq4 = *reinterpret_cast<const uint4 *>(reg + k_byte(t, 16 * c));
    uint8_t kq[16], vq[16];
    __builtin_memcpy(kq, &kq4, 16);
#pragma unroll
    for (int e = 0; e < 16; ++e) vq[e] = vl[v_byte(D, t, 16 * c + e) - v_offset(D)];
    dequant16<D, G, MODE>(kq, km, kd);
    dequant16<D, G, MODE>(vq, vm, vd);
  }
}

// ---------------------------------------------------------------------------
// Scatter: snapshot rows [src_start[b], +L) -> slots[b][0..L).  Inverse of the
// gather; restoreQuantized (QuantizedKVCache.swift:122-129) and the int8
// scatterBack slice (ContinuousBatcher.swift:743-801).
// ---------------------------------------------------------------------------
// One workgroup per (64-row chunk of the source rows, head, sequence).  A
// chunk whose 64 slots are one whole block in order (a restore into fresh
// blocks) is written block-wise: K as 16-byte pieces, V rows staged in LDS
// and written in the pool's transposed order as 16-byte pieces, metadata as
// words.  Any other chunk goes row by row (one wave per row, byte stores).
// Slots < 0 and source rows outside [0, S_in) are skipped.
template <int D, int G>
__global__ __launch_bounds__(256) void k_scatter(LayerView lv, const uint8_t *__restrict__ keys,
                                                 const uint8_t *__restrict__ values,
                                                 const uint16_t *__restrict__ ks, const uint16_t *__restrict__ kz,
                                                 const uint16_t *__restrict__ vs, const uint16_t *__restrict__ vz,
                                                 int32_t H, int32_t S_in, const int32_t *__restrict__ src_start,
                                                 const int32_t *__restrict__ slots, int32_t L) {
  constexpr int E = D / 64;
  constexpr int CH = D / 16;  // 16-byte pieces per row
  constexpr int VB = 64 * D;  // V bytes of one (block, head)
  __shared__ __attribute__((aligned(16))) uint8_t vrow[VB];  // V rows [token][D]
  __shared__ int whole_s;
  const int x = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int tid = threadIdx.x, lane = tid & 63;
  const int i0 = 64 * x;
  const int sst = src_start[b];
  if (tid < 64) {  // wave 0, all lanes: is the chunk one whole block in order?
    const int i = i0 + tid;
    const int slot = i < L ? slots[(int64_t)b * L + i] : -1;
    const int base = __shfl(slot, 0, 64);
    const bool ok = i < L && sst + i >= 0 && sst + i < S_in && base >= 0 && (base & 63) == 0 &&
                    (base >> 6) < lv.num_blocks && slot == base + tid;
    const bool all = __all(ok);
    if (tid == 0) whole_s = all ? 1 : 0;
  }
  __syncthreads();
  if (whole_s) {
    uint8_t *reg = head_region(lv, slots[(int64_t)b * L + i0] >> 6, h);
    const int64_t row0 = ((int64_t)b * H + h) * S_in + sst + i0;  // snapshot row of the chunk's first token
    for (int p = tid; p < 64 * CH; p += 256) {
      const int t = p & 63, c = p >> 6;
      *reinterpret_cast<uint4 *>(reg + k_byte(t, 16 * c)) =
          *reinterpret_cast<const uint4 *>(keys + (row0 + t) * D + 16 * c);
      *reinterpret_cast<uint4 *>(vrow + t * D + 16 * c) =
          *reinterpret_cast<const uint4 *>(values + (row0 + t) * D + 16 * c);
    }
    for (int p = tid; p < 64 * G; p += 256) {
      const int t = p / G, g = p % G;
      const int64_t m = (row0 + t) * G + g;
      *reinterpret_cast<uint32_t *>(reg + km_offset(D) + ((t * G + g) << 2)) =
          (uint32_t)ks[m] | ((uint32_t)kz[m] << 16);
      *reinterpret_cast<uint32_t *>(reg + vm_offset(D, G) + ((t * G + g) << 2)) =
          (uint32_t)vs[m] | ((uint32_t)vz[m] << 16);
    }
    __syncthreads();
    // 16-byte piece q of the V region: token group tg, half hi (positions
    // 16 hi .. 16 hi + 15), d = (q % 64) * E + (sel >> 1)  (v_pos_byte)
    for (int q = tid; q < VB / 16; q += 256) {
      const int tg = q / (2 * D), r = q % (2 * D);
      const int sel = r >> 6, hi = sel & 1, d = (r & 63) * E + (sel >> 1);
      uint32_t w[4];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        uint32_t acc = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int tok = 32 * tg + vtok(16 * hi + 4 * qq + e);
          acc |= (uint32_t)vrow[tok * D + d] << (8 * e);
        }
        w[qq] = acc;
      }
      *reinterpret_cast<uint4 *>(reg + v_offset(D) + 16 * q) = uint4{w[0], w[1], w[2], w[3]};
    }
    return;
  }
  for (int i = i0 + (tid >> 6); i < min(i0 + 64, L); i += 4) {  // row by row, one wave per row
    const int slot = slots[(int64_t)b * L + i];
    const int st = sst + i;
    if (slot < 0 || st < 0 || st >= S_in) continue;
    const int blk = slot >> 6, t = slot & 63;
    if (blk >= lv.num_blocks) continue;
    const int64_t row = ((int64_t)b * H + h) * S_in + st;
    uint8_t *reg = head_region(lv, blk, h);
#pragma unroll
    for (int e = 0; e < E; ++e) {
      const int d = lane * E + e;
      reg[k_byte(t, d)] = keys[row * D + d];
      reg[v_byte(D, t, d)] = values[row * D + d];
    }
    if (lane < G) {
      const uint32_t km = (uint32_t)ks[row * G + lane] | ((uint32_t)kz[row * G + lane] << 16);
      const uint32_t vm = (uint32_t)vs[row * G + lane] | ((uint32_t)vz[row * G + lane] << 16);
      *reinterpret_cast<uint32_t *>(reg + km_offset(D) + ((t * G + lane) << 2)) = km;
      *reinterpret_cast<uint32_t *>(reg + vm_offset(D, G) + ((t * G + lane) << 2)) = vm;
    }
  }
}

// ---------------------------------------------------------------------------
// Whole-block copies (copy-on-write), every layer: one workgroup per
// (pair, layer) streaming block_stride bytes with 16-byte accesses.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void k_copy_blocks(uint8_t *base, int64_t layer_stride, int64_t block_stride,
                                                     int32_t num_blocks, int32_t num_layers,
                                                     const int32_t *__restrict__ src_dst, int32_t n) {
  const int pair = blockIdx.x / num_layers, layer = blockIdx.x % num_layers;
  if (pair >= n) return;
  const int src = src_dst[2 * pair], dst = src_dst[2 * pair + 1];
  if ((unsigned)src >= (unsigned)num_blocks || (unsigned)dst >= (unsigned)num_blocks || src == dst) return;
  const uint4 *s = reinterpret_cast<const uint4 *>(base + layer * layer_stride + src * block_stride);
  uint4 *d = reinterpret_cast<uint4 *>(base + layer * layer_stride + dst * block_stride);
  const int64_t n16 = block_stride >> 4;
  for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) d[i] = s[i];
}

// Same copy with up to 64 (src, dst) pairs passed by value in the kernel
// arguments, for copy-on-write pairs queued by the host block manager.
struct CopyPairsArg {
  int32_t n;
  int32_t sd[2 * 64];
};
__global__ __launch_bounds__(256) void k_copy_pairs(uint8_t *base, int64_t layer_stride, int64_t block_stride,
                                                    int32_t num_blocks, int32_t num_layers, CopyPairsArg pa) {
  const int pair = blockIdx.x / num_layers, layer = blockIdx.x % num_layers;
  if (pair >= pa.n) return;
  const int src = pa.sd[2 * pair], dst = pa.sd[2 * pair + 1];
  if ((unsigned)src >= (unsigned)num_blocks || (unsigned)dst >= (unsigned)num_blocks || src == dst) return;
  const uint4 *s = reinterpret_cast<const uint4 *>(base + layer * layer_stride + src * block_stride);
  uint4 *d = reinterpret_cast<uint4 *>(base + layer * layer_stride + dst * block_stride);
  const int64_t n16 = block_stride >> 4;
  for (int64_t i = threadIdx.x; i < n16; i += blockDim.x) d[i] = s[i];
}

// ---------------------------------------------------------------------------
// Merge of attention partials (log2-domain running max m, sum l, unnormalised
// o) into the output.  One wave per (row, kv-head, sequence).  Partials that
// saw no visible key carry m = -inf and contribute nothing.
// ---------------------------------------------------------------------------
// Combines the n consecutive partial slots starting at `slot0` for row r.
// Merge of the n consecutive partial slots slot0 .. slot0+n-1 of one query
// row (row rr of RR rows per slot) into the output row at obase.  The (m, l)
// pairs of the first 64 slots (lane s: slot s) and the o vectors of the
// first K0 slots (32 registers' worth) are loaded in one round; later slots
// (rare) loop.
template <int D>
__device__ __forceinline__ void merge_slots(const AttnArgs &a, int64_t slot0, int n, int rr, int RR, int64_t obase) {
  constexpr int E = D / 64;  // d = lane + 64 e
  constexpr int K0 = 32 / E;
  __shared__ float w_lds[64];
  const int lane = threadIdx.x;
  const float2 *ml2 = reinterpret_cast<const float2 *>(a.ws_ml);
  auto orow = [&](int k) { return a.ws_o + ((slot0 + k) * RR + rr) * (int64_t)D + lane; };
  float2 ml = lane < n ? ml2[(slot0 + lane) * RR + rr] : float2{-INFINITY, 0.0f};
  float ov[K0][E];
#pragma unroll
  for (int k = 0; k < K0; ++k)
#pragma unroll
    for (int e = 0; e < E; ++e) ov[k][e] = k < n ? orow(k)[64 * e] : 0.0f;
  float M = ml.x;
  for (int s0 = 64; s0 < n; s0 += 64)
    if (s0 + lane < n) M = fmaxf(M, ml2[(slot0 + s0 + lane) * RR + rr].x);
  M = wave_allmax(M);
  float acc[E], lpart = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.0f;
  for (int s0 = 0; s0 < n; s0 += 64) {
    const int cnt = min(64, n - s0);
    if (s0 > 0) ml = lane < cnt ? ml2[(slot0 + s0 + lane) * RR + rr] : float2{-INFINITY, 0.0f};
    const float w = lane < cnt && ml.x != -INFINITY ? fast_exp2(ml.x - M) : 0.0f;
    lpart += w * ml.y;
    w_lds[lane] = w;
    __syncthreads();
    int k = 0;
    if (s0 == 0) {
#pragma unroll
      for (int kk = 0; kk < K0; ++kk) {
        const float wk = kk < cnt ? w_lds[kk] : 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] += wk * ov[kk][e];
      }
      k = K0;
    }
#pragma unroll 4
    for (; k < cnt; ++k) {
      const float wk = w_lds[k];
      const float *op = orow(s0 + k);
#pragma unroll
      for (int e = 0; e < E; ++e) acc[e] += wk * op[64 * e];
    }
    __syncthreads();
  }
  const float Lsum = uniform_f32(wave_allsum(lpart));  // lane 0's rounding of the sum in every lane
  const float inv = (M == -INFINITY || !(Lsum > 0.0f)) ? 0.0f : 1.0f / Lsum;
#pragma unroll
  for (int e = 0; e < E; ++e) store_out(a.out, obase + lane + 64 * e, acc[e] * inv, a.out_dtype);
}

// After either attention kernel (flat block order per (KV head, row group),
// T blocks split evenly over the waves): sequence b's blocks are flat
// [s, s + nb), covered by waves flat_wave_of(s) .. flat_wave_of(s + nb - 1),
// whose partials sit in consecutive slots wave + b.  A sequence inside one
// wave was written by the attention kernel; one with no blocks for this row
// gets zeros here.
template <int D>
__global__ __launch_bounds__(64) void k_attn_merge_flat(AttnArgs a) {
  const int r = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int lane = threadIdx.x;
  const int64_t obase = out_row_base(a, b, hk, r, D);
  const int rg = r / a.rows_per_group, rr = r % a.rows_per_group;
  int s = 0, nb = 0;
  const int T = flat_total_and_start(a, b, rg, s, nb);
  if (nb == 0) {
#pragma unroll
    for (int e = 0; e < D / 64; ++e) store_out(a.out, obase + lane + 64 * e, 0.0f, a.out_dtype);
    return;
  }
  const int Wt = min(a.waves, T);  // waves that took part (each holds >= 1 block)
  const int first = flat_wave_of(s, T, Wt), last = flat_wave_of(s + nb - 1, T, Wt);
  if (first == last) return;
  const int64_t slot0 = ((int64_t)hk * a.row_groups + rg) * (a.waves + a.B) + first + b;
  merge_slots<D>(a, slot0, last - first + 1, rr, a.rows_per_group, obase);
}

// Shared-prefix cascade: sequence b's keys are the P shared prefix blocks
// followed by its own suffix blocks.  The prefix pass attends every
// sequence's query rows to the prefix once (one virtual sequence of length
// 64 P whose query positions are the B sequences, no causal window), the
// suffix pass each sequence to its suffix; both leave partials only.  This
// kernel combines, per (row h, KV head, sequence b), the prefix pass's
// partials of row b*R + h (one per wave of its split) with the suffix pass's
// partials of row h -- the same softmax merge as k_attn_merge_flat, over two
// lists of slots.
struct MergeSrc {
  const float *o, *ml;
  int64_t slot0;
  int n, rr, RR;
};

template <int D>
__device__ __forceinline__ void merge_two(const MergeSrc (&src)[2], void *out, int64_t obase, int out_dtype) {
  constexpr int E = D / 64;  // d = lane + 64 e
  __shared__ float w_lds[64];
  const int lane = threadIdx.x;
  const int n = src[0].n + src[1].n;
  auto part = [&](int k, const float **o, const float2 **ml) {
    const int i = k < src[0].n ? 0 : 1;
    const int64_t slot = src[i].slot0 + (i ? k - src[0].n : k);
    const int64_t pi = slot * src[i].RR + src[i].rr;
    *o = src[i].o + pi * D;
    *ml = reinterpret_cast<const float2 *>(src[i].ml) + pi;
  };
  float M = -INFINITY;
  for (int k0 = 0; k0 < n; k0 += 64)
    if (k0 + lane < n) {
      const float *o;
      const float2 *ml;
      part(k0 + lane, &o, &ml);
      M = fmaxf(M, ml->x);
    }
  M = uniform_f32(wave_allmax(M));
  float acc[E], lpart = 0.0f;
#pragma unroll
  for (int e = 0; e < E; ++e) acc[e] = 0.0f;
  for (int k0 = 0; k0 < n; k0 += 64) {
    const int cnt = min(64, n - k0);
    float w = 0.0f;
    if (lane < cnt) {
      const float *o;
      const float2 *ml;
      part(k0 + lane, &o, &ml);
      const float2 v = *ml;
      w = v.x != -INFINITY ? fast_exp2(v.x - M) : 0.0f;
      lpart += w * v.y;
    }
    w_lds[lane] = w;
    __syncthreads();
    // 16 partial rows in flight at a time: their loads all issue before the
    // sums that use them
    constexpr int KC = 16;
    for (int k1 = 0; k1 < cnt; k1 += KC) {
      float ov[KC][E];
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const float *o;
        const float2 *ml;
        part(k0 + min(k1 + j, cnt - 1), &o, &ml);
#pragma unroll
        for (int e = 0; e < E; ++e) ov[j][e] = o[lane + 64 * e];
      }
#pragma unroll
      for (int j = 0; j < KC; ++j) {
        const float wk = k1 + j < cnt ? w_lds[k1 + j] : 0.0f;
#pragma unroll
        for (int e = 0; e < E; ++e) acc[e] += wk * ov[j][e];
      }
    }
    __syncthreads();
  }
  const float Lsum = uniform_f32(wave_allsum(lpart));
  const float inv = (M == -INFINITY || !(Lsum > 0.0f)) ? 0.0f : 1.0f / Lsum;
#pragma unroll
  for (int e = 0; e < E; ++e) store_out(out, obase + lane + 64 * e, acc[e] * inv, out_dtype);
}

template <int D>
__global__ __launch_bounds__(64) void k_attn_merge_cascade(AttnArgs ap, AttnArgs as) {
  const int h = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  MergeSrc src[2];
  // prefix pass: row b * R + h of the single virtual sequence, split over
  // min(waves, P) waves (every row group reads all P blocks)
  {
    const int rp = b * ap.R + h;
    const int rg = rp / ap.rows_per_group;
    const int Tp = seq_blocks(ap, ap.len_const);
    src[0].o = ap.ws_o;
    src[0].ml = ap.ws_ml;
    src[0].rr = rp % ap.rows_per_group;
    src[0].RR = ap.rows_per_group;
    src[0].slot0 = ((int64_t)hk * ap.row_groups + rg) * (ap.waves + 1);
    src[0].n = Tp > 0 ? min(ap.waves, Tp) : 0;
  }
  // suffix pass: sequence b's waves, row h
  {
    const int rg = h / as.rows_per_group;
    int s = 0, nb = 0;
    const int T = flat_total_and_start(as, b, rg, s, nb);
    src[1].o = as.ws_o;
    src[1].ml = as.ws_ml;
    src[1].rr = h % as.rows_per_group;
    src[1].RR = as.rows_per_group;
    src[1].n = 0;
    src[1].slot0 = 0;
    if (nb > 0) {
      const int Wt = min(as.waves, T);
      const int first = flat_wave_of(s, T, Wt), last = flat_wave_of(s + nb - 1, T, Wt);
      src[1].slot0 = ((int64_t)hk * as.row_groups + rg) * (as.waves + as.B) + first + b;
      src[1].n = last - first + 1;
    }
  }
  merge_two<D>(src, as.out, out_row_base(as, b, hk, h, D), as.out_dtype);
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
#define KRILL_DISPATCH_D(D_, ...)                 \
  switch (D_) {                                   \
    case 64: {                                    \
      constexpr int D = 64;                       \
      __VA_ARGS__;                                \
    } break;                                      \
    case 128: {                                   \
      constexpr int D = 128;                      \
      __VA_ARGS__;                                \
    } break;                                      \
    case 256: {                                   \
      constexpr int D = 256;                      \
      __VA_ARGS__;                                \
    } break;                                      \
    case 512: {                                   \
      constexpr int D = 512;                      \
      __VA_ARGS__;                                \
    } break;                                      \
    default:                                      \
      return hipErrorInvalidValue;                \
  }

static inline unsigned wave_blocks(int64_t waves) { return (unsigned)((waves + 3) / 4); }

template <bool ROPE>
static hipError_t launch_append_rope(const PoolGeometry &g, int32_t layer, const void *k, const void *v, int64_t sb,
                                     int64_t sh, int64_t sl, const int32_t *slots, int32_t B, int32_t L,
                                     const RopeArgs &rope, hipStream_t st) {
  const int64_t waves = 2 * (int64_t)B * g.Hkv * L;
  if (waves == 0) return hipSuccess;
  const LayerView lv = layer_view(g, layer);
  const uint16_t *kk = static_cast<const uint16_t *>(k), *vv = static_cast<const uint16_t *>(v);
  if (L >= 32 && B <= 65535 && g.Hkv <= 65535 && !(g.mode == MODE_REF && g.D > 128) && g.D <= 256) {
    // chunks of 64 rows staged per block in LDS (the row mode at D = 256 --
    // a 256-element group per thread -- stays on the per-row kernel, and so
    // does D = 512, whose two V block images alone would take 64 KB of LDS)
    const dim3 grid((unsigned)((L + 63) / 64), (unsigned)g.Hkv, (unsigned)B), block(256);
    KRILL_DISPATCH_D(g.D, {
      if constexpr (D > 256) {
        return hipErrorInvalidValue;
      } else if (g.mode == MODE_REF) {
        if (g.in_dtype == DT_BF16)
          k_quantize_append_blocks<D, MODE_REF, DT_BF16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, L, rope);
        else
          k_quantize_append_blocks<D, MODE_REF, DT_F16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, L, rope);
      } else {
        if (g.in_dtype == DT_BF16)
          k_quantize_append_blocks<D, MODE_AFFINE, DT_BF16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, L, rope);
        else
          k_quantize_append_blocks<D, MODE_AFFINE, DT_F16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, L, rope);
      }
    });
    return hipGetLastError();
  }
  const dim3 grid(wave_blocks(waves)), block(256);
  KRILL_DISPATCH_D(g.D, {
    if (g.mode == MODE_REF) {
      if (g.in_dtype == DT_BF16)
        k_quantize_append<D, MODE_REF, DT_BF16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, B, L, g.Hkv, rope);
      else
        k_quantize_append<D, MODE_REF, DT_F16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, B, L, g.Hkv, rope);
    } else {
      if (g.in_dtype == DT_BF16)
        k_quantize_append<D, MODE_AFFINE, DT_BF16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, B, L, g.Hkv, rope);
      else
        k_quantize_append<D, MODE_AFFINE, DT_F16, ROPE><<<grid, block, 0, st>>>(lv, kk, vv, sb, sh, sl, slots, B, L, g.Hkv, rope);
    }
  });
  return hipGetLastError();
}

hipError_t launch_quantize_append(const PoolGeometry &g, int32_t layer, const void *k, const void *v,
                                  int64_t sb, int64_t sh, int64_t sl, const int32_t *slots, int32_t B,
                                  int32_t L, hipStream_t st, const int32_t *rope_pos, const float *rope_cs,
                                  int32_t rope_max_pos) {
  const RopeArgs rope{rope_pos, rope_cs, rope_max_pos};
  return rope_pos ? launch_append_rope<true>(g, layer, k, v, sb, sh, sl, slots, B, L, rope, st)
                  : launch_append_rope<false>(g, layer, k, v, sb, sh, sl, slots, B, L, rope, st);
}

hipError_t launch_gather(const PoolGeometry &g, int32_t layer, const int32_t *tables, const int32_t *lens,
                         int32_t B, int32_t max_blocks, int32_t S_out, int32_t left_pad, void *keys,
                         void *values, void *ks, void *kz, void *vs, void *vz, hipStream_t st) {
  if ((int64_t)B * g.Hkv * S_out == 0) return hipSuccess;
  if (B > 65535 || g.Hkv > 65535) return hipErrorInvalidValue;
  const LayerView lv = layer_view(g, layer);
  // data workgroups: the <= S_out tokens that land in the output span at most
  // ceil(S_out / 64) + 1 blocks; then one zero workgroup per 64 output rows
  const int32_t tiles = (S_out + 63) / 64, nbx = tiles + 1;
  const dim3 grid((unsigned)(nbx + tiles), (unsigned)g.Hkv, (unsigned)B), block(256);
  auto *k8 = static_cast<uint8_t *>(keys), *v8 = static_cast<uint8_t *>(values);
  auto *a = static_cast<uint16_t *>(ks), *bz = static_cast<uint16_t *>(kz), *c = static_cast<uint16_t *>(vs),
       *d = static_cast<uint16_t *>(vz);
  KRILL_DISPATCH_D(g.D, {
    if (g.G == 1)
      k_gather<D, 1><<<grid, block, 0, st>>>(lv, tables, lens, g.Hkv, max_blocks, S_out, left_pad, nbx, k8, v8, a,
                                             bz, c, d);
    else
      k_gather<D, D / 64><<<grid, block, 0, st>>>(lv, tables, lens, g.Hkv, max_blocks, S_out, left_pad, nbx, k8, v8,
                                                  a, bz, c, d);
  });
  return hipGetLastError();
}

hipError_t launch_gather_dequant(const PoolGeometry &g, int32_t layer, const int32_t *tables,
                                 const int32_t *lens, int32_t B, int32_t max_blocks, int32_t S_out,
                                 int32_t left_pad, void *k_out, void *v_out, hipStream_t st) {
  if ((int64_t)B * g.Hkv * S_out == 0) return hipSuccess;
  if (B > 65535 || g.Hkv > 65535) return hipErrorInvalidValue;
  const LayerView lv = layer_view(g, layer);
  const int32_t tiles = (S_out + 63) / 64, nbx = tiles + 1;
  const dim3 grid((unsigned)(nbx + tiles), (unsigned)g.Hkv, (unsigned)B), block(256);
  auto *ko = static_cast<uint16_t *>(k_out), *vo = static_cast<uint16_t *>(v_out);
  KRILL_DISPATCH_D(g.D, {
    if (g.mode == MODE_REF)
      k_gather_dequant<D, 1, MODE_REF><<<grid, block, 0, st>>>(lv, tables, lens, g.Hkv, max_blocks, S_out, left_pad,
                                                              nbx, ko, vo);
    else
      k_gather_dequant<D, D / 64, MODE_AFFINE><<<grid, block, 0, st>>>(lv, tables, lens, g.Hkv, max_blocks, S_out,
                                                                       left_pad, nbx, ko, vo);
  });
  return hipGetLastError();
}

hipError_t launch_scatter(const PoolGeometry &g, int32_t layer, const void *keys, const void *values,
                          const void *ks, const void *kz, const void *vs, const void *vz, int32_t B,
                          int32_t S_in, const int32_t *src_start, const int32_t *slots, int32_t L,
                          hipStream_t st) {
  if ((int64_t)B * L * g.Hkv == 0) return hipSuccess;
  if (B > 65535 || g.Hkv > 65535) return hipErrorInvalidValue;
  const LayerView lv = layer_view(g, layer);
  const dim3 grid((unsigned)((L + 63) / 64), (unsigned)g.Hkv, (unsigned)B), block(256);
  auto *k8 = static_cast<const uint8_t *>(keys), *v8 = static_cast<const uint8_t *>(values);
  auto *a = static_cast<const uint16_t *>(ks), *bz = static_cast<const uint16_t *>(kz),
       *c = static_cast<const uint16_t *>(vs), *d = static_cast<const uint16_t *>(vz);
  KRILL_DISPATCH_D(g.D, {
    if (g.G == 1)
      k_scatter<D, 1><<<grid, block, 0, st>>>(lv, k8, v8, a, bz, c, d, g.Hkv, S_in, src_start, slots, L);
    else
      k_scatter<D, D / 64><<<grid, block, 0, st>>>(lv, k8, v8, a, bz, c, d, g.Hkv, S_in, src_start, slots, L);
  });
  return hipGetLastError();
}

hipError_t launch_copy_blocks(const PoolGeometry &g, const int32_t *src_dst, int32_t n, hipStream_t st) {
  if (n <= 0) return hipSuccess;
  k_copy_blocks<<<dim3((unsigned)(n * g.num_layers)), dim3(256), 0, st>>>(
      g.base, g.layer_stride, g.block_stride, g.num_blocks, g.num_layers, src_dst, n);
  return hipGetLastError();
}

hipError_t launch_copy_pairs(const PoolGeometry &g, const CopyPair *pairs, int32_t n, hipStream_t st) {
  for (int32_t off = 0; off < n; off += 64) {
    CopyPairsArg pa;
    pa.n = std::min<int32_t>(64, n - off);
    for (int32_t i = 0; i < pa.n; ++i) {
      pa.sd[2 * i] = pairs[off + i].src;
      pa.sd[2 * i + 1] = pairs[off + i].dst;
    }
    k_copy_pairs<<<dim3((unsigned)(pa.n * g.num_layers)), dim3(256), 0, st>>>(g.base, g.layer_stride, g.block_stride,
                                                                            g.num_blocks, g.num_layers, pa);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

int32_t plan_attention(const PoolGeometry &g, int32_t B, int32_t Hq, int32_t Lq, int32_t max_seq_len,
                       int32_t split_blocks, int32_t path, AttnPlan *plan) {
  if (g.Hkv <= 0 || Hq <= 0 || Hq % g.Hkv != 0 || Lq <= 0 || B < 0 || max_seq_len < 0) return -1;
  const int32_t R = Hq / g.Hkv;
  AttnPlan p{};
  p.NR = R * Lq;
  // head_dim 512: the VALU kernel with each block split over four waves of
  // 128 dims (the MFMA kernel's LDS ring would hold 70 KB per stage), the
  // query rows in groups of at most 8 (the largest divisor of NR up to 8),
  // one grid row group each
  const bool dsplit = g.D > 256;
  if (dsplit && path == 2) return -2;
  p.use_mfma = !dsplit && (path == 2 || (path == 0 && p.NR > 8));
  if (!p.use_mfma && !dsplit && p.NR > 8) return -2;
  const int32_t nb_max = std::max(1, (max_seq_len + 63) / 64);
  const int64_t tmax = (int64_t)B * nb_max;
  const int64_t cus = g.num_cus > 0 ? g.num_cus : 256;
  if (p.use_mfma) {
    // MFMA: 16 query rows per wave (a row group); the row groups of a KV head
    // go to workgroups of up to 4 waves that share one LDS ring, so a block
    // is fetched once per 4 row groups and the smaller register file of a
    // 16-row wave leaves room for two waves per SIMD.
    // 17-32 rows (speculative verify) at D <= 128: one 32-row group per
    // workgroup whose two waves split each block's tokens instead, so no
    // byte is converted twice.  More than 64 rows at D <= 128 (chunked
    // prefill): 32-row waves in groups of four, each converted byte feeding
    // two row tiles, when a batch of max_seq_len sequences gives every
    // workgroup of that grid at least 16 blocks to stream (the cascade's
    // shared prefix of 65 blocks does not: its 16-row grid keeps more
    // workgroups busy).
    p.token_split = 1;
    const int64_t grp32 = ((p.NR + 31) / 32 + 3) / 4;
    const bool rows32 = p.NR > 64 && g.D <= 128 &&
                        tmax >= 16 * (cus * mfma_groups_per_cu(g, 2, 4, 1) / ((int64_t)g.Hkv * grp32));
    if (p.NR > 16 && p.NR <= 32 && g.D <= 128) {
      p.nrt = 2;
      p.rows_per_group = 32;
      p.row_groups = 1;
      p.group_waves = 1;
      p.token_split = 2;
    } else if (rows32) {
      p.nrt = 2;
      p.rows_per_group = 32;
      p.row_groups = (p.NR + 31) / 32;
      p.group_waves = 4;
    } else {
      p.nrt = 1;
      p.rows_per_group = 16;
      p.row_groups = (p.NR + 15) / 16;
      p.group_waves = p.row_groups >= 3 ? 4 : p.row_groups;
    }
  } else if (dsplit) {
    int32_t rpg = std::min<int32_t>(8, p.NR);
    while (p.NR % rpg != 0) --rpg;
    p.nrt = 0;
    p.rows_per_group = rpg;
    p.row_groups = p.NR / rpg;
    p.group_waves = 1;
    p.token_split = 1;
  } else {
    p.nrt = 0;
    p.rows_per_group = p.NR;
    p.row_groups = 1;
    p.group_waves = 1;
    p.token_split = 1;
  }
  // Both kernels: per (KV head, row group) the blocks of all sequences in
  // flat order, split evenly over a grid of workgroups (one wave each on the
  // VALU path).  Automatic: the GPU's resident capacity for the kernel
  // instantiation (every SIMD gets the same load, one round); with
  // split_blocks set: enough workgroups for that many blocks each when every
  // sequence is max_seq_len long.  Never more than 64 blocks per workgroup
  // (one VGPR of block-table entries).
  int64_t waves;
  if (split_blocks > 0) {
    const int64_t pw = std::min(split_blocks, 64);
    waves = (tmax + pw - 1) / pw;
  } else if (p.use_mfma) {
    const int64_t groups = (p.row_groups + p.group_waves - 1) / p.group_waves;
    waves = std::max<int64_t>(1, cus * mfma_groups_per_cu(g, p.nrt, p.group_waves, p.token_split) /
                                     ((int64_t)g.Hkv * groups));
  } else if (dsplit) {
    // workgroups of 4 waves (one per 128-dim slice)
    const int64_t wg_per_cu = std::max<int32_t>(1, valu_waves_per_cu(g, p.rows_per_group) / (g.D / 128));
    waves = std::max<int64_t>(1, cus * wg_per_cu / ((int64_t)g.Hkv * p.row_groups));
  } else {
    waves = std::max<int64_t>(1, cus * valu_waves_per_cu(g, p.NR) / g.Hkv);
  }
  waves = std::max<int64_t>(waves, (tmax + 63) / 64);
  p.split_blocks = split_blocks > 0 ? std::min(split_blocks, 64) : 0;
  p.nb_cap = nb_max;
  p.waves = (int32_t)waves;
  p.slots = (int64_t)g.Hkv * p.row_groups * (p.waves + B);
  p.ws_bytes = ws_layout(p.slots, p.rows_per_group, g.D).total;
  *plan = p;
  return 0;
}

hipError_t launch_attn_merge(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                             hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const dim3 grid((unsigned)p.NR, (unsigned)g.Hkv, (unsigned)a.B);
  KRILL_DISPATCH_D(g.D, { k_attn_merge_flat<D><<<grid, dim3(64), 0, st>>>(args); });
  return hipGetLastError();
}

// The newest-token append as its own launch (the MFMA path does not fuse it).
static hipError_t launch_append_newest(const PoolGeometry &g, int32_t layer, const AttnLaunch &a,
                                       const AttnPlan &p, hipStream_t st) {
  const int64_t waves = 2 * (int64_t)a.B * g.Hkv;
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const dim3 grid(wave_blocks(waves)), block(256);
  KRILL_DISPATCH_D(g.D, {
    if (g.mode == MODE_REF) {
      if (g.in_dtype == DT_BF16)
        k_append_newest<D, MODE_REF, DT_BF16><<<grid, block, 0, st>>>(args);
      else
        k_append_newest<D, MODE_REF, DT_F16><<<grid, block, 0, st>>>(args);
    } else {
      if (g.in_dtype == DT_BF16)
        k_append_newest<D, MODE_AFFINE, DT_BF16><<<grid, block, 0, st>>>(args);
      else
        k_append_newest<D, MODE_AFFINE, DT_F16><<<grid, block, 0, st>>>(args);
    }
  });
  return hipGetLastError();
}

hipError_t launch_attention_shared_prefix(const PoolGeometry &g, int32_t layer, const AttnLaunch &pa,
                                         const AttnPlan &pp, const AttnLaunch &sa, const AttnPlan &sp,
                                         hipStream_t st) {
  if (sa.B == 0) return hipSuccess;
  if (pa.B != 1 || pa.len_const < 0 || pa.causal || !pa.partial_only || !sa.partial_only || sa.Lq != 1 ||
      pa.Lq != sa.B)
    return hipErrorInvalidValue;
  hipError_t e = pp.use_mfma ? launch_attn_mfma(g, layer, pa, pp, st) : launch_attn_valu(g, layer, pa, pp, st);
  if (e != hipSuccess) return e;
  if (sa.k_new && sp.use_mfma) {  // the newest tokens (in the suffix blocks) before the MFMA suffix pass
    e = launch_append_newest(g, layer, sa, sp, st);
    if (e != hipSuccess) return e;
  }
  e = sp.use_mfma ? launch_attn_mfma(g, layer, sa, sp, st) : launch_attn_valu(g, layer, sa, sp, st);
  if (e != hipSuccess) return e;
  const AttnArgs ap = make_attn_args(g, layer, pa, pp), as = make_attn_args(g, layer, sa, sp);
  const dim3 grid((unsigned)ap.R, (unsigned)g.Hkv, (unsigned)sa.B);
  KRILL_DISPATCH_D(g.D, { k_attn_merge_cascade<D><<<grid, dim3(64), 0, st>>>(ap, as); });
  return hipGetLastError();
}

hipError_t launch_attention_windowed(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                                     const int32_t *starts, int32_t window, hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  if (window < 2 || a.len_const >= 0) return hipErrorInvalidValue;
  // the decode step with the append (and RoPE) fused runs on the VALU
  // kernel's window variants (the MFMA path has no RoPE of the queries, and
  // its separate append launch reads absolute table columns the windowed
  // plan does not cover)
  if (a.rope_cs && (!a.k_new || g.D > 256)) return hipErrorInvalidValue;
  if (a.k_new && (p.use_mfma || a.Lq != 1)) return hipErrorInvalidValue;
  AttnLaunch w = a;
  w.win_start = starts;
  w.window = window;
  return launch_attention(g, layer, w, p, st);
}

hipError_t launch_attention(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  if (a.B == 0) return hipSuccess;
  if (a.k_new && p.use_mfma) {
    hipError_t e = launch_append_newest(g, layer, a, p, st);
    if (e != hipSuccess) return e;
  }
  hipError_t e = p.use_mfma ? launch_attn_mfma(g, layer, a, p, st) : launch_attn_valu(g, layer, a, p, st);
  if (e != hipSuccess) return e;
  // windowed decode kernel at head_dim <= 256: merged inside its workgroups
  if (!p.use_mfma && a.window > 0 && g.D <= 256) return hipSuccess;
  return launch_attn_merge(g, layer, a, p, st);
}

}  // namespace krill
