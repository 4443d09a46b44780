// Paged int8 decode attention on the VALU (no MFMA): the path for up to 8
// query rows per KV head (GQA group x query length).
//
// Computes o = softmax(scale * q K^T) V over each sequence's paged int8
// cache -- what MLXFast.scaledDotProductAttention computes on the
// dequantized cache at Sources/KrillCore/Gemma4Model.swift:516-517 and
// Sources/KrillCore/Attention.swift:95-98, with the left-pad mask of
// Sources/KrillEngine/BatchedDecode.swift:277-287 replaced by per-row lengths
// (the -10000 mask underflows those weights to exactly zero, :22-28).
//
// Two launches: a prep kernel rounds the queries to fp16 once per
// (sequence, KV head) and sums them per scale group; the main kernel runs one
// wave64 per (split of 64-token blocks, KV head, sequence).  Per block:
//  * scores, one token per lane: the lane reads its token's K row (D bytes,
//    16-byte loads that are contiguous across lanes in the d-chunk-major
//    layout), turns byte pairs into fp16 (1024 + u) with one v_perm_b32, and
//    accumulates v_dot2c_f32_f16 against fp16 query pairs that are
//    wave-uniform and therefore come from scalar registers (scalar loads of
//    the prep output).  Affine mode uses linearity per 64-group:
//      q.k = s * (q.(1024 + u) - 1024 * sum q) + z * sum q,
//    so no element is dequantised.  Reference row mode dequantises exactly
//    (f16(f16(u*s) + z), QuantizedKVCache.swift:200-204) before the dot.
//  * online softmax in the log2 domain with a lazily raised running max: a
//    block only pays for a wave reduction when some score exceeds the
//    running max by more than 8 (a wave vote), so weights stay below 2^8;
//  * weights w = p * s_v (fp16) go to LDS in V storage order; each lane
//    then owns D/64 V^T rows (d values), loaded as contiguous 16-byte pieces,
//    and reduces token pairs with v_dot2c_f32_f16.  The V zero points and the
//    1024 offset collapse into one per-(row, group) term.
//  * the next block's K and V are loaded as soon as the current block's
//    registers are consumed, so loads overlap the other phase's math.
// A sequence with one split writes the output directly; otherwise every
// split writes (m, l, o) to the workspace and k_attn_merge combines them in a
// second launch.  (Merging inside the last split to finish would need an
// agent-scope release/acquire per split, which on this multi-XCD part is a
// whole-L2 writeback and invalidate per wave.)
#include <hip/hip_runtime.h>

#include "attn_common.hpp"

namespace krill {

typedef __attribute__((address_space(4))) const float scalar_f32;

// acc += sum_i k[i] . q_(OFF + i), i < 8, where q_n is lane n of this lane's
// 16-lane row of `q` (v_dot2c_f32_f16 with a DPP row_newbcast source).  The
// leading s_nop covers the VALU-write -> DPP-read hazard of the operands.
// The compiler cannot see the DOT instructions inside the asm, so it does not
// guard their result: a VALU instruction other than another v_dot2c reading
// `acc` as its accumulator needs 3 wait states after the last one (without
// them it reads a value missing the last dots).  TAIL marks the block that
// finishes `acc`; it ends with the wait.
#define KRILL_DOT8_BODY                                                                    \
  "s_nop 1\n\t"                                                                            \
  "v_dot2c_f32_f16_dpp %0, %1, %2 row_newbcast:%10 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %3 row_newbcast:%11 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %4 row_newbcast:%12 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %5 row_newbcast:%13 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %6 row_newbcast:%14 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %7 row_newbcast:%15 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %8 row_newbcast:%16 row_mask:0xf bank_mask:0xf\n\t"         \
  "v_dot2c_f32_f16_dpp %0, %1, %9 row_newbcast:%17 row_mask:0xf bank_mask:0xf"
#define KRILL_DOT8_OPERANDS                                                                           \
  : "+v"(acc)                                                                                         \
  : "v"(q), "v"(k[0]), "v"(k[1]), "v"(k[2]), "v"(k[3]), "v"(k[4]), "v"(k[5]), "v"(k[6]), "v"(k[7]), \
    "n"(OFF), "n"(OFF + 1), "n"(OFF + 2), "n"(OFF + 3), "n"(OFF + 4), "n"(OFF + 5), "n"(OFF + 6), "n"(OFF + 7)
template <int OFF, bool TAIL>
__device__ __forceinline__ void dot8_bcast(float &acc, uint32_t q, const half2_t (&k)[8]) {
  if constexpr (TAIL)
    asm(KRILL_DOT8_BODY "\n\ts_nop 3" KRILL_DOT8_OPERANDS);
  else
    asm(KRILL_DOT8_BODY KRILL_DOT8_OPERANDS);
}
#undef KRILL_DOT8_BODY
#undef KRILL_DOT8_OPERANDS

// fp16 queries and their per-group sums.
template <int D, int NR, int G>
__global__ __launch_bounds__(64) void k_attn_prep(AttnArgs a) {
  const int hk = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
  const int64_t row0 = ((int64_t)b * a.Hkv + hk) * NR;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int hq = hk * a.R + r % a.R, j = r / a.R;
    const uint16_t *qp = a.q + (((int64_t)b * a.Hq + hq) * a.Lq + j) * D;
    float gs[G];
#pragma unroll
    for (int g = 0; g < G; ++g) gs[g] = 0.0f;
#pragma unroll
    for (int k = 0; k < D / 64; ++k) {
      const int d = lane + 64 * k;
      const _Float16 h = (_Float16)load_q(qp + d, a.q_dtype);
      a.q16[(row0 + r) * D + d] = __builtin_bit_cast(uint16_t, h);
      gs[(64 * k) / (D / G)] += (float)h;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const float t = wave_allsum(gs[g]);
      if (lane == 0) a.qsum[(row0 + r) * G + g] = t;
    }
  }
}

template <int D, int NR, int MODE>
__global__ __launch_bounds__(64) void k_attn_valu(AttnArgs a) {
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int NP = D / 16;   // 16-byte K pieces per token row
  constexpr int PPG = NP / G;  // pieces per scale group
  constexpr int DPL = D / 64;  // V^T rows (d values) per lane

  __shared__ __attribute__((aligned(16))) uint16_t w_lds[NR * G * 64];
  __shared__ __attribute__((aligned(16))) uint16_t sz_lds[2 * 64];

  const int lane = threadIdx.x;
  const int split = blockIdx.x, hk = blockIdx.y, b = blockIdx.z;
  const int len = a.lens[b];
  const int nb = seq_blocks(a, len);
  if (nb == 0) {
    if (split == 0) {
#pragma unroll
      for (int r = 0; r < NR; ++r)
        for (int d = lane; d < D; d += 64) store_out(a.out, out_row_base(a, b, hk, r, D) + d, 0.0f, a.out_dtype);
    }
    return;
  }
  const int blk0 = split * a.split_blocks;
  if (blk0 >= nb) return;
  const int blk1 = min(nb, blk0 + a.split_blocks);
  const int n_splits = (nb + a.split_blocks - 1) / a.split_blocks;

  const int64_t qrow = ((int64_t)b * a.Hkv + hk) * NR;
  // fp16 query pairs: qv[r][c] holds pair 16*c + (lane & 15) of row r, so
  // every 16-lane row carries the whole query (one VGPR per 32 d)
  uint32_t qv[NR][D / 32];
  {
    const uint32_t *q16 = reinterpret_cast<const uint32_t *>(a.q16 + qrow * D);
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int c = 0; c < D / 32; ++c) qv[r][c] = q16[r * (D / 2) + 16 * c + (lane & 15)];
  }
  scalar_f32 *qs = (scalar_f32 *)(a.qsum + qrow * G);
  int lim[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) lim[r] = len - a.Lq + r / a.R + 1;
  const int gl = MODE == MODE_AFFINE ? (DPL * lane) / 64 : 0;  // scale group of this lane's V rows
  const int pos = ((lane >> 5) << 5) + vpos(lane & 31);        // this lane's token in V order

  float m_run[NR], l_part[NR], c_part[NR][G], acc[NR][DPL];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    m_run[r] = -INFINITY;
    l_part[r] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) c_part[r][g] = 0.0f;
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[r][e] = 0.0f;
  }
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};

  // Physical block ids of this split (at most 64 blocks): lane i holds the
  // entry of block blk0 + i, read back with v_readlane, so no table load sits
  // between a prefetch and its use (a load there would have to drain the
  // prefetch before its value could move to a scalar register).
  int tab;
  {
    const int i = blk0 + lane;
    const int phys = i < blk1 ? a.tables[(int64_t)b * a.max_blocks + i] : 0;
    tab = (unsigned)phys < (unsigned)a.lv.num_blocks ? phys : 0;
  }
  auto region_of = [&](int blk) -> const uint8_t * {
    return head_region(a.lv, __builtin_amdgcn_readlane(tab, blk - blk0), hk);
  };
  uint4 kr[NP];
  uint4 vr[2][2 * DPL];
  auto load_k = [&](const uint8_t *reg) {
#pragma unroll
    for (int p = 0; p < NP; ++p) kr[p] = *reinterpret_cast<const uint4 *>(reg + k_byte(lane, 16 * p));
  };
  auto load_v = [&](const uint8_t *reg) {
#pragma unroll
    for (int tg = 0; tg < 2; ++tg)
#pragma unroll
      for (int i = 0; i < 2 * DPL; ++i)
        vr[tg][i] = *reinterpret_cast<const uint4 *>(reg + v_offset(D) + ((tg * D + DPL * lane) << 5) + 16 * i);
  };

  // this lane's token's (scale, zero) pairs, K and V
  uint32_t km[G], vm[G];
  auto load_meta = [&](const uint8_t *reg, uint32_t (&kmo)[G], uint32_t (&vmo)[G]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
      kmo[g] = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + ((lane * G + g) << 2));
      vmo[g] = *reinterpret_cast<const uint32_t *>(reg + vm_offset(D, G) + ((lane * G + g) << 2));
    }
  };

  // Loads of block n+1 are issued in a fixed order inside the loop: K bytes
  // and metadata once block n's K registers are consumed, V bytes once its V
  // registers are; waits on a load never cover a younger prefetch.  The
  // first block's loads are settled before the loop so the loop-head waits
  // follow the steady-state order only.
  const uint8_t *reg = region_of(blk0);
  load_k(reg);
  load_meta(reg, km, vm);
  load_v(reg);
#pragma unroll
  for (int p = 0; p < NP; ++p) settle(kr[p]);
#pragma unroll
  for (int tg = 0; tg < 2; ++tg)
#pragma unroll
    for (int i = 0; i < 2 * DPL; ++i) settle(vr[tg][i]);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    settle(km[g]);
    settle(vm[g]);
  }

  for (int blk = blk0; blk < blk1; ++blk) {
    const int tbase = blk << 6;
    const bool has_next = blk + 1 < blk1;
    const uint8_t *nreg = has_next ? region_of(blk + 1) : reg;

    // ---- scores: this lane's token against every query row; the query
    // pair of each dot comes from lane (pair & 15) of the lane's 16-lane row
    // through the DPP broadcast of v_dot2c.
    float accg[NR][G];
#pragma unroll
    for (int r = 0; r < NR; ++r)
#pragma unroll
      for (int g = 0; g < G; ++g) accg[r][g] = 0.0f;
    half2_t ks2 = m1024, kz2 = m1024;
    if constexpr (MODE == MODE_REF) {
      const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(km[0] & 0xffffu));
      const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)(km[0] >> 16));
      ks2 = half2_t{s, s};
      kz2 = half2_t{z, z};
    }
#pragma unroll
    for (int p = 0; p < NP; ++p) {
      if (p > 0) order_after(kr[p], accg[NR - 1][MODE == MODE_AFFINE ? (p - 1) / PPG : 0]);
      const uint32_t w4[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
      half2_t kp[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        kp[2 * i] = bytes01_plus1024(w4[i]);
        kp[2 * i + 1] = bytes23_plus1024(w4[i]);
      }
      if constexpr (MODE == MODE_REF) {
#pragma unroll
        for (int i = 0; i < 8; ++i) kp[i] = (kp[i] + m1024) * ks2 + kz2;
      }
      const int g = MODE == MODE_AFFINE ? p / PPG : 0;
      // the last piece of a scale group finishes accg[.][g]
      const bool tail = MODE == MODE_AFFINE ? (p + 1) % PPG == 0 : p == NP - 1;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        if (p & 1) {
          if (tail)
            dot8_bcast<8, true>(accg[r][g], qv[r][p >> 1], kp);
          else
            dot8_bcast<8, false>(accg[r][g], qv[r][p >> 1], kp);
        } else {
          if (tail)
            dot8_bcast<0, true>(accg[r][g], qv[r][p >> 1], kp);
          else
            dot8_bcast<0, false>(accg[r][g], qv[r][p >> 1], kp);
        }
      }
    }
    // K registers are free: fetch the next block's K bytes and metadata.
    // Unconditional on purpose (the last block re-reads itself from L2): a
    // conditional load would keep the consumed registers alive through the
    // loop header.
    load_k(nreg);
    uint32_t km_next[G], vm_next[G];
    load_meta(nreg, km_next, vm_next);

    float s[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float v;
      if constexpr (MODE == MODE_AFFINE) {
        v = 0.0f;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const float kss = f16_bits_to_f32((uint16_t)(km[g] & 0xffffu));
          const float kzz = f16_bits_to_f32((uint16_t)(km[g] >> 16));
          v += kss * accg[r][g] + (kzz - 1024.0f * kss) * qs[r * G + g];
        }
      } else {
        v = accg[r][0];
      }
      s[r] = (tbase + lane < lim[r]) ? v * a.scale_log2 : -INFINITY;
    }

    // ---- online softmax with a lazily raised running max
    bool raise = blk == blk0;
    if (!raise) {
      bool over = false;
#pragma unroll
      for (int r = 0; r < NR; ++r) over |= s[r] > m_run[r] + 8.0f;
      raise = __any(over);
    }
    if (raise) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float mb = wave_allmax(s[r]);
        const float mn = fmaxf(m_run[r], mb);
        const float al = m_run[r] == -INFINITY ? 0.0f : fast_exp2(m_run[r] - mn);
        m_run[r] = mn;
        l_part[r] *= al;
#pragma unroll
        for (int g = 0; g < G; ++g) c_part[r][g] *= al;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[r][e] *= al;
      }
    }
    float pr[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      pr[r] = fast_exp2(s[r] - (m_run[r] == -INFINITY ? 0.0f : m_run[r]));
      l_part[r] += pr[r];
    }

    // ---- weights to LDS in V storage order
    const bool valid = tbase + lane < len;
    if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float vsf = valid ? f16_bits_to_f32((uint16_t)(vm[g] & 0xffffu)) : 0.0f;
        const float vzf = valid ? f16_bits_to_f32((uint16_t)(vm[g] >> 16)) : 0.0f;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const _Float16 wv = (_Float16)(pr[r] * vsf);
          w_lds[(r * G + g) * 64 + pos] = __builtin_bit_cast(uint16_t, wv);
          c_part[r][g] += pr[r] * vzf - 1024.0f * (float)wv;
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r) w_lds[r * 64 + pos] = __builtin_bit_cast(uint16_t, (_Float16)pr[r]);
      sz_lds[pos] = valid ? (uint16_t)(vm[0] & 0xffffu) : (uint16_t)0;
      sz_lds[64 + pos] = valid ? (uint16_t)(vm[0] >> 16) : (uint16_t)0;
    }
    __syncthreads();

    // ---- P.V: lane owns V^T rows d = DPL*lane .. +DPL, 32 tokens per group
    const uint32_t *w32 = reinterpret_cast<const uint32_t *>(w_lds);
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      if (tg > 0) {
#pragma unroll
        for (int i = 0; i < 2 * DPL; ++i) order_after(vr[1][i], acc[NR - 1][DPL - 1]);
      }
      half2_t vp[DPL][16];
#pragma unroll
      for (int e = 0; e < DPL; ++e)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const uint4 w = vr[tg][2 * e + h];
          vp[e][8 * h + 0] = bytes01_plus1024(w.x);
          vp[e][8 * h + 1] = bytes23_plus1024(w.x);
          vp[e][8 * h + 2] = bytes01_plus1024(w.y);
          vp[e][8 * h + 3] = bytes23_plus1024(w.y);
          vp[e][8 * h + 4] = bytes01_plus1024(w.z);
          vp[e][8 * h + 5] = bytes23_plus1024(w.z);
          vp[e][8 * h + 6] = bytes01_plus1024(w.w);
          vp[e][8 * h + 7] = bytes23_plus1024(w.w);
        }
      if constexpr (MODE == MODE_REF) {
        const uint32_t *s32 = reinterpret_cast<const uint32_t *>(sz_lds);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const half2_t sp = u32_as_h2(s32[tg * 16 + i]);
          const half2_t zp = u32_as_h2(s32[32 + tg * 16 + i]);
#pragma unroll
          for (int e = 0; e < DPL; ++e) vp[e][i] = (vp[e][i] + m1024) * sp + zp;
        }
      }
      // weights of row r + 1 are read while row r is reduced
      uint4 wn[4];
      {
        const uint4 *wp = reinterpret_cast<const uint4 *>(w32 + gl * 32 + tg * 16);
#pragma unroll
        for (int i = 0; i < 4; ++i) wn[i] = wp[i];
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const uint4 a0 = wn[0], a1 = wn[1], a2 = wn[2], a3 = wn[3];
        asm volatile("" ::: "memory");
        if (r + 1 < NR) {
          const uint4 *wp = reinterpret_cast<const uint4 *>(w32 + ((r + 1) * G + gl) * 32 + tg * 16);
#pragma unroll
          for (int i = 0; i < 4; ++i) wn[i] = wp[i];
        }
        const uint32_t ww[16] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w,
                                 a2.x, a2.y, a2.z, a2.w, a3.x, a3.y, a3.z, a3.w};
#pragma unroll
        for (int e = 0; e < DPL; ++e)
#pragma unroll
          for (int i = 0; i < 16; ++i) acc[r][e] = dot2(u32_as_h2(ww[i]), vp[e][i], acc[r][e]);
      }
    }
    load_v(nreg);  // V registers are free: fetch the next block
#pragma unroll
    for (int g = 0; g < G; ++g) {
      km[g] = km_next[g];
      vm[g] = vm_next[g];
    }
    reg = nreg;
    __syncthreads();
  }

  // ---- epilogue
  float o[NR][DPL], lsum[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    lsum[r] = wave_allsum(l_part[r]);
    float cg = 0.0f;
    if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const float c = wave_allsum(c_part[r][g]);
        cg = g == gl ? c : cg;
      }
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) o[r][e] = acc[r][e] + cg;
  }
  if (n_splits == 1) {
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float inv = lsum[r] > 0.0f ? 1.0f / lsum[r] : 0.0f;
      const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
      for (int e = 0; e < DPL; ++e) store_out(a.out, ob + DPL * lane + e, o[r][e] * inv, a.out_dtype);
    }
    return;
  }
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int64_t pi = part_index(a, b, hk, split, r);
#pragma unroll
    for (int e = 0; e < DPL; ++e) a.ws_o[pi * D + DPL * lane + e] = o[r][e];
    if (lane == 0) {
      a.ws_ml[pi * 2] = m_run[r];
      a.ws_ml[pi * 2 + 1] = lsum[r];
    }
  }
}

template <int D, int MODE, int NR>
static void launch_one(const AttnArgs &args, int B, dim3 grid, hipStream_t st) {
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  k_attn_prep<D, NR, G><<<dim3((unsigned)args.Hkv, (unsigned)B), dim3(64), 0, st>>>(args);
  k_attn_valu<D, NR, MODE><<<grid, dim3(64), 0, st>>>(args);
}

template <int D, int MODE>
static hipError_t launch_valu_nr(const AttnArgs &args, int NR, int B, dim3 grid, hipStream_t st) {
  switch (NR) {
    case 1: launch_one<D, MODE, 1>(args, B, grid, st); break;
    case 2: launch_one<D, MODE, 2>(args, B, grid, st); break;
    case 3: launch_one<D, MODE, 3>(args, B, grid, st); break;
    case 4: launch_one<D, MODE, 4>(args, B, grid, st); break;
    case 5: launch_one<D, MODE, 5>(args, B, grid, st); break;
    case 6: launch_one<D, MODE, 6>(args, B, grid, st); break;
    case 7: launch_one<D, MODE, 7>(args, B, grid, st); break;
    case 8: launch_one<D, MODE, 8>(args, B, grid, st); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attn_valu(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  // one VGPR of block-table entries per split
  if (p.split_blocks < 1 || p.split_blocks > 64) return hipErrorInvalidValue;
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const dim3 grid((unsigned)p.max_splits, (unsigned)g.Hkv, (unsigned)a.B);
  switch (g.D) {
    case 64:
      return g.mode == MODE_REF ? launch_valu_nr<64, MODE_REF>(args, p.NR, a.B, grid, st)
                                : launch_valu_nr<64, MODE_AFFINE>(args, p.NR, a.B, grid, st);
    case 128:
      return g.mode == MODE_REF ? launch_valu_nr<128, MODE_REF>(args, p.NR, a.B, grid, st)
                                : launch_valu_nr<128, MODE_AFFINE>(args, p.NR, a.B, grid, st);
    case 256:
      return g.mode == MODE_REF ? launch_valu_nr<256, MODE_REF>(args, p.NR, a.B, grid, st)
                                : launch_valu_nr<256, MODE_AFFINE>(args, p.NR, a.B, grid, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace krill
