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
// One wave64 per (split of 64-token blocks, kv head, sequence).  Per block:
//  * scores: NC = D/32 lanes share a token, each lane owns 32 d of K
//    (two 16-byte loads, contiguous across lanes), bytes become fp16
//    (1024 + q) with one v_perm_b32 per pair, v_dot2_f32_f16 against the
//    fp16 query held in registers, then a shuffle-sum across the NC lanes.
//    Affine mode uses linearity: q.k = s*(q.(1024+u) - 1024*sum q) + z*sum q
//    per 64-group, so no per-element dequantisation is needed.  Reference
//    row mode dequantises exactly (f16(f16(u*s)+z), two packed-fp16
//    roundings, QuantizedKVCache.swift:200-204) before the dot.
//  * online softmax in the log2 domain (wave shuffles), weights w = p*s_v
//    written to LDS in V storage order as fp16;
//  * P.V: each lane owns D/32 columns x 16 token positions per 32-token
//    group; V bytes (stored token-contiguous per d) are read with 16-byte
//    loads and reduced with v_dot2_f32_f16 over token pairs; the V zero
//    points and the 1024 offset collapse into one per-(row, group) term.
// Partial (m, l, o) go to the workspace for the split-K merge, or straight
// to the output when the sequence has a single split.
#include <hip/hip_runtime.h>

#include "attn_common.hpp"

namespace krill {

template <int D, int NR, int MODE>
__global__ __launch_bounds__(64) void k_attn_valu(AttnArgs a) {
  constexpr int NC = D / 32;   // lanes per token in the score loop
  constexpr int TPI = 64 / NC; // tokens per score iteration
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int ND = D / 32;   // d columns per lane in the P.V loop
  constexpr int KPG = ND / G;  // of which per scale group
  constexpr int LPG = NC / G;  // score lanes per scale group

  __shared__ __attribute__((aligned(16))) uint16_t w_lds[NR * G * 64];
  __shared__ __attribute__((aligned(16))) uint16_t s_lds[64];
  __shared__ __attribute__((aligned(16))) uint16_t z_lds[64];

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

  const int dq = lane % NC, tl = lane / NC;
  const int my_g = MODE == MODE_AFFINE ? dq / LPG : 0;
  const bool writer = (dq % LPG) == 0;

  // Query slice of this lane: d in [32*dq, 32*dq + 32) as 16 fp16 pairs.
  half2_t qh[NR][16];
  float qc[NR];
  int lim[NR];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    const int hq = hk * a.R + r % a.R, j = r / a.R;
    lim[r] = len - a.Lq + j + 1;
    const uint16_t *qp = a.q + (((int64_t)b * a.Hq + hq) * a.Lq + j) * D + 32 * dq;
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const _Float16 h0 = (_Float16)load_q(qp + 2 * i, a.q_dtype);
      const _Float16 h1 = (_Float16)load_q(qp + 2 * i + 1, a.q_dtype);
      qh[r][i] = half2_t{h0, h1};
      s += (float)h0 + (float)h1;
    }
    qc[r] = s;
  }

  float m_run[NR], l_part[NR], c_part[NR], acc[NR][ND];
#pragma unroll
  for (int r = 0; r < NR; ++r) {
    m_run[r] = -INFINITY;
    l_part[r] = 0.0f;
    c_part[r] = 0.0f;
#pragma unroll
    for (int k = 0; k < ND; ++k) acc[r][k] = 0.0f;
  }
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};

  for (int blk = blk0; blk < blk1; ++blk) {
    int phys = a.tables[(int64_t)b * a.max_blocks + blk];
    phys = (unsigned)phys < (unsigned)a.lv.num_blocks ? phys : 0;
    const uint8_t *reg = head_region(a.lv, phys, hk);
    const int tbase = blk << 6;

    // ---- scores (log2 domain)
    float sc[NC][NR];
#pragma unroll
    for (int it = 0; it < NC; ++it) {
      const int tok = it * TPI + tl;
      const uint4 *kp = reinterpret_cast<const uint4 *>(reg + ((dq * 64 + tok) << 5));
      const uint4 k0 = kp[0], k1 = kp[1];
      const uint32_t km = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + ((tok * G + my_g) << 2));
      const uint32_t kw[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      half2_t kv[16];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        kv[2 * i] = bytes01_plus1024(kw[i]);
        kv[2 * i + 1] = bytes23_plus1024(kw[i]);
      }
      const _Float16 ksh = __builtin_bit_cast(_Float16, (uint16_t)(km & 0xffffu));
      const _Float16 kzh = __builtin_bit_cast(_Float16, (uint16_t)(km >> 16));
      if constexpr (MODE == MODE_REF) {
        const half2_t s2 = half2_t{ksh, ksh}, z2 = half2_t{kzh, kzh};
#pragma unroll
        for (int i = 0; i < 16; ++i) kv[i] = (kv[i] + m1024) * s2 + z2;
      }
      const float ksf = (float)ksh, zz = (float)kzh - 1024.0f * (float)ksh;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float d = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d = dot2(qh[r][i], kv[i], d);
        float part = MODE == MODE_AFFINE ? fmaf(ksf, d, zz * qc[r]) : d;
#pragma unroll
        for (int m = 1; m < NC; m <<= 1) part += shfl_xor(part, m);
        sc[it][r] = (tbase + tok < lim[r]) ? part * a.scale_log2 : -INFINITY;
      }
    }

    // ---- online softmax
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float mb = sc[0][r];
#pragma unroll
      for (int it = 1; it < NC; ++it) mb = fmaxf(mb, sc[it][r]);
#pragma unroll
      for (int m = NC; m < 64; m <<= 1) mb = fmaxf(mb, shfl_xor(mb, m));
      const float mn = fmaxf(m_run[r], mb);
      const float mu = mn == -INFINITY ? 0.0f : mn;
      const float al = fast_exp2(m_run[r] - mu);
      m_run[r] = mn;
      float ps = 0.0f;
#pragma unroll
      for (int it = 0; it < NC; ++it) {
        sc[it][r] = fast_exp2(sc[it][r] - mu);
        ps += sc[it][r];
      }
      l_part[r] = l_part[r] * al + (dq == 0 ? ps : 0.0f);
      c_part[r] *= al;
#pragma unroll
      for (int k = 0; k < ND; ++k) acc[r][k] *= al;
    }

    // ---- weights to LDS, in V storage order
    if (writer) {
#pragma unroll
      for (int it = 0; it < NC; ++it) {
        const int tok = it * TPI + tl;
        const int pos = ((tok >> 5) << 5) + vpos(tok & 31);
        const bool valid = tbase + tok < len;
        const uint32_t vm =
            valid ? *reinterpret_cast<const uint32_t *>(reg + vm_offset(D, G) + ((tok * G + my_g) << 2)) : 0u;
        if constexpr (MODE == MODE_AFFINE) {
          const float vsf = f16_bits_to_f32((uint16_t)(vm & 0xffffu));
          const float vzf = f16_bits_to_f32((uint16_t)(vm >> 16));
#pragma unroll
          for (int r = 0; r < NR; ++r) {
            const float p = sc[it][r];
            const _Float16 wv = (_Float16)(p * vsf);
            w_lds[(r * G + my_g) * 64 + pos] = __builtin_bit_cast(uint16_t, wv);
            c_part[r] += p * vzf - 1024.0f * (float)wv;
          }
        } else {
#pragma unroll
          for (int r = 0; r < NR; ++r) w_lds[r * 64 + pos] = __builtin_bit_cast(uint16_t, (_Float16)sc[it][r]);
          s_lds[pos] = (uint16_t)(vm & 0xffffu);
          z_lds[pos] = (uint16_t)(vm >> 16);
        }
      }
    }
    __syncthreads();

    // ---- P.V
    const int hh = lane & 1, dl = lane >> 1;
    const uint32_t *w32 = reinterpret_cast<const uint32_t *>(w_lds);
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      const int p0 = tg * 32 + hh * 16;
#pragma unroll
      for (int g = 0; g < G; ++g) {
        half2_t wv[NR][8];
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          const uint4 *wp = reinterpret_cast<const uint4 *>(w32 + (r * G + g) * 32 + (p0 >> 1));
          const uint4 a0 = wp[0], a1 = wp[1];
          const uint32_t ww[8] = {a0.x, a0.y, a0.z, a0.w, a1.x, a1.y, a1.z, a1.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) wv[r][i] = u32_as_h2(ww[i]);
        }
        half2_t sp[8], zp[8];
        if constexpr (MODE == MODE_REF) {
          const uint4 *spp = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint32_t *>(s_lds) + (p0 >> 1));
          const uint4 *zpp = reinterpret_cast<const uint4 *>(reinterpret_cast<const uint32_t *>(z_lds) + (p0 >> 1));
          const uint4 s0 = spp[0], s1 = spp[1], z0 = zpp[0], z1 = zpp[1];
          const uint32_t ss[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
          const uint32_t zzz[8] = {z0.x, z0.y, z0.z, z0.w, z1.x, z1.y, z1.z, z1.w};
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            sp[i] = u32_as_h2(ss[i]);
            zp[i] = u32_as_h2(zzz[i]);
          }
        }
#pragma unroll
        for (int kk = 0; kk < KPG; ++kk) {
          const int k = g * KPG + kk;
          const int d = 32 * k + dl;
          const uint4 vw = *reinterpret_cast<const uint4 *>(reg + v_offset(D) + ((tg * D + d) << 5) + hh * 16);
          half2_t vp[8] = {bytes01_plus1024(vw.x), bytes23_plus1024(vw.x), bytes01_plus1024(vw.y),
                           bytes23_plus1024(vw.y), bytes01_plus1024(vw.z), bytes23_plus1024(vw.z),
                           bytes01_plus1024(vw.w), bytes23_plus1024(vw.w)};
          if constexpr (MODE == MODE_REF) {
#pragma unroll
            for (int i = 0; i < 8; ++i) vp[i] = (vp[i] + m1024) * sp[i] + zp[i];
          }
#pragma unroll
          for (int r = 0; r < NR; ++r) {
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[r][k] = dot2(wv[r][i], vp[i], acc[r][k]);
          }
        }
      }
    }
    __syncthreads();
  }

  // ---- epilogue
  const int hh = lane & 1, dl = lane >> 1;
#pragma unroll
  for (int r = 0; r < NR; ++r) {
#pragma unroll
    for (int k = 0; k < ND; ++k) acc[r][k] += shfl_xor(acc[r][k], 1);
    const float l = wave_sum_range<1, 32>(l_part[r]);
    float cg[G];
#pragma unroll
    for (int g = 0; g < G; ++g)
      cg[g] = MODE == MODE_AFFINE ? wave_sum_range<1, 32>(my_g == g ? c_part[r] : 0.0f) : 0.0f;
    if (n_splits == 1) {
      if (hh == 0) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
        for (int k = 0; k < ND; ++k) store_out(a.out, ob + 32 * k + dl, (acc[r][k] + cg[k / KPG]) * inv, a.out_dtype);
      }
    } else {
      const int64_t pi = part_index(a, b, hk, split, r);
      if (hh == 0) {
#pragma unroll
        for (int k = 0; k < ND; ++k) a.ws_o[pi * D + 32 * k + dl] = acc[r][k] + cg[k / KPG];
      }
      if (lane == 0) {
        a.ws_ml[pi * 2] = m_run[r];
        a.ws_ml[pi * 2 + 1] = l;
      }
    }
  }
}

template <int D, int MODE>
static hipError_t launch_valu_nr(const AttnArgs &args, int NR, dim3 grid, hipStream_t st) {
  switch (NR) {
    case 1: k_attn_valu<D, 1, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 2: k_attn_valu<D, 2, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 3: k_attn_valu<D, 3, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 4: k_attn_valu<D, 4, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 5: k_attn_valu<D, 5, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 6: k_attn_valu<D, 6, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 7: k_attn_valu<D, 7, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    case 8: k_attn_valu<D, 8, MODE><<<grid, dim3(64), 0, st>>>(args); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attn_valu(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const dim3 grid((unsigned)p.max_splits, (unsigned)g.Hkv, (unsigned)a.B);
  switch (g.D) {
    case 64:
      return g.mode == MODE_REF ? launch_valu_nr<64, MODE_REF>(args, p.NR, grid, st)
                                : launch_valu_nr<64, MODE_AFFINE>(args, p.NR, grid, st);
    case 128:
      return g.mode == MODE_REF ? launch_valu_nr<128, MODE_REF>(args, p.NR, grid, st)
                                : launch_valu_nr<128, MODE_AFFINE>(args, p.NR, grid, st);
    case 256:
      return g.mode == MODE_REF ? launch_valu_nr<256, MODE_REF>(args, p.NR, grid, st)
                                : launch_valu_nr<256, MODE_AFFINE>(args, p.NR, grid, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace krill
