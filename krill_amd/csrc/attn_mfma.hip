// Paged int8 attention with MFMA tiles: the speculative-verify / chunked-
// prefill path, used when a KV head serves more than 8 query rows
// (GQA group x new tokens).  Reference semantics: the same SDPA call with
// L > 1 new rows and the block-causal mask of
// Sources/KrillEngine/BatchedDecode.swift:299-312 (row j of the new window
// sees every cached key plus new keys 0..j), equivalently
// Sources/KrillCore/LlamaModel.swift:186-202.
//
// One wave64 per (split of 64-token blocks, kv head x row group, sequence);
// a row group holds NRT tiles of 16 query rows (NRT <= 2, register bound).  The kernel works
// on transposed scores so no operand is ever transposed in registers:
//   S^T[tok][row] = K[tok][d] . Q^T[d][row]      v_mfma_f32_16x16x32_f16
//   O^T[d][row]  += V^T[d][tok] . P^T[tok][row]  v_mfma_f32_16x16x32_f16
// K rows are stored 32-d-chunk major, so the A operand (8 d of one token per
// lane) is one 8-byte load; V is stored token-contiguous per d in exactly the
// token order in which the S^T accumulator hands P to the P.V B operand.
// Bytes become exact fp16 with v_perm_b32 + one packed subtract; affine
// scale/bias are applied to the fp32 scores (per group) and folded into the
// fp16 weights P*s_v, which are split hi + lo so the weight rounding stays
// below 2^-22 relative.  Rows beyond the causal limit of a whole row group
// skip their blocks (chunked prefill does half the work of a dense mask).
#include <hip/hip_runtime.h>

#include "attn_common.hpp"

namespace krill {

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ half8_t bytes8_exact(uint2 w) {
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};
  const half2_t a = bytes01_plus1024(w.x) + m1024, b = bytes23_plus1024(w.x) + m1024;
  const half2_t c = bytes01_plus1024(w.y) + m1024, d = bytes23_plus1024(w.y) + m1024;
  return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}

template <int D, int MODE, int NRT>
__global__ __launch_bounds__(64) void k_attn_mfma(AttnArgs a, int32_t row_groups) {
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int KS = D / 32;  // 32-d steps of Q.K^T
  constexpr int NDT = D / 16; // 16-d tiles of P.V
  const int lane = threadIdx.x;
  const int n = lane & 15, q4 = lane >> 4;
  const int split = blockIdx.x;
  const int hk = blockIdx.y / row_groups, rg = blockIdx.y % row_groups;
  const int b = blockIdx.z;
  const int len = a.lens[b];
  const int nb = seq_blocks(a, len);
  const int rbase = rg * 16 * NRT;

  int lim[NRT];
  bool rvalid[NRT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    const int r = rbase + 16 * rt + n;
    rvalid[rt] = r < a.NR;
    lim[rt] = rvalid[rt] ? len - a.Lq + r / a.R + 1 : 0;
  }
  if (nb == 0) {
    if (split == 0) {
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
        if (rvalid[rt] && q4 == 0)
          for (int d = 0; d < D; ++d)
            store_out(a.out, out_row_base(a, b, hk, rbase + 16 * rt + n, D) + d, 0.0f, a.out_dtype);
    }
    return;
  }
  const int blk0 = split * a.split_blocks;
  if (blk0 >= nb) return;
  const int n_splits = (nb + a.split_blocks - 1) / a.split_blocks;
  // causal extent of the whole row group
  const int rlast = min(a.NR, rbase + 16 * NRT) - 1;
  const int lim_max = len - a.Lq + rlast / a.R + 1;
  const int nb_vis = min(nb, (lim_max + 63) >> 6);
  const int blk1 = min(min(nb, blk0 + a.split_blocks), nb_vis);

  // Q^T operands: lane holds q[row n][32*ks + 8*q4 .. +8] per row tile.
  half8_t qB[NRT][KS];
  float qsum[NRT][G];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
    for (int g = 0; g < G; ++g) qsum[rt][g] = 0.0f;
    const int r = rbase + 16 * rt + n;
    const int hq = hk * a.R + r % a.R, j = r / a.R;
    const uint16_t *qp = a.q + (((int64_t)b * a.Hq + hq) * a.Lq + j) * D;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      half8_t v;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const _Float16 h = rvalid[rt] ? (_Float16)load_q(qp + 32 * ks + 8 * q4 + e, a.q_dtype) : (_Float16)0.0f;
        v[e] = h;
        qsum[rt][MODE == MODE_AFFINE ? ks / 2 : 0] += (float)h;
      }
      qB[rt][ks] = v;
    }
#pragma unroll
    for (int g = 0; g < G; ++g) {
      qsum[rt][g] += shfl_xor(qsum[rt][g], 16);
      qsum[rt][g] += shfl_xor(qsum[rt][g], 32);
    }
  }

  float m_run[NRT], l_part[NRT], c_part[NRT][G];
  float4_t oacc[NRT][NDT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    m_run[rt] = -INFINITY;
    l_part[rt] = 0.0f;
#pragma unroll
    for (int g = 0; g < G; ++g) c_part[rt][g] = 0.0f;
#pragma unroll
    for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};

  for (int blk = blk0; blk < blk1; ++blk) {
    int phys = a.tables[(int64_t)b * a.max_blocks + blk];
    phys = (unsigned)phys < (unsigned)a.lv.num_blocks ? phys : 0;
    const uint8_t *reg = head_region(a.lv, phys, hk);
    const int tbase = blk << 6;

    // ---- S^T = K . Q^T, four 16-token tiles
    float sc[4][NRT][4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      const int tokA = 16 * tt + n;  // A-operand row
      half2_t ks2 = half2_t{(_Float16)0.0f, (_Float16)0.0f}, kz2 = ks2;
      if constexpr (MODE == MODE_REF) {
        const uint32_t km = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + (tokA << 2));
        const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(km & 0xffffu));
        const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)(km >> 16));
        ks2 = half2_t{s, s};
        kz2 = half2_t{z, z};
      }
      float4_t sacc[NRT][G];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int g = 0; g < G; ++g) sacc[rt][g] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint2 kb = *reinterpret_cast<const uint2 *>(reg + k_byte(tokA, 32 * ks + 8 * q4));
        half8_t A;
        if constexpr (MODE == MODE_REF) {
          half2_t p0 = (bytes01_plus1024(kb.x) + m1024) * ks2 + kz2;
          half2_t p1 = (bytes23_plus1024(kb.x) + m1024) * ks2 + kz2;
          half2_t p2 = (bytes01_plus1024(kb.y) + m1024) * ks2 + kz2;
          half2_t p3 = (bytes23_plus1024(kb.y) + m1024) * ks2 + kz2;
          A = half8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        } else {
          A = bytes8_exact(kb);
        }
        const int g = MODE == MODE_AFFINE ? ks / 2 : 0;
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) sacc[rt][g] = mfma16x16x32(A, qB[rt][ks], sacc[rt][g]);
      }
      // lane holds tokens 16*tt + 4*q4 + e for row n
      const int tok0 = 16 * tt + 4 * q4;
      float kss[4][G], kzz[4][G];
      if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const uint32_t km = *reinterpret_cast<const uint32_t *>(reg + km_offset(D) + (((tok0 + e) * G + g) << 2));
            kss[e][g] = f16_bits_to_f32((uint16_t)(km & 0xffffu));
            kzz[e][g] = f16_bits_to_f32((uint16_t)(km >> 16));
          }
      }
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float s;
          if constexpr (MODE == MODE_AFFINE) {
            s = 0.0f;
#pragma unroll
            for (int g = 0; g < G; ++g) s += kss[e][g] * sacc[rt][g][e] + kzz[e][g] * qsum[rt][g];
          } else {
            s = sacc[rt][0][e];
          }
          sc[tt][rt][e] = (tbase + tok0 + e < lim[rt]) ? s * a.scale_log2 : -INFINITY;
        }
    }

    // ---- online softmax (row n of each tile; its 64 scores live in the
    // four lanes n, n+16, n+32, n+48)
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      float mb = -INFINITY;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) mb = fmaxf(mb, sc[tt][rt][e]);
      mb = fmaxf(mb, shfl_xor(mb, 16));
      mb = fmaxf(mb, shfl_xor(mb, 32));
      const float mn = fmaxf(m_run[rt], mb);
      const float mu = mn == -INFINITY ? 0.0f : mn;
      const float al = fast_exp2(m_run[rt] - mu);
      m_run[rt] = mn;
      float ps = 0.0f;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sc[tt][rt][e] = fast_exp2(sc[tt][rt][e] - mu);
          ps += sc[tt][rt][e];
        }
      l_part[rt] = l_part[rt] * al + ps;
#pragma unroll
      for (int g = 0; g < G; ++g) c_part[rt][g] *= al;
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] *= al;
    }

    // ---- O^T += V^T . P^T over two 32-token groups
#pragma unroll
    for (int tg = 0; tg < 2; ++tg) {
      // logical k = 8*q4 + i  <->  token 32*tg + (i < 4 ? 4*q4 + i : 16 + 4*q4 + i - 4)
      float vss[8][G], vzz[8][G];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int tok = 32 * tg + (i < 4 ? 4 * q4 + i : 16 + 4 * q4 + (i - 4));
        const bool valid = tbase + tok < len;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          const uint32_t vm =
              valid ? *reinterpret_cast<const uint32_t *>(reg + vm_offset(D, G) + ((tok * G + g) << 2)) : 0u;
          vss[i][g] = f16_bits_to_f32((uint16_t)(vm & 0xffffu));
          vzz[i][g] = f16_bits_to_f32((uint16_t)(vm >> 16));
        }
      }
      half8_t Bhi[NRT][G], Blo[NRT][G];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          const float p = sc[2 * tg + (i >> 2)][rt][i & 3];
#pragma unroll
          for (int g = 0; g < G; ++g) {
            const float w = MODE == MODE_AFFINE ? p * vss[i][g] : p;
            const _Float16 hi = (_Float16)w;
            const _Float16 lo = (_Float16)(w - (float)hi);
            Bhi[rt][g][i] = hi;
            Blo[rt][g][i] = lo;
            if constexpr (MODE == MODE_AFFINE) c_part[rt][g] += p * vzz[i][g];
          }
        }
      }
      half2_t sp[4], zp[4];
      if constexpr (MODE == MODE_REF) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          sp[i] = half2_t{(_Float16)vss[2 * i][0], (_Float16)vss[2 * i + 1][0]};
          zp[i] = half2_t{(_Float16)vzz[2 * i][0], (_Float16)vzz[2 * i + 1][0]};
        }
      }
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt) {
        const int d = 16 * dt + n;
        const uint2 vb = *reinterpret_cast<const uint2 *>(reg + v_pos_byte(D, tg, d, 8 * q4));
        half8_t A;
        if constexpr (MODE == MODE_REF) {
          half2_t p0 = (bytes01_plus1024(vb.x) + m1024) * sp[0] + zp[0];
          half2_t p1 = (bytes23_plus1024(vb.x) + m1024) * sp[1] + zp[1];
          half2_t p2 = (bytes01_plus1024(vb.y) + m1024) * sp[2] + zp[2];
          half2_t p3 = (bytes23_plus1024(vb.y) + m1024) * sp[3] + zp[3];
          A = half8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
        } else {
          A = bytes8_exact(vb);
        }
        const int g = MODE == MODE_AFFINE ? dt / 4 : 0;
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          oacc[rt][dt] = mfma16x16x32(A, Bhi[rt][g], oacc[rt][dt]);
          oacc[rt][dt] = mfma16x16x32(A, Blo[rt][g], oacc[rt][dt]);
        }
      }
    }
  }

  // ---- epilogue: lane holds O^T[d = 16*dt + 4*q4 + e][row n]
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) {
    float l = l_part[rt];
    l += shfl_xor(l, 16);
    l += shfl_xor(l, 32);
    float cg[G];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      float c = c_part[rt][g];
      c += shfl_xor(c, 16);
      c += shfl_xor(c, 32);
      cg[g] = c;
    }
    if (!rvalid[rt]) continue;
    const int r = rbase + 16 * rt + n;
    if (n_splits == 1) {
      const float inv = l > 0.0f ? 1.0f / l : 0.0f;
      const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = 16 * dt + 4 * q4 + e;
          store_out(a.out, ob + d, (oacc[rt][dt][e] + cg[MODE == MODE_AFFINE ? d / 64 : 0]) * inv, a.out_dtype);
        }
    } else {
      const int64_t pi = part_index(a, b, hk, split, r);
#pragma unroll
      for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int d = 16 * dt + 4 * q4 + e;
          a.ws_o[pi * D + d] = oacc[rt][dt][e] + cg[MODE == MODE_AFFINE ? d / 64 : 0];
        }
      if (q4 == 0) {
        a.ws_ml[pi * 2] = m_run[rt];
        a.ws_ml[pi * 2 + 1] = l;
      }
    }
  }
}

template <int D, int MODE>
static hipError_t launch_mfma_nrt(const AttnArgs &args, int NRT, int row_groups, dim3 grid, hipStream_t st) {
  switch (NRT) {
    case 1: k_attn_mfma<D, MODE, 1><<<grid, dim3(64), 0, st>>>(args, row_groups); break;
    case 2: k_attn_mfma<D, MODE, 2><<<grid, dim3(64), 0, st>>>(args, row_groups); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_attn_mfma(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const int NRT = p.nrt;
  const dim3 grid((unsigned)p.max_splits, (unsigned)(g.Hkv * p.row_groups), (unsigned)a.B);
  switch (g.D) {
    case 64:
      return g.mode == MODE_REF ? launch_mfma_nrt<64, MODE_REF>(args, NRT, p.row_groups, grid, st)
                                : launch_mfma_nrt<64, MODE_AFFINE>(args, NRT, p.row_groups, grid, st);
    case 128:
      return g.mode == MODE_REF ? launch_mfma_nrt<128, MODE_REF>(args, NRT, p.row_groups, grid, st)
                                : launch_mfma_nrt<128, MODE_AFFINE>(args, NRT, p.row_groups, grid, st);
    case 256:
      return g.mode == MODE_REF ? launch_mfma_nrt<256, MODE_REF>(args, NRT, p.row_groups, grid, st)
                                : launch_mfma_nrt<256, MODE_AFFINE>(args, NRT, p.row_groups, grid, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace krill
