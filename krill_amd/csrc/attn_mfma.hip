// Paged int8 attention with MFMA tiles: the speculative-verify / chunked-
// prefill path, used when a KV head serves more than 8 query rows
// (GQA group x new tokens).  Reference semantics: the same SDPA call with
// L > 1 new rows and the block-causal mask of
// Sources/KrillEngine/BatchedDecode.swift:299-312 (row j of the new window
// sees every cached key plus new keys 0..j), equivalently
// Sources/KrillCore/LlamaModel.swift:186-202.
//
// Work split as on the decode path: per (KV head, row group of 16 * NRT
// query rows) the blocks of all sequences are laid end to end and split
// evenly over the workgroups of the grid, crossing sequence boundaries; a
// sequence covered by several workgroups is combined by k_attn_merge_flat.
// A workgroup holds W waves, one row group each, that walk the same blocks
// (those the workgroup's last row group can see, for a causal window) and
// share one LDS ring.
//
// Memory: every block's head region (K, V and metadata, a whole number of
// contiguous 1 KB runs in the pool layout) is copied verbatim into the LDS
// ring with direct-to-LDS buffer loads (16 bytes per lane, no registers
// involved; with W waves each issues every W-th run), the next blocks in
// flight while the current one is computed; MFMA operands are then read from
// LDS.  One workgroup barrier per block (W > 1) publishes the block's runs to
// every wave and releases the stage the previous block used.
//
// Math: transposed scores, so no operand is ever transposed in registers:
//   S^T[tok][row] = K[tok][d] . Q^T[d][row]      v_mfma_f32_16x16x32_f16
//   O^T[d][row]  += V^T[d][tok] . P^T[tok][row]  v_mfma_f32_16x16x32_f16
// The 16-byte K chunks hold the 8 d of an A operand contiguously; V is stored
// per d in exactly the token order in which the S^T accumulator hands P to
// the P.V B operand.  Bytes become fp16 with one v_perm_b32 per pair (1024 + u,
// affine mode centres the K and V bytes, u - 128, exact, so the fp32 sums
// stay small, and adds the zero point plus 128 s on the side); affine
// scale/bias are applied to the fp32 scores (per group) and folded into the
// weights P*s_v, which enter P.V as a pair of fp16 operands (high and low
// part) against the exact V bytes.  The softmax max is raised lazily, so
// the weights stay below 2^8 and most blocks skip the accumulator rescale.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "attn_common.hpp"

namespace krill {


// LDS bytes of one staged block: the head region rounded up to whole 1 KB
// runs (one 16-byte-per-lane direct load each).
__host__ __device__ constexpr int mfma_stage_bytes(int D, int G) { return (head_region_bytes(D, G) + 1023) & ~1023; }
// Ring depth.  One wave per workgroup: two stages (measured: a third stage
// per wave costs a wave per compute unit, which costs more than the deeper
// prefetch gains).  W > 1 waves: three stages when 8 / W workgroups (two
// waves per SIMD) still fit the 160 KB of LDS of a compute unit, else two.
__host__ __device__ constexpr int mfma_stages(int D, int G, int W) {
  return W > 1 && 3 * mfma_stage_bytes(D, G) * (8 / W) <= 160 * 1024 ? 3 : 2;
}

// Two waves per SIMD for the 32-row, 4-wave, 128-d affine shape (chunked
// prefill): left alone the register allocator lands a few registers past
// the 256 that two waves may hold and the occupancy halves.
template <int D, int MODE, int NRT, int W>
constexpr int mfma_min_waves() { return D == 128 && MODE == MODE_AFFINE && NRT == 2 && W == 4 ? 2 : 1; }

// VAR: 0 plain; 1 RoPE of the queries; 2 sliding window (keys below
// max(win_start[b], position - window + 1) masked).
// TS: 1 -- the W waves of a workgroup hold W row groups and every wave
// works on all 64 tokens of a block; 2 (W = 2) -- both waves hold the same
// row group and split each block's tokens (wave w: tokens 32 w .. 32 w + 31,
// its own softmax state), so no byte is converted twice; at each segment
// end the two states are combined through the ring stage just consumed.
template <int D, int MODE, int NRT, int VAR, int W, int TS>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(mfma_min_waves<D, MODE, NRT, W>())))
void k_attn_mfma(AttnArgs a) {
  constexpr bool ROPE = VAR == 1, WIN = VAR == 2;
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int KS = D / 32;   // 32-d steps of Q.K^T
  constexpr int NDT = D / 16;  // 16-d tiles of P.V
  constexpr int RR = 16 * NRT; // query rows of this wave
  constexpr int STAGE = mfma_stage_bytes(D, G);
  constexpr int NCH = STAGE / 1024;  // direct loads per block
  // CVT (four-wave groups, affine, head_dim 128: chunked prefill, the
  // cascade's prefix pass): the four waves convert each staged block once,
  // a quarter each, into fp16 K and V^T tiles in LDS that all four read,
  // instead of every wave converting the whole block for its own rows; the
  // tiles take the LDS of the third ring stage
  constexpr bool CVT = W == 4 && TS == 1 && MODE == MODE_AFFINE && D == 128;
  constexpr int NST = CVT ? 2 : mfma_stages(D, G, W);
  constexpr int NK = 64 * D / 1024;  // runs holding the K bytes
  // W > 1: the fewest runs of a stage any wave of the group issues
  constexpr int NCH_W = NCH / W;
  static_assert((NST - 1) * NCH <= 63, "vmcnt immediate range");
  static_assert(W == 1 || W == 2 || W == 4, "waves per workgroup");
  static_assert(TS == 1 || (TS == 2 && W == 2), "token split: two waves");
  constexpr int WR = TS > 1 ? 1 : W;   // row groups per workgroup
  constexpr int NTT = 4 / TS;          // 16-token score tiles per wave and block
  constexpr int NTG = 2 / TS;          // 32-token P.V groups per wave and block
  static_assert(TS == 1 || NRT * NDT * 64 * 16 + NRT * 64 * 8 <= STAGE, "combine buffer fits a stage");
  __shared__ __attribute__((aligned(1024))) uint8_t ring[NST * STAGE];
  // CVT tiles: K [token][d] with rows KTS bytes apart, V^T [d][position] with
  // rows VTS bytes apart (the padding puts the 16 rows a lane quarter reads
  // in different banks)
  constexpr int KTS = D * 2 + 16, VTS = 64 * 2 + 16;
  __shared__ __attribute__((aligned(16))) uint8_t cvt_lds[CVT ? 64 * KTS + D * VTS : 16];

  const int lane = threadIdx.x & 63;
  const int wid = W > 1 ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;
  const int n = lane & 15, q4 = lane >> 4;
  const int RGB = (a.row_groups + WR - 1) / WR;  // workgroups per KV head and block range
  // range index rotated by the KV head, as in the decode kernel: range w of
  // the heads on different XCDs, while the row groups of one head, which
  // read the same bytes, keep range w on one XCD and share its L2
  const int hk = blockIdx.y / RGB, rg = (blockIdx.y % RGB) * WR + (TS > 1 ? 0 : wid);
  const int wv = (int)((blockIdx.x + (unsigned)hk) % gridDim.x);
  const int tt0 = TS > 1 ? wid * NTT : 0;  // first score tile / P.V group of this wave
  const int tg0 = TS > 1 ? wid * NTG : 0;
  const int RG = a.row_groups;
  const int rbase = rg * RR;  // rg >= RG (a group's spare wave): no valid row

  // ---- this workgroup's flat blocks [i0, iend) of the (head, row group) order
  const int NWG = a.waves;
  int c0 = 0, lenv = lane < a.B ? seq_len_view<WIN>(a, lane) : 0;
  int nbv = seq_blocks_rg(a, lenv, rg);
  int incl = wave_incl_scan(nbv);
  int T = __builtin_amdgcn_readlane(incl, 63);
  for (int cc = 64; cc < a.B; cc += 64) {
    const int bb = cc + lane;
    T += __builtin_amdgcn_readfirstlane(wave_allsum_int(bb < a.B ? seq_blocks_rg(a, seq_len_view<WIN>(a, bb), rg) : 0));
  }
  const int Wt = min(NWG, T);  // every participating workgroup holds >= 1 block
  if (wv >= Wt) return;
  const int i0 = (int)(((int64_t)wv * T + Wt - 1) / Wt);
  const int iend = (int)(((int64_t)(wv + 1) * T + Wt - 1) / Wt);
  int b = -1, s = 0;
  {
    int carry = 0;
    for (c0 = 0; c0 < a.B; c0 += 64) {
      if (c0 > 0) {
        const int bb = c0 + lane;
        lenv = bb < a.B ? seq_len_view<WIN>(a, bb) : 0;
        nbv = seq_blocks_rg(a, lenv, rg);
        incl = wave_incl_scan(nbv) + carry;
      }
      const unsigned long long m = __ballot(c0 + lane < a.B && incl > i0);
      if (m) {
        const int l = __builtin_ctzll(m);
        b = c0 + l;
        s = __builtin_amdgcn_readlane(incl - nbv, l);
        break;
      }
      carry = __builtin_amdgcn_readlane(incl, 63);
    }
  }
  if (b < 0) return;
  auto seq_len = [&](int bs) -> int { return bs - c0 < 64 ? __builtin_amdgcn_readlane(lenv, bs - c0) : seq_len_view<WIN>(a, bs); };

  // block-table entries of flat blocks i0 .. iend-1 (<= 64), lane j: block i0 + j
  int tab = 0, iend_eff = iend;
  {
    const int f = i0 + lane;
    int bs = b, ss = s;
    while (bs < a.B && ss < iend) {
      const int nbs = seq_blocks_rg(a, seq_len(bs), rg);
      if (f < iend && f >= ss && f < ss + nbs) {
        const int phys = a.tables[(int64_t)bs * a.max_blocks + table_offset<WIN>(a, bs) + (f - ss)];
        tab = (unsigned)phys < (unsigned)a.lv.num_blocks ? phys : 0;
      }
      ss += nbs;
      ++bs;
    }
    if (ss < iend) iend_eff = ss;
  }
  // Copies 1 KB runs [C0, C1) of flat block i into stage `buf` (after the
  // group's last block the resource is empty: the loads return zeros without
  // a memory access).  Runs [0, NK) are the K bytes, the rest V and metadata.
  // With W waves, wave wid copies runs C0 + wid, C0 + wid + W, ...
  auto issue = [&](int i, int buf, auto c0_, auto c1_) {
    constexpr int C0 = decltype(c0_)::value, C1 = decltype(c1_)::value;
    const bool ok = i < iend_eff;
    const int phys = __builtin_amdgcn_readlane(tab, ok ? i - i0 : 0);
    const __amdgpu_buffer_rsrc_t r = block_rsrc(head_region(a.lv, phys, hk), ok ? a.lv.head_bytes : 0);
    uint8_t *dst = ring + buf * STAGE;
    if constexpr (W == 1) {
#pragma unroll
      for (int c = C0; c < C1; ++c)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(dst + c * 1024), 16, c * 1024 + lane * 16, 0, 0, 2);
    } else {
#pragma unroll
      for (int c0 = C0; c0 < C1; c0 += W) {
        const int c = c0 + wid;
        if (c0 + W <= C1 || c < C1)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t *)(dst + c * 1024), 16, c * 1024 + lane * 16, 0, 0, 2);
      }
    }
  };
  using KRuns0 = std::integral_constant<int, 0>;
  using KRuns1 = std::integral_constant<int, NK>;
  using AllRuns = std::integral_constant<int, NCH>;

  // ---- Q^T operands of sequence bq: lane holds q[row n][32 ks + 8 q4 .. +8]
  half8_t qB[NRT][KS];
  float qsum[NRT][G];
  float q_up[NRT];  // the lane's row: softmax scale in log2 units times the query's 2^k
  bool rvalid[NRT];
#pragma unroll
  for (int rt = 0; rt < NRT; ++rt) rvalid[rt] = rbase + 16 * rt + n < a.NR;
  uint4 qraw[NRT][KS];
  int qlen = 0;  // length of the sequence whose queries are loaded (RoPE positions)
  auto load_q = [&](int bq) {
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const int r = rvalid[rt] ? rbase + 16 * rt + n : 0;
      const int hq = hk * a.R + r % a.R, j = r / a.R;
      const uint16_t *qp = q_row(a, bq, hq, j);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) qraw[rt][ks] = *reinterpret_cast<const uint4 *>(qp + 32 * ks + 8 * q4);
    }
    if constexpr (ROPE) qlen = seq_len(bq);
  };
  auto finish_q = [&]() {
    if constexpr (ROPE) {
      // lane's row (query position j = r / R, token qlen - Lq + j): the 8
      // elements of step ks < KS/2 turn with those of step ks + KS/2
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        const int r = rvalid[rt] ? rbase + 16 * rt + n : 0;
        const float *crow = rope_row(a, qlen - a.Lq + r / a.R, D);
#pragma unroll
        for (int ks = 0; ks < KS / 2; ++ks) {
          const int d = 32 * ks + 8 * q4;
          uint32_t lo[4] = {qraw[rt][ks].x, qraw[rt][ks].y, qraw[rt][ks].z, qraw[rt][ks].w};
          uint32_t hi[4] = {qraw[rt][ks + KS / 2].x, qraw[rt][ks + KS / 2].y, qraw[rt][ks + KS / 2].z,
                            qraw[rt][ks + KS / 2].w};
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const float2 c2 = *reinterpret_cast<const float2 *>(crow + d + 2 * w);
            const float2 s2 = *reinterpret_cast<const float2 *>(crow + D / 2 + d + 2 * w);
            if (a.q_dtype == DT_BF16)
              rope_pair_words<DT_BF16>(lo[w], hi[w], c2, s2);
            else
              rope_pair_words<DT_F16>(lo[w], hi[w], c2, s2);
          }
          qraw[rt][ks] = uint4{lo[0], lo[1], lo[2], lo[3]};
          qraw[rt][ks + KS / 2] = uint4{hi[0], hi[1], hi[2], hi[3]};
        }
      }
    }
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
      for (int g = 0; g < G; ++g) qsum[rt][g] = 0.0f;
      // bf16 rows at the fp16 range limit are scaled by 2^-k before the
      // rounding, their scores by 2^k (q_range_scale); the row's elements
      // sit in lanes n, n + 16, n + 32, n + 48
      float down = 1.0f, up = 1.0f;
      if (a.q_dtype == DT_BF16) {
        float mx = 0.0f;
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const uint32_t w4[4] = {qraw[rt][ks].x, qraw[rt][ks].y, qraw[rt][ks].z, qraw[rt][ks].w};
#pragma unroll
          for (int e = 0; e < 4; ++e)
            mx = fmaxf(mx, fmaxf(fabsf(__builtin_bit_cast(float, w4[e] << 16)),
                                 fabsf(__builtin_bit_cast(float, w4[e] & 0xffff0000u))));
        }
        mx = fmaxf(mx, shfl_xor(mx, 16));
        mx = fmaxf(mx, shfl_xor(mx, 32));
        down = q_range_scale(mx, up);
      }
      q_up[rt] = a.scale_log2 * up;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const uint32_t w4[4] = {qraw[rt][ks].x, qraw[rt][ks].y, qraw[rt][ks].z, qraw[rt][ks].w};
        half8_t v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          _Float16 lo, hi;
          if (a.q_dtype == DT_BF16) {
            lo = (_Float16)(__builtin_bit_cast(float, w4[e] << 16) * down);
            hi = (_Float16)(__builtin_bit_cast(float, w4[e] & 0xffff0000u) * down);
          } else {
            lo = __builtin_bit_cast(_Float16, (uint16_t)(w4[e] & 0xffffu));
            hi = __builtin_bit_cast(_Float16, (uint16_t)(w4[e] >> 16));
          }
          if (!rvalid[rt]) lo = hi = (_Float16)0.0f;
          v[2 * e] = lo;
          v[2 * e + 1] = hi;
          qsum[rt][MODE == MODE_AFFINE ? ks / 2 : 0] += (float)lo + (float)hi;
        }
        qB[rt][ks] = v;
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        qsum[rt][g] += shfl_xor(qsum[rt][g], 16);
        qsum[rt][g] += shfl_xor(qsum[rt][g], 32);
      }
    }
  };

  // queries first, then the first blocks (NST of them; W > 1: NST - 1, the
  // next one goes out once every wave is past the first barrier): waits on
  // the queries do not cover the block copies
  load_q(b);
#pragma unroll
  for (int k = 0; k < (W == 1 ? NST : NST - 1); ++k) issue(i0 + k, k, KRuns0{}, AllRuns{});
  finish_q();

  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};
  int i = i0;
  while (true) {
    const int len = seq_len(b);
    const int e = s + seq_blocks_rg(a, len, rg);
    const int seg_end = min(e, iend_eff);
    int lim[NRT];
#pragma unroll
    for (int rt = 0; rt < NRT; ++rt) {
      const int r = rbase + 16 * rt + n;
      lim[rt] = rvalid[rt] ? key_limit(a, len, r / a.R) : 0;
    }
    const int lim_lo = key_limit(a, len, rbase / a.R);  // keys seen by the group's first row
    int lo[NRT], wst = 0, lo_hi = 0;  // sliding window: per-row first key, first retained key, group's largest
    if constexpr (WIN) {
      wst = win_view_start(a, b);
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        const int r = rbase + 16 * rt + n;
        lo[rt] = max(wst, len - a.Lq + r / a.R - a.window + 1);
      }
      const int rlast = min(a.NR, rbase + RR) - 1;
      lo_hi = max(wst, len - a.Lq + rlast / a.R - a.window + 1);
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

    for (; i < seg_end; ++i) {
      const int buf = (i - i0) % NST;
      if constexpr (W == 1) {
        // stage `buf` holds block i once every load but the (NST - 1) * NCH
        // youngest (the other stages' copies, issued in the same K-then-rest
        // order) has completed
        asm volatile("s_waitcnt vmcnt(%0)" ::"n"((NST - 1) * NCH) : "memory");
      } else {
        // this wave's runs of block i have landed once at most the runs of
        // the NST - 2 later blocks in flight remain (at least NCH_W each);
        // its reads of block i - 1 have returned; the barrier then holds
        // every wave's runs of block i and frees the stage of block i - 1
        // for block i + NST - 1
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"((NST - 2) * NCH_W) : "memory");
        issue(i + NST - 1, (i + NST - 1 - i0) % NST, KRuns0{}, AllRuns{});
      }
      const uint8_t *st = ring + buf * STAGE;
      if constexpr (CVT) {
        // wave wid: K of tokens 16 wid .. +15 (lane: token 16 wid + lane / 4,
        // dims 32 (lane % 4) .. +31) and V^T rows 32 wid .. +31 (lane: row
        // 32 wid + lane / 2, token group lane % 2, its 32 positions), as exact
        // fp16 u - 128; then every wave's part is in before any is read
        {
          const int tok = 16 * wid + (lane >> 2), d0 = 32 * (lane & 3);
          const uint4 a = *reinterpret_cast<const uint4 *>(st + k_byte(tok, d0));
          const uint4 b = *reinterpret_cast<const uint4 *>(st + k_byte(tok, d0 + 16));
          uint8_t *o = cvt_lds + tok * KTS + d0 * 2;
          *reinterpret_cast<half8_t *>(o) = bytes8_centred(uint2{a.x, a.y});
          *reinterpret_cast<half8_t *>(o + 16) = bytes8_centred(uint2{a.z, a.w});
          *reinterpret_cast<half8_t *>(o + 32) = bytes8_centred(uint2{b.x, b.y});
          *reinterpret_cast<half8_t *>(o + 48) = bytes8_centred(uint2{b.z, b.w});
        }
        {
          const int d = 32 * wid + (lane >> 1), tgv = lane & 1;
          const uint4 a = *reinterpret_cast<const uint4 *>(st + v_pos_byte(D, tgv, d, 0));
          const uint4 b = *reinterpret_cast<const uint4 *>(st + v_pos_byte(D, tgv, d, 16));
          uint8_t *o = cvt_lds + 64 * KTS + d * VTS + 32 * tgv * 2;
          *reinterpret_cast<half8_t *>(o) = bytes8_centred(uint2{a.x, a.y});
          *reinterpret_cast<half8_t *>(o + 16) = bytes8_centred(uint2{a.z, a.w});
          *reinterpret_cast<half8_t *>(o + 32) = bytes8_centred(uint2{b.x, b.y});
          *reinterpret_cast<half8_t *>(o + 48) = bytes8_centred(uint2{b.z, b.w});
        }
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
      const int tbase = (i - s) << 6;
      // some row of this group does not see every token of the block (causal
      // edge or the sequence's last block): only then are scores masked
      bool edge = tbase + 64 > lim_lo;
      if constexpr (WIN) edge = edge || tbase < lo_hi;  // or below some row's window

      // ---- S^T = K . Q^T, four 16-token tiles.  Affine mode feeds the bytes
      // as exact fp16 u - 128 and folds the offset into the zero point:
      // q.k = s * (q.(u - 128)) + (z + 128 s) * sum q (per 64-d group).
      float sc[NTT][NRT][4];  // local tile t = score tile tt0 + t
#pragma unroll
      for (int t = 0; t < NTT; ++t) {
        const int tt = tt0 + t;
        const int tokA = 16 * tt + n;  // A-operand row
        half2_t ks2 = half2_t{(_Float16)0.0f, (_Float16)0.0f}, kz2 = ks2;
        if constexpr (MODE == MODE_REF) {
          const uint32_t km = *reinterpret_cast<const uint32_t *>(st + km_offset(D) + (tokA << 2));
          const _Float16 sk = __builtin_bit_cast(_Float16, (uint16_t)(km & 0xffffu));
          const _Float16 zk = __builtin_bit_cast(_Float16, (uint16_t)(km >> 16));
          ks2 = half2_t{sk, sk};
          kz2 = half2_t{zk, zk};
        }
        float4_t sacc[NRT][G];
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
          for (int g = 0; g < G; ++g) sacc[rt][g] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          half8_t A;
          if constexpr (CVT) {
            A = *reinterpret_cast<const half8_t *>(cvt_lds + tokA * KTS + (32 * ks + 8 * q4) * 2);
          } else if constexpr (MODE == MODE_REF) {
            const uint2 kb = *reinterpret_cast<const uint2 *>(st + k_byte(tokA, 32 * ks + 8 * q4));
            half2_t p0 = (bytes01_plus1024(kb.x) + m1024) * ks2 + kz2;
            half2_t p1 = (bytes23_plus1024(kb.x) + m1024) * ks2 + kz2;
            half2_t p2 = (bytes01_plus1024(kb.y) + m1024) * ks2 + kz2;
            half2_t p3 = (bytes23_plus1024(kb.y) + m1024) * ks2 + kz2;
            A = half8_t{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
          } else {
            A = bytes8_centred(*reinterpret_cast<const uint2 *>(st + k_byte(tokA, 32 * ks + 8 * q4)));
          }
          const int g = MODE == MODE_AFFINE ? ks / 2 : 0;
#pragma unroll
          for (int rt = 0; rt < NRT; ++rt) sacc[rt][g] = mfma16x16x32(A, qB[rt][ks], sacc[rt][g]);
        }
        // lane holds tokens 16*tt + 4*q4 + e for row n
        const int tok0 = 16 * tt + 4 * q4;
        if constexpr (MODE == MODE_AFFINE) {
          // (scale, zero) pairs of tokens tok0 .. tok0+3, G per token: 16 G contiguous bytes
          uint32_t km[4 * G];
#pragma unroll
          for (int c = 0; c < G; ++c) {
            const uint4 w = *reinterpret_cast<const uint4 *>(st + km_offset(D) + ((tok0 * G) << 2) + 16 * c);
            km[4 * c] = w.x;
            km[4 * c + 1] = w.y;
            km[4 * c + 2] = w.z;
            km[4 * c + 3] = w.w;
          }
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            float kss[G], kzz[G];
#pragma unroll
            for (int g = 0; g < G; ++g) {
              kss[g] = f16_bits_to_f32((uint16_t)(km[e * G + g] & 0xffffu));
              kzz[g] = fmaf(128.0f, kss[g], f16_bits_to_f32((uint16_t)(km[e * G + g] >> 16)));
            }
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
              float sv = 0.0f;
#pragma unroll
              for (int g = 0; g < G; ++g) sv = fmaf(kss[g], sacc[rt][g][e], fmaf(kzz[g], qsum[rt][g], sv));
              sc[t][rt][e] = sv * q_up[rt];
            }
          }
        } else {
#pragma unroll
          for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[t][rt][e] = sacc[rt][0][e] * q_up[rt];
        }
      }
      // the K bytes of this stage are consumed: refill them NST blocks ahead
      if constexpr (W == 1) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + NST, buf, KRuns0{}, KRuns1{});
      }
      if (edge) {
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
          for (int rt = 0; rt < NRT; ++rt)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int tok = tbase + 16 * (tt0 + t) + 4 * q4 + e;
              if (tok >= lim[rt] || (WIN && tok < lo[rt])) sc[t][rt][e] = -INFINITY;
            }
      }

      // ---- online softmax with a lazily raised running max (row n of each
      // tile; its 64 scores live in the four lanes n, n+16, n+32, n+48): the
      // max only moves when some score exceeds it by more than 2^8, so the
      // weights stay below 2^8 and most blocks skip the rescale
      float mb[NRT];
      bool over = false;
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        float v = -INFINITY;
#pragma unroll
        for (int t = 0; t < NTT; ++t)
          v = fmaxf(v, fmaxf(fmaxf(sc[t][rt][0], sc[t][rt][1]), fmaxf(sc[t][rt][2], sc[t][rt][3])));
        v = fmaxf(v, shfl_xor(v, 16));
        v = fmaxf(v, shfl_xor(v, 32));
        mb[rt] = v;
        over |= v > m_run[rt] + 8.0f;
      }
      if (__any(over)) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          const float mn = fmaxf(m_run[rt], mb[rt]);
          const float al = m_run[rt] == -INFINITY ? 0.0f : fast_exp2(m_run[rt] - mn);
          m_run[rt] = mn;
          l_part[rt] *= al;
#pragma unroll
          for (int g = 0; g < G; ++g) c_part[rt][g] *= al;
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) oacc[rt][dt] *= al;
        }
      }
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        const float mu = m_run[rt] == -INFINITY ? 0.0f : m_run[rt];
        float ps = 0.0f;
#pragma unroll
        for (int t = 0; t < NTT; ++t)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            sc[t][rt][e] = fast_exp2(sc[t][rt][e] - mu);
            ps += sc[t][rt][e];
          }
        l_part[rt] += ps;
      }

      // ---- O^T += V^T . P^T over two 32-token groups; weights p * s_v
      // (below 2^8 * s_v) as fp16 high and low parts, V bytes as exact fp16
      // u - 128, the zero points (and 128 s_v) summed on the side
#pragma unroll
      for (int tgi = 0; tgi < NTG; ++tgi) {
        const int tg = tg0 + tgi;
        // logical k = 8*q4 + i  <->  token 32*tg + (i < 4 ? 4*q4 + i : 16 + 4*q4 + i - 4)
        // the (scale, zero) words of the 8 k positions (zero past the data)
        uint32_t vmw[8][G];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int tokh = 32 * tg + 16 * h + 4 * q4;  // 4 tokens, G pairs each: 16 G bytes
#pragma unroll
          for (int c = 0; c < G; ++c) {
            const uint4 w = *reinterpret_cast<const uint4 *>(st + vm_offset(D, G) + ((tokh * G) << 2) + 16 * c);
            const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
            for (int k2 = 0; k2 < 4; ++k2) vmw[4 * h + (4 * c + k2) / G][(4 * c + k2) % G] = ww[k2];
          }
          if (edge) {  // metadata past the sequence's end is not data
#pragma unroll
            for (int e = 0; e < 4; ++e)
              if (tbase + tokh + e >= len || (WIN && tbase + tokh + e < wst))
#pragma unroll
                for (int g = 0; g < G; ++g) vmw[4 * h + e][g] = 0u;
          }
        }
        // Each binary32 weight w = p * s_v (affine) or p (row mode) goes in as
        // two fp16 operands, w_hi = f16(w) and w_lo = f16(w - w_hi), against
        // the same exact V operand: one fp16 weight would carry a relative
        // error of 2^-11 into every product, up to 2^-11 of a group's value
        // range in the output when a few keys hold the softmax weight; the
        // pair leaves about 2^-22.  One scale group at a time, so only its
        // operands are live.
#pragma unroll
        for (int g = 0; g < G; ++g) {
          half8_t Bh[NRT], Bl[NRT];
#pragma unroll
          for (int rt = 0; rt < NRT; ++rt) {
            float w8[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
              const float p = sc[2 * tgi + (k >> 2)][rt][k & 3];  // score tile 2 tg + k / 4
              const float vsf = f16_bits_to_f32((uint16_t)(vmw[k][g] & 0xffffu));
              w8[k] = MODE == MODE_AFFINE ? p * vsf : p;
              // the zero point and the 128 taken off the V bytes: p (z + 128 s)
              if constexpr (MODE == MODE_AFFINE)
                c_part[rt][g] = fmaf(p, fmaf(128.0f, vsf, f16_bits_to_f32((uint16_t)(vmw[k][g] >> 16))), c_part[rt][g]);
            }
            split_hi_lo(float4{w8[0], w8[1], w8[2], w8[3]}, float4{w8[4], w8[5], w8[6], w8[7]}, Bh[rt], Bl[rt]);
          }
          uint4 sc4 = {0u, 0u, 0u, 0u}, zc4 = {0u, 0u, 0u, 0u};
          if constexpr (MODE == MODE_REF) {
            sc4 = uint4{(vmw[0][0] & 0xffffu) | (vmw[1][0] << 16), (vmw[2][0] & 0xffffu) | (vmw[3][0] << 16),
                        (vmw[4][0] & 0xffffu) | (vmw[5][0] << 16), (vmw[6][0] & 0xffffu) | (vmw[7][0] << 16)};
            zc4 = uint4{(vmw[0][0] >> 16) | (vmw[1][0] & 0xffff0000u), (vmw[2][0] >> 16) | (vmw[3][0] & 0xffff0000u),
                        (vmw[4][0] >> 16) | (vmw[5][0] & 0xffff0000u), (vmw[6][0] >> 16) | (vmw[7][0] & 0xffff0000u)};
          }
#pragma unroll
          for (int t2 = 0; t2 < NDT / G; ++t2) {
            const int dt = g * (NDT / G) + t2;
            const int d = 16 * dt + n;
            half8_t A;
            if constexpr (CVT) {
              A = *reinterpret_cast<const half8_t *>(cvt_lds + 64 * KTS + d * VTS + (32 * tg + 8 * q4) * 2);
            } else {
              const uint2 vb = *reinterpret_cast<const uint2 *>(st + v_pos_byte(D, tg, d, 8 * q4));
              A = MODE == MODE_REF ? bytes8_dequant_ref(vb, sc4, zc4) : bytes8_centred(vb);
            }
#pragma unroll
            for (int rt = 0; rt < NRT; ++rt) {
              oacc[rt][dt] = mfma16x16x32(A, Bh[rt], oacc[rt][dt]);
              oacc[rt][dt] = mfma16x16x32(A, Bl[rt], oacc[rt][dt]);
            }
          }
        }
      }
      // every LDS read of this stage has returned: refill the rest
      if constexpr (W == 1) {
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        issue(i + NST, buf, KRuns1{}, AllRuns{});
      }
    }

    if constexpr (TS > 1) {
      // ---- token split: wave 1's state of this segment (its half of every
      // block's tokens) joins wave 0's through the ring stage of the block
      // just consumed (no load targets it before the next block's barrier):
      // O = a0 O0 + a1 O1, l = a0 l0 + a1 l1, a_w = 2^(m_w - max(m0, m1)).
      // Each wave first folds its zero-point sums into O.
      float *xo = reinterpret_cast<float *>(ring + ((i - 1 - i0) % NST) * STAGE);
      float lw[NRT];
#pragma unroll
      for (int rt = 0; rt < NRT; ++rt) {
        float l = l_part[rt];
        l += shfl_xor(l, 16);
        l += shfl_xor(l, 32);
        lw[rt] = l;
#pragma unroll
        for (int g = 0; g < G; ++g) {
          float c = c_part[rt][g];
          c += shfl_xor(c, 16);
          c += shfl_xor(c, 32);
          c_part[rt][g] = 0.0f;
#pragma unroll
          for (int t2 = 0; t2 < NDT / G; ++t2) oacc[rt][g * (NDT / G) + t2] += c;
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");  // both waves are done with the stage
      if (wid == 1) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) *reinterpret_cast<float4_t *>(xo + ((rt * NDT + dt) * 64 + lane) * 4) = oacc[rt][dt];
          *reinterpret_cast<float2 *>(xo + NRT * NDT * 256 + (rt * 64 + lane) * 2) = float2{m_run[rt], lw[rt]};
        }
      }
      asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      if (wid == 0) {
#pragma unroll
        for (int rt = 0; rt < NRT; ++rt) {
          const float2 ml1 = *reinterpret_cast<const float2 *>(xo + NRT * NDT * 256 + (rt * 64 + lane) * 2);
          const float M = fmaxf(m_run[rt], ml1.x);
          const float a0 = m_run[rt] == -INFINITY ? 0.0f : fast_exp2(m_run[rt] - M);
          const float a1 = ml1.x == -INFINITY ? 0.0f : fast_exp2(ml1.x - M);
#pragma unroll
          for (int dt = 0; dt < NDT; ++dt) {
            const float4_t o1 = *reinterpret_cast<const float4_t *>(xo + ((rt * NDT + dt) * 64 + lane) * 4);
            oacc[rt][dt] = oacc[rt][dt] * a0 + o1 * a1;
          }
          m_run[rt] = M;
          l_part[rt] = q4 == 0 ? a0 * lw[rt] + a1 * ml1.y : 0.0f;  // the epilogue sums the four quarter lanes
        }
      }
    }

    // ---- end of the segment: lane holds O^T[d = 16*dt + 4*q4 + e][row n].
    // The whole sequence in this wave -> output; otherwise a partial in slot
    // (hk * row_groups + rg) * (waves + B) + wave + b.  Token split: wave 0
    // writes the combined state.
    const bool whole = !a.partial_only && s >= i0 && e <= iend;
    const int64_t slot = ((int64_t)hk * RG + rg) * (a.waves + a.B) + wv + b;
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
      if (!rvalid[rt] || (TS > 1 && wid != 0)) continue;
      const int r = rbase + 16 * rt + n;
      if (whole) {
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt)
#pragma unroll
          for (int e2 = 0; e2 < 4; ++e2) {
            const int d = 16 * dt + 4 * q4 + e2;
            store_out(a.out, ob + d, (oacc[rt][dt][e2] + cg[MODE == MODE_AFFINE ? d / 64 : 0]) * inv, a.out_dtype);
          }
      } else {
        const int64_t pi = slot * RR + 16 * rt + n;
#pragma unroll
        for (int dt = 0; dt < NDT; ++dt) {
          float4 o;
          const int d = 16 * dt + 4 * q4;
          const float c = cg[MODE == MODE_AFFINE ? d / 64 : 0];
          o.x = oacc[rt][dt][0] + c;
          o.y = oacc[rt][dt][1] + c;
          o.z = oacc[rt][dt][2] + c;
          o.w = oacc[rt][dt][3] + c;
          *reinterpret_cast<float4 *>(a.ws_o + pi * D + d) = o;
        }
        if (q4 == 0) reinterpret_cast<float2 *>(a.ws_ml)[pi] = float2{m_run[rt], l};
      }
    }
    if (i >= iend_eff) break;
    // next sequence with blocks for this row group (the merge zero-fills the others)
    ++b;
    s = e;
    while (b < a.B && seq_blocks_rg(a, seq_len(b), rg) == 0) ++b;
    if (b >= a.B) break;
    load_q(b);
    finish_q();
  }
  // the loads issued after the last block (empty resources) still write the
  // ring: let them land before the wave ends
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
}

template <int D, int MODE, int NRT, int W, int TS>
static hipError_t launch_mfma_w(const AttnArgs &args, dim3 grid, hipStream_t st) {
  const dim3 block(64 * W);
  if (args.rope_cs)
    k_attn_mfma<D, MODE, NRT, 1, W, TS><<<grid, block, 0, st>>>(args);
  else if (args.window > 0)
    k_attn_mfma<D, MODE, NRT, 2, W, TS><<<grid, block, 0, st>>>(args);
  else
    k_attn_mfma<D, MODE, NRT, 0, W, TS><<<grid, block, 0, st>>>(args);
  return hipGetLastError();
}

// (nrt, group_waves, token_split) shapes the plan may choose: 16-row waves
// in workgroups of 1, 2 or 4 row groups, or (D <= 128) a 32-row group split
// over two waves by tokens, or (D <= 128) 32-row waves in workgroups of 4.
template <int D, int MODE>
static hipError_t launch_mfma_dm(const AttnArgs &args, const AttnPlan &p, dim3 grid, hipStream_t st) {
  if (p.token_split == 2) {
    if constexpr (D <= 128) {
      if (p.nrt == 2 && p.group_waves == 1) return launch_mfma_w<D, MODE, 2, 2, 2>(args, grid, st);
    }
    return hipErrorInvalidValue;
  }
  if (p.token_split != 1) return hipErrorInvalidValue;
  if (p.nrt == 2) {
    if constexpr (D <= 128) {
      if (p.group_waves == 4) return launch_mfma_w<D, MODE, 2, 4, 1>(args, grid, st);
    }
    return hipErrorInvalidValue;
  }
  if (p.nrt != 1) return hipErrorInvalidValue;
  switch (p.group_waves) {
    case 1: return launch_mfma_w<D, MODE, 1, 1, 1>(args, grid, st);
    case 2: return launch_mfma_w<D, MODE, 1, 2, 1>(args, grid, st);
    case 4: return launch_mfma_w<D, MODE, 1, 4, 1>(args, grid, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_attn_mfma(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  // one VGPR of block-table entries per workgroup
  if (p.waves < 1 || (int64_t)p.waves * 64 < (int64_t)a.B * p.nb_cap) return hipErrorInvalidValue;
  if (p.rows_per_group != 16 * p.nrt || p.row_groups * p.rows_per_group < p.NR) return hipErrorInvalidValue;
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const int groups = (p.row_groups + p.group_waves - 1) / p.group_waves;
  const dim3 grid((unsigned)p.waves, (unsigned)(g.Hkv * groups));
  switch (g.D) {
    case 64:
      return g.mode == MODE_REF ? launch_mfma_dm<64, MODE_REF>(args, p, grid, st)
                                : launch_mfma_dm<64, MODE_AFFINE>(args, p, grid, st);
    case 128:
      return g.mode == MODE_REF ? launch_mfma_dm<128, MODE_REF>(args, p, grid, st)
                                : launch_mfma_dm<128, MODE_AFFINE>(args, p, grid, st);
    case 256:
      return g.mode == MODE_REF ? launch_mfma_dm<256, MODE_REF>(args, p, grid, st)
                                : launch_mfma_dm<256, MODE_AFFINE>(args, p, grid, st);
    default:
      return hipErrorInvalidValue;
  }
}

template <int D, int MODE, int NRT, int W, int TS>
static int32_t occupancy_mfma() {
  int n = 0;
  const hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(
      &n, reinterpret_cast<const void *>(&k_attn_mfma<D, MODE, NRT, 0, W, TS>), 64 * W, 0);
  if (e != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
    n = (160 * 1024) / (mfma_stages(D, G, W) * mfma_stage_bytes(D, G));
  }
  return n;
}

template <int D, int MODE>
static int32_t occupancy_mfma_sel(int sel) {
  switch (sel) {
    case 0: return occupancy_mfma<D, MODE, 1, 1, 1>();
    case 1: return occupancy_mfma<D, MODE, 1, 2, 1>();
    case 2: return occupancy_mfma<D, MODE, 1, 4, 1>();
    case 3:
      if constexpr (D <= 128) return occupancy_mfma<D, MODE, 2, 2, 2>();
      return 1;
    default:
      if constexpr (D <= 128) return occupancy_mfma<D, MODE, 2, 4, 1>();
      return 1;
  }
}

int32_t mfma_groups_per_cu(const PoolGeometry &g, int32_t nrt, int32_t group_waves, int32_t token_split) {
  const int dsel = g.D == 64 ? 0 : g.D == 128 ? 1 : 2;
  const int sel = token_split == 2 ? 3 : nrt == 2 ? 4 : group_waves == 4 ? 2 : group_waves == 2 ? 1 : 0;
  if (g.num_cus <= 0) {  // host-only pool: the LDS bound (the ring per workgroup, 160 KB per CU)
    static const int est[3][5] = {{5, 5, 3, 8, 3}, {3, 3, 2, 4, 2}, {1, 1, 1, 1, 1}};
    return est[dsel][sel];
  }
  static int cache[2][3][5] = {};  // [mode][D][shape], filled on first use per process
  int &c = cache[g.mode == MODE_AFFINE][dsel][sel];
  if (c == 0) {
    int v;
    if (g.D == 64) v = g.mode == MODE_REF ? occupancy_mfma_sel<64, MODE_REF>(sel) : occupancy_mfma_sel<64, MODE_AFFINE>(sel);
    else if (g.D == 128) v = g.mode == MODE_REF ? occupancy_mfma_sel<128, MODE_REF>(sel) : occupancy_mfma_sel<128, MODE_AFFINE>(sel);
    else v = g.mode == MODE_REF ? occupancy_mfma_sel<256, MODE_REF>(sel) : occupancy_mfma_sel<256, MODE_AFFINE>(sel);
    c = v;
  }
  return c;
}

}  // namespace krill
