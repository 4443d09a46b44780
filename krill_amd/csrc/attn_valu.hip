// Paged int8 decode attention, one token per lane for the scores: the path
// for up to 8 query rows per KV head (GQA group x query length).
//
// Computes o = softmax(scale * q K^T) V over each sequence's paged int8
// cache -- what MLXFast.scaledDotProductAttention computes on the
// dequantized cache at Sources/KrillCore/Gemma4Model.swift:516-517 and
// Sources/KrillCore/Attention.swift:95-98, with the left-pad mask of
// Sources/KrillEngine/BatchedDecode.swift:277-287 replaced by per-row lengths
// (the -10000 mask underflows those weights to exactly zero, :22-28).
//
// Work split: per KV head, the 64-token blocks of all sequences are laid end
// to end (flat order) and each wave64 takes the same number of consecutive
// blocks, crossing sequence boundaries, so every wave streams the same bytes
// whatever the length mix.  A wave processes its range one sequence segment
// at a time; for each it rounds the query rows to fp16 pairs held in VGPRs
// (each 16-lane DPP row holds the whole query) and, in affine mode, sums
// them per 64-d group.  Per block:
//  * scores, one token per lane: the lane reads its token's K row (D bytes,
//    16-byte loads that are contiguous across lanes in the d-chunk-major
//    layout), turns byte pairs into fp16 (1024 + u) with one v_perm_b32, and
//    accumulates v_dot2c_f32_f16 whose query operand is broadcast from the
//    right lane of the row by DPP row_newbcast.  Affine mode centres the
//    bytes (u - 128, exact in fp16, so the fp32 sums stay small) and uses
//    linearity per 64-group:
//      q.k = s * (q.(u - 128)) + (z + 128 s) * sum q,
//    so no element is dequantised.  Reference row mode dequantises exactly
//    (f16(f16(u*s) + z), QuantizedKVCache.swift:200-204) before the dot.
//    Where P.V runs on the matrix cores (below) -- head_dim 128 with 3-8
//    rows on the flat split, and head_dim 512 (four d-slice waves, up to 8
//    rows each) -- the same fp16 operands go to v_mfma_f32_16x16x32_f16
//    instead (S^T tiles of 16 tokens x 16 rows, 16 MFMAs per block and wave
//    in place of 64 v_dot2c per row and 128-d slice), and the per-group
//    sums return to one token per lane through LDS;
//  * online softmax in the log2 domain with a lazily raised running max: a
//    block only pays for a wave reduction when some score exceeds the
//    running max by more than 8 (a wave vote), so weights stay below 2^8;
//  * weights w = p * s_v (binary32) go to LDS in V storage order, and P.V
//    runs on the matrix cores: O^T += V^T . P^T per 16-row d tile with
//    v_mfma_f32_16x16x32_f16, A = the V bytes as exact fp16 (u - 128; row
//    mode: dequantized), B = each weight as an fp16 high part plus the fp16
//    rounding of its remainder (two MFMAs, about 2^-22 relative error left;
//    one fp16 weight would put up to 2^-11 of a group's value range into the
//    output whenever a few keys hold the softmax weight).  The V zero points
//    collapse into one per-(row, group) term.  On the VALU this product was
//    two thirds of the kernel's instructions, which made the kernel issue-
//    bound; on the matrix cores it is 32 MFMAs per block.
//  * the next block's K bytes and metadata are loaded as soon as the
//    current block's K registers are consumed (in flight through the
//    softmax and P.V), its V bytes once the V registers are.
// A sequence that lies inside one wave's range is written directly;
// otherwise each wave writes its segment's (m, l, o) to the workspace and
// k_attn_merge_flat combines them in a second launch.  (Merging inside the
// last wave to finish would need an agent-scope release/acquire per wave,
// which on this multi-XCD part is a whole-L2 writeback and invalidate.)
#include <hip/hip_runtime.h>

#include "attn_common.hpp"

namespace krill {

#ifdef KRILL_WAVE_STAMPS
// Diagnostic build only (make stamps): per wave of the last launch, the
// realtime clock (100 MHz) at its start, when its first block and queries
// are in registers and at its end, its hardware ids, its blocks and
// sequence segments.
constexpr int kStampWaves = 65536;
__device__ unsigned long long g_wave_stamps[kStampWaves * 6];
#endif

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

// Streaming (non-temporal) loads: each block byte is read once per launch.
__device__ __forceinline__ uint4 ld_stream16(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2));
}
// N consecutive 32-bit words (N = 1, 2 or 4) in one load.
template <int N>
__device__ __forceinline__ void ld_stream_words(__amdgpu_buffer_rsrc_t r, int off, uint32_t (&w)[N]) {
  if constexpr (N == 1) {
    w[0] = __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, 2);
  } else if constexpr (N == 2) {
    const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 2);
    w[0] = v[0];
    w[1] = v[1];
  } else {
    static_assert(N == 4, "1, 2 or 4 words");
    const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 2);
    w[0] = v[0];
    w[1] = v[1];
    w[2] = v[2];
    w[3] = v[3];
  }
}

// Waves per SIMD the register budget aims for: 3 (168 VGPRs) for D = 64,
// else 2 (the MFMA accumulators of 16 rows x D take 2 D / 16 VGPRs; with K
// and V both in registers D = 128 needs about 220).  Measured on the
// Qwen3-14B B = 32 step (D = 128, 5 rows): 2 waves with K and V in
// registers 68.4 us per call; 3 waves with K staged in LDS 75.0 us (the
// compiler orders every LDS access after the outstanding direct-to-LDS
// loads, which drains the K prefetch); 2 waves with K in LDS 70.0 us.
// head_dim 512: each block is split over d_slices = 4 waves of one
// workgroup, 128 dims each (a 512-byte K row per lane and 32 V tiles would not
// fit one wave's registers).  Every wave holds its slice's query pairs, K
// pieces, V tiles and output tiles, exactly the register set of the D = 128
// kernel (the slice's scores on the matrix cores, MSC below); the partial
// scores of the four slices meet in LDS (one barrier per block), and every
// wave then runs the same softmax on the same sums.
template <int D>
constexpr int d_slices() {
  return D > 256 ? D / 128 : 1;
}
// KRILL_PV_ON_VALU (the libkrillhip_pvvalu.so diagnostic build) keeps P.V
// on the VALU with binary32 weights wherever one wave holds the whole head,
// for timing the two forms against each other on one build.
template <int D, int NR>
constexpr bool pv_on_mfma() {
#ifdef KRILL_PV_ON_VALU
  return D > 256;
#else
  return (D <= 128 && NR >= 3) || D > 256;
#endif
}
template <int D, int NR>
constexpr int valu_waves_per_simd() {
  if constexpr (D > 256) return 2;
  if constexpr (pv_on_mfma<D, NR>()) return D <= 64 ? 3 : 2;
  return D <= 64 || (D == 128 && NR <= 5) ? 3 : 2;
}

// Sliding-window launches with the whole head in one wave (VAR 2 and 3,
// head_dim <= 256): a window keeps every sequence short and about equally
// long, so instead of the flat split each (sequence, KV head) gets one
// workgroup whose waves split that sequence's blocks and combine their
// partials in LDS after a barrier -- no merge launch.  Waves per workgroup:
// what a compute unit holds of the kernel (8 at two waves per SIMD, 6 at
// three, 8 at four), halved while the waves' LDS (scaled weights, V scale
// pairs, the new row, the RoPE row, the partial) exceeds 64 KB; 0 for the
// flat split.
template <int D, int NR, int MODE, int VAR>
constexpr int seq_waves() {
  if constexpr (!(VAR == 2 || VAR == 3) || D > 256) {
    return 0;
  } else {
    constexpr int GW = MODE == MODE_AFFINE ? D / 64 : 1;
    constexpr int pwb = NR * GW * 64 * 4 + 2 * 64 * 2 + 2 * D + (VAR == 3 ? 4 * D : 0) + NR * (D + 4) * 4;
    constexpr int wps = valu_waves_per_simd<D, NR>();
    int w = wps == 3 ? 6 : 8;
    while (w > 1 && w * pwb > 64 * 1024) w /= 2;
    return w;
  }
}
// Most blocks of one sequence a windowed workgroup's wave may read (one VGPR
// of block-table entries per wave).
template <int D, int NR, int MODE, int VAR>
constexpr int seq_max_blocks() {
  return 64 * seq_waves<D, NR, MODE, VAR>();
}

// LDS written and read by the lanes of one wave only: a wave's LDS
// operations complete in order, so waiting for its outstanding ones (and
// keeping the compiler from moving memory operations across) orders the
// writes before the other lanes' reads without a workgroup barrier.
__device__ __forceinline__ void wave_lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

// The step's new K/V rows of sequence b, head hk: lane l loads the raw
// elements d = l*E .. l*E+E-1 (E = D/64), the quantizer's lane ownership.
template <int D>
__device__ __forceinline__ void load_new_rows(const AttnArgs &a, int b, int hk, uint16_t (&rk)[D / 64],
                                              uint16_t (&rv)[D / 64]) {
  constexpr int E = D / 64;
  const int64_t off = (int64_t)b * a.kn_sb + (int64_t)hk * a.kn_sh + (threadIdx.x & 63) * E;
#pragma unroll
  for (int e = 0; e < E; ++e) {
    rk[e] = a.k_new[off + e];
    rv[e] = a.v_new[off + e];
  }
}

// Quantizes rows loaded by load_new_rows with the append kernels'
// quantize_row, leaving the K row's D bytes and then the V row's in `newrow`
// (LDS) and the (scale, zero) words of each group in pkm / pvm (uniform).
// The wave patches the token into its registers when it reaches its block
// and stores it (store_newest) at the end of the segment, where the
// segment's output stores go too: a store issued mid-segment would hold up
// every later wait on the in-order memory counter.
template <int D, int MODE, int DT>
__device__ __forceinline__ void prepare_newest(const uint16_t (&rk)[D / 64], const uint16_t (&rv)[D / 64],
                                               uint8_t *newrow, uint32_t (&pkm)[MODE == MODE_AFFINE ? D / 64 : 1],
                                               uint32_t (&pvm)[MODE == MODE_AFFINE ? D / 64 : 1]) {
  constexpr int E = D / 64;
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  constexpr int LPG = MODE == MODE_AFFINE ? 64 / E : 64;  // lanes per scale group
  const int lane = threadIdx.x & 63;
  float xk[E], xv[E];
#pragma unroll
  for (int e = 0; e < E; ++e) {
    xk[e] = elem_to_f32<DT>(rk[e]);
    xv[e] = elem_to_f32<DT>(rv[e]);
  }
  uint8_t qk[E], qv[E];
  float ks, kz, vs, vz;
  quantize_row<D, MODE, DT>(xk, qk, ks, kz);
  quantize_row<D, MODE, DT>(xv, qv, vs, vz);
#pragma unroll
  for (int e = 0; e < E; ++e) {
    newrow[lane * E + e] = qk[e];
    newrow[D + lane * E + e] = qv[e];
  }
  const uint32_t mk = (uint32_t)f32_to_f16_bits(ks) | ((uint32_t)f32_to_f16_bits(kz) << 16);
  const uint32_t mv = (uint32_t)f32_to_f16_bits(vs) | ((uint32_t)f32_to_f16_bits(vz) << 16);
#pragma unroll
  for (int g = 0; g < G; ++g) {
    pkm[g] = __builtin_amdgcn_readlane(mk, g * LPG);
    pvm[g] = __builtin_amdgcn_readlane(mv, g * LPG);
  }
}

// Stores the token prepared by prepare_newest as token t of physical block
// phys: the bytes and words store_row writes for the same rows.
template <int D, int MODE>
__device__ __forceinline__ void store_newest(const AttnArgs &a, int hk, int phys, int t, const uint8_t *newrow,
                                             const uint32_t (&pkm)[MODE == MODE_AFFINE ? D / 64 : 1],
                                             const uint32_t (&pvm)[MODE == MODE_AFFINE ? D / 64 : 1]) {
  constexpr int E = D / 64;
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  const int lane = threadIdx.x & 63;
  uint8_t *reg = head_region(a.lv, phys, hk);
  const int d0 = lane * E;
  uint8_t *kd = reg + k_byte(t, d0);
  if constexpr (E == 1) {
    kd[0] = newrow[d0];
  } else if constexpr (E == 2) {
    *reinterpret_cast<uint16_t *>(kd) = *reinterpret_cast<const uint16_t *>(newrow + d0);
  } else if constexpr (E == 4) {
    *reinterpret_cast<uint32_t *>(kd) = *reinterpret_cast<const uint32_t *>(newrow + d0);
  } else {
    *reinterpret_cast<uint2 *>(kd) = *reinterpret_cast<const uint2 *>(newrow + d0);
  }
#pragma unroll
  for (int e = 0; e < E; ++e) reg[v_byte(D, t, d0 + e)] = newrow[D + d0 + e];
  uint32_t mk = pkm[0], mv = pvm[0];  // lane g < G stores group g's words
#pragma unroll
  for (int g = 1; g < G; ++g) {
    mk = lane == g ? pkm[g] : mk;
    mv = lane == g ? pvm[g] : mv;
  }
  if (lane < G) {
    *reinterpret_cast<uint32_t *>(reg + km_offset(D) + ((t * G + lane) << 2)) = mk;
    *reinterpret_cast<uint32_t *>(reg + vm_offset(D, G) + ((t * G + lane) << 2)) = mv;
  }
}

// VAR: 0 plain; 1 RoPE of the queries (and the fused new K row); 2 sliding
// window (keys below max(win_start[b], position - window + 1) masked); 3
// both (the sliding layers of a rotating model's decode step).
// head_dim 512 (d_slices > 1): workgroups of d_slices waves, wave w the dims
// [DW w, DW w + DW); the query rows of a KV head in row groups of NR rows
// (blockIdx.z), each its own flat block order and partial slots.
template <int D, int NR, int MODE, int VAR>
__global__ __launch_bounds__(64 * (seq_waves<D, NR, MODE, VAR>() > 0 ? seq_waves<D, NR, MODE, VAR>() : d_slices<D>()),
                             (valu_waves_per_simd<D, NR>())) void k_attn_valu(AttnArgs a) {
  constexpr bool ROPE = VAR == 1 || VAR == 3, WIN = VAR == 2 || VAR == 3;
  constexpr int DS = d_slices<D>();  // waves per workgroup, one per d-slice
  // windowed: one workgroup per (sequence, KV head), partials merged in LDS
  constexpr int SW = seq_waves<D, NR, MODE, VAR>();
  constexpr bool SEQ = SW > 0;
  constexpr int NWV = SEQ ? SW : DS;  // waves with LDS of their own
  constexpr int DW = D / DS;         // dims of one wave
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;    // scale groups per token (pool layout)
  constexpr int GW = MODE == MODE_AFFINE ? DW / 64 : 1;  // the wave's scale groups
  constexpr int NP = DW / 16;  // the wave's 16-byte K pieces per token row
  constexpr int PPG = NP / GW; // pieces per scale group
  constexpr int DPL = D / 64;  // V^T rows (d values) per lane (pool layout)
  // P.V on the matrix cores (16 query rows per MFMA tile, so worth it from 3
  // rows on and while its 2 D / 16 accumulator registers per lane fit) or on
  // the VALU (lane owns D / 64 rows of V^T, fp32 FMAs)
  constexpr bool PVM = pv_on_mfma<D, NR>();
  constexpr bool LOAD_TOGETHER = !PVM && valu_waves_per_simd<D, NR>() >= 3;  // next block's loads in one pass
  // MSC -- P.V on the matrix cores and a flat split (head_dim 128, 3-8
  // rows), or d-slices (head_dim 512): the scores there too.  Lane l loads
  // the 16-byte piece of token 16 j + (l & 15), chunk 4 c + (l >> 4) of the
  // slice into kr[j KPN + c]; its two 8-byte halves are the A operands of two
  // v_mfma_f32_16x16x32_f16 steps (the contraction runs over the slice's
  // dims in that order, the query operand qB likewise), which leave S^T
  // tiles per token tile j and 64-d chunk group c; the tiles go through LDS
  // back to one token per lane for the scaling and the slices' exchange.
  constexpr bool MSC = DS > 1 || (D == 128 && PVM && !SEQ);
  constexpr int KPN = NP / 4;  // 64-d chunk groups of the slice (its scale groups in affine mode)
  constexpr int ATS = 68;      // LDS row stride (floats) of the transposed score sums

  __shared__ __attribute__((aligned(16))) float w_lds_all[NWV][NR * GW * 64];
  __shared__ __attribute__((aligned(16))) uint16_t sz_lds_all[NWV][2 * 64];
  // windowed: each wave's partial -- row r: o at r (D + 4), then m, l
  constexpr int PST = D + 4;
  __shared__ __attribute__((aligned(16))) float part_lds[SEQ ? SW : 1][SEQ ? NR * PST : 4];
  // the slices' partial scores, two buffers (block parity)
  __shared__ __attribute__((aligned(16))) float sc_lds[DS > 1 ? 2 : 1][DS][DS > 1 ? NR * 64 : 1];
  // MSC, per wave: the per-group score sums [g][row][token] of the block,
  // and at a segment's start the staging of the fp16 query words [row][64]
  __shared__ __attribute__((aligned(16))) float msc_lds[MSC ? NWV : 1][MSC ? GW * NR * ATS : 4];

  const int lane = DS > 1 || SEQ ? (int)(threadIdx.x & 63) : (int)threadIdx.x;
  const int wsl = DS > 1 ? (int)(threadIdx.x >> 6) : 0;  // this wave's d-slice
  const int wid = SEQ ? __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)) : 0;  // wave of the workgroup
  float *const w_lds = w_lds_all[SEQ ? wid : wsl];
  uint16_t *const sz_lds = sz_lds_all[SEQ ? wid : wsl];
  const int p0 = wsl * NP;                             // first K piece of the slice
  const int g0 = MODE == MODE_AFFINE ? wsl * GW : 0;   // first scale group of the slice
  const int rg = DS > 1 ? (int)blockIdx.z : 0;         // row group
  const int r0 = rg * NR;                              // its first query row
  int sbuf = 0;                                        // partial-score buffer of the block
  // blocks of a sequence of (view) length len that this row group reads
  auto nblk = [&](int len) -> int { return DS > 1 ? seq_blocks_rg(a, len, rg) : seq_blocks(a, len); };
  // Every KV head splits its blocks into the same ranges, and workgroups go
  // to the 8 XCDs round-robin by linear id, so with the range index equal to
  // blockIdx.x (the wave count a multiple of 8) range w of every head would
  // land on the same XCD.  Rotating the range by the head sends range w of
  // the 8 heads to 8 different XCDs: the ranges that cost more (sequence
  // ends inside them) no longer pile up on one XCD.
  const int hk = blockIdx.y;
  const int wv = (int)((blockIdx.x + (unsigned)hk) % gridDim.x);
#ifdef KRILL_WAVE_STAMPS
  const unsigned long long st_t0 = __builtin_amdgcn_s_memrealtime();
  unsigned long long st_t1 = 0;
  int st_seg = 0;
#endif
  // This wave's blocks: flat indices [i0, iend) of the concatenated block
  // lists of all sequences.  The T blocks are split evenly over the grid's
  // waves (sized to the resident wave capacity of the GPU; min(W, T) of them
  // take part), wave w taking [ceil(w T / W), ceil((w+1) T / W)), so every
  // wave streams the same bytes whatever the length mix and every SIMD
  // carries the same load.
  // Sequence lengths of the first 64 sequences stay in `lenv` (lane j:
  // sequence c0 + j, c0 = the chunk holding the wave's first sequence).
  const int W = a.waves;
  int c0 = 0, lenv = lane < a.B ? seq_len_view<WIN>(a, lane) : 0;
  int nbv = nblk(lenv);
  int incl = wave_incl_scan(nbv);
  int T = __builtin_amdgcn_readlane(incl, 63);
  for (int cc = 64; cc < a.B; cc += 64) {
    const int bb = cc + lane;
    T += __builtin_amdgcn_readfirstlane(wave_allsum_int(bb < a.B ? nblk(seq_len_view<WIN>(a, bb)) : 0));
  }
  // At most T waves take part, so every participating wave holds at least
  // one block (the merge relies on it: each wave between a sequence's first
  // and last writes that sequence's partial).
  // Windowed (SEQ): the workgroup's sequence blockIdx.x, split evenly over
  // its SW waves; a wave without blocks still leaves an (empty) partial.
  int i0 = 0, iend = 0;
  int b = -1, s = 0;  // sequence holding block i0 and the flat index of its first block
  if constexpr (SEQ) {
    const int bq = (int)blockIdx.x;
    int carry = 0;
    for (c0 = 0; c0 < a.B; c0 += 64) {
      if (c0 > 0) {
        const int bb = c0 + lane;
        lenv = bb < a.B ? seq_len_view<WIN>(a, bb) : 0;
        nbv = nblk(lenv);
        incl = wave_incl_scan(nbv) + carry;
      }
      if (bq < c0 + 64) {
        s = __builtin_amdgcn_readlane(incl - nbv, bq - c0);
        break;
      }
      carry = __builtin_amdgcn_readlane(incl, 63);
    }
    b = bq;
    const int nbq = nblk(__builtin_amdgcn_readlane(lenv, bq - c0));
    i0 = s + (wid * nbq + SW - 1) / SW;
    iend = s + ((wid + 1) * nbq + SW - 1) / SW;
  } else {
  const int Wt = min(W, T);
  if (wv >= Wt) return;
  i0 = (int)(((int64_t)wv * T + Wt - 1) / Wt);
  iend = (int)(((int64_t)(wv + 1) * T + Wt - 1) / Wt);
  {
    int carry = 0;
    for (c0 = 0; c0 < a.B; c0 += 64) {
      if (c0 > 0) {
        const int bb = c0 + lane;
        lenv = bb < a.B ? seq_len_view<WIN>(a, bb) : 0;
        nbv = nblk(lenv);
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
  }
  auto seq_len = [&](int bs) -> int { return bs - c0 < 64 ? __builtin_amdgcn_readlane(lenv, bs - c0) : seq_len_view<WIN>(a, bs); };

  // Decode step with the append fused: the wave that reads a sequence's last
  // block writes the sequence's newest token there (position len - 1; not
  // written when that block lies beyond the blocks read).  The token is
  // quantized and stored while the wave's block loads are in flight, and the
  // wave patches it into its registers when it reaches that block.  The raw
  // rows of the first segment's sequence are loaded alongside the block table.
  constexpr int E = D / 64;
  uint16_t rk[E], rv[E];
  bool own = false;
  if (a.k_new) {  // (every row group patches the token in; row group 0 stores it)
    const int len0 = seq_len(b), nb0 = nblk(len0);
    own = nb0 > 0 && s + nb0 <= iend && ((len0 - 1) >> 6) == nb0 - 1;
    if (own) load_new_rows<D>(a, b, hk, rk, rv);
  }

  // Physical block ids of flat blocks i0 .. iend-1 (at most 64): lane j holds
  // the entry of block i0 + j, read back with v_readlane, so no table load
  // sits between a prefetch and its use (a load there would have to drain the
  // prefetch before its value could move to a scalar register).
  int tab = 0, iend_eff = iend;
  bool tab_ok = false;  // the table entry names a block of the pool
  {
    const int f = i0 + lane;
    int bs = b, ss = s;
    while (bs < a.B && ss < iend) {
      const int nbs = nblk(seq_len(bs));
      if (f < iend && f >= ss && f < ss + nbs) {
        const int phys = a.tables[(int64_t)bs * a.max_blocks + table_offset<WIN>(a, bs) + (f - ss)];
        tab_ok = (unsigned)phys < (unsigned)a.lv.num_blocks;
        tab = tab_ok ? phys : 0;
      }
      ss += nbs;
      ++bs;
    }
    if (ss < iend) iend_eff = ss;  // the last sequence ends inside this range
  }
  const uint64_t tab_okm = __ballot(tab_ok);
  // RoPE with the whole head in one wave: the cos/sin rows of the loaded
  // sequence's query positions (row j: position qlen - Lq + j, Lq <= 8) are
  // copied into LDS by direct loads issued right behind the queries, ahead of
  // the first block's loads, so they land with that block instead of one
  // memory round trip after it; finish_q and the newest token's RoPE read
  // them there.
  constexpr bool RSTAGE = ROPE && DS == 1;
  // (windowed workgroups: one row per wave, the RoPE step being a decode step)
  __shared__ __attribute__((aligned(16))) float rope_lds[RSTAGE ? (SEQ ? SW : 8) * D : 1];
  float *const rope_w = rope_lds + (SEQ && RSTAGE ? wid * D : 0);
  __shared__ __attribute__((aligned(16))) uint8_t newrow_all[NWV][2 * D];
  uint8_t *const newrow = newrow_all[SEQ ? wid : wsl];  // the whole quantized row, per wave
  int patch_i = -1, patch_t = 0;  // flat block holding the segment's newest token, its position
  uint32_t pkm[G], pvm[G];
#pragma unroll
  for (int g = 0; g < G; ++g) pkm[g] = pvm[g] = 0u;
  // the newest token of sequence bs (its rows loaded), last block at flat f
  auto prepare = [&](int bs, int f) {
    const int len2 = seq_len(bs);
    if (!((tab_okm >> (f - i0)) & 1)) return;
    // RoPE turns the row by its absolute position (the window's view of a
    // sequence starts some whole blocks in)
    // (staged: the token's position is the query position of this decode
    // step, row 0 of the LDS copy; the queries of sequence bs are loaded)
    const int rpos = WIN ? len_of(a, bs) - 1 : len2 - 1;
    const float *crow = nullptr;
    if constexpr (ROPE) crow = RSTAGE ? rope_w + (a.Lq - 1) * D : rope_row(a, rpos, D);
    // the compiler does not order LDS reads after the direct loads into LDS
    // (their data lands when vmcnt counts them done): wait for them here
    if constexpr (RSTAGE) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (a.q_dtype == DT_BF16) {
      if constexpr (ROPE) rope_row_lanes<D, DT_BF16>(rk, crow);
      prepare_newest<D, MODE, DT_BF16>(rk, rv, newrow, pkm, pvm);
    } else {
      if constexpr (ROPE) rope_row_lanes<D, DT_F16>(rk, crow);
      prepare_newest<D, MODE, DT_F16>(rk, rv, newrow, pkm, pvm);
    }
    patch_i = f;
    patch_t = (len2 - 1) & 63;
  };
  auto rsrc_of = [&](int i) -> __amdgpu_buffer_rsrc_t {
    const bool ok = i < iend_eff;
    const int phys = __builtin_amdgcn_readlane(tab, ok ? i - i0 : 0);
    return block_rsrc(head_region(a.lv, phys, hk), ok ? a.lv.head_bytes : 0);
  };

  const int pos = ((lane >> 5) << 5) + vpos(lane & 31);        // this lane's token in V order
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};
  const half2_t m1152 = half2_t{(_Float16)-1152.0f, (_Float16)-1152.0f};

  // V^T tiles for the matrix-core P.V: tile dt, MFMA row m holds row
  // d = tile_d(dt, m); lane l loads the 16 storage positions 16 (l >> 4) ..
  // +15 of that row (group l >> 5, half (l >> 4) & 1): for a fixed tile the
  // 16 lanes of a quarter read 16 consecutive 16-byte pieces.
  constexpr int ND = DW / 16;  // the wave's V^T tiles (matrix-core P.V): tiles dt0 .. dt0 + ND - 1 of the row
  const int dt0 = wsl * ND;
  auto tile_d = [](int dt, int m) { return DPL * (16 * (dt / DPL) + m) + dt % DPL; };
  // byte offset of tile gd's 16-byte piece for lane quarter (tg, h), row m
  auto v_tile_off = [](int gd, int tg, int h, int m) {
    return v_offset(D) + tg * 32 * D + (((2 * (gd % DPL) + h) * 64 + 16 * (gd / DPL) + m) << 4);
  };
  // head_dim 512, affine (VRM): the rows of a stored tile span the slice's
  // two scale groups (m < 8, m >= 8), so the wave regroups them: its tile
  // vt = 4 gv + u, row rho, is row 8 gv + 4 (u >> 1) + (rho >> 2) of the
  // slice's stored tile 4 (u & 1) + (rho & 3), i.e. d = DW wsl + 64 gv +
  // 32 (u >> 1) + 8 (rho >> 2) + 4 (u & 1) + (rho & 3): every tile lies in
  // group gv, and the four rows of an output quarter are consecutive d
  constexpr bool VRM = DS > 1 && MODE == MODE_AFFINE;
  static_assert(!VRM || (ND == 8 && GW == 2), "regrouping for two scale groups of 8 tiles");
  auto vr_tile = [](int vt, int rho) { return VRM ? 4 * ((vt % 4) & 1) + (rho & 3) : vt; };
  auto vr_row = [](int vt, int rho) { return VRM ? 8 * (vt / 4) + 4 * ((vt % 4) >> 1) + (rho >> 2) : rho; };
  const int gl = MODE == MODE_AFFINE ? (DPL * lane) / 64 : 0;  // VALU P.V: scale group of this lane's V rows
  constexpr int NV = PVM ? ND : 4 * DPL;  // 16-byte V pieces per lane
  uint4 kr[NP];
  uint4 vr[NV];
  // byte offset of K register p's piece: one token per lane, or (MSC) the
  // MFMA operand order
  auto k_off = [&](int p) -> int {
    return MSC ? k_byte(16 * (p / KPN) + (lane & 15), 16 * (p0 + 4 * (p % KPN) + (lane >> 4)))
               : k_byte(lane, 16 * (p0 + p));
  };
  auto load_k = [&](__amdgpu_buffer_rsrc_t r) {
#pragma unroll
    for (int p = 0; p < NP; ++p) kr[p] = ld_stream16(r, k_off(p));
  };
  auto load_v = [&](__amdgpu_buffer_rsrc_t r) {
    if constexpr (PVM) {
      const int tg = lane >> 5, h = (lane >> 4) & 1, m = lane & 15;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) vr[dt] = ld_stream16(r, v_tile_off(dt0 + vr_tile(dt, m), tg, h, vr_row(dt, m)));
    } else {
      // vr[tg 2 DPL + i]: d = DPL lane + i / 2, half i % 2 of token group tg
#pragma unroll
      for (int tg = 0; tg < 2; ++tg)
#pragma unroll
        for (int i2 = 0; i2 < 2 * DPL; ++i2)
          vr[tg * 2 * DPL + i2] = ld_stream16(r, v_offset(D) + tg * 32 * D + ((i2 * 64 + lane) << 4));
    }
  };
  // this lane's token's (scale, zero) pairs of the slice's groups, K and V
  uint32_t km[GW], vm[GW];
  auto load_meta = [&](__amdgpu_buffer_rsrc_t r, uint32_t (&kmo)[GW], uint32_t (&vmo)[GW]) {
    ld_stream_words<GW>(r, km_offset(D) + (lane * G + g0) * 4, kmo);
    ld_stream_words<GW>(r, vm_offset(D, G) + (lane * G + g0) * 4, vmo);
  };

  // fp16 query pairs: qv[r][c] holds pair 16*c + (lane & 15) of row r, so
  // every 16-lane row carries the whole query (one VGPR per 32 d).  Affine
  // mode also needs the sum of each 64-d group of the fp16 query (pairs
  // 32g .. 32g+31 = columns 2g and 2g+1), reduced inside each 16-lane row.
  uint32_t qv[NR][DW / 32];
  // MSC: lane (n, q4) holds, for chunk group c and half h, the fp16 words
  // 32 c + 8 q4 + 4 h .. +3 of row n (zero for n >= NR)
  half8_t qB[MSC ? KPN : 1][2];
  float qs[NR][GW];
  // per row: the factor its scores take (the softmax scale in log2 units
  // times the query's 2^k; d-slices: 2^k alone, on the slice's part)
  float q_up[NR];
  const bool q_bf16 = a.q_dtype == DT_BF16;
  int qlen = 0;  // length of the sequence whose queries are loaded (RoPE positions)
  int qseq = 0;  // that sequence
  auto load_q = [&](int bq) {  // raw pairs of sequence bq (the slice's dims)
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const int hq = hk * a.R + (r0 + r) % a.R, j = (r0 + r) / a.R;
      const uint32_t *qp = reinterpret_cast<const uint32_t *>(q_row(a, bq, hq, j)) + wsl * (DW / 2);
#pragma unroll
      for (int c = 0; c < DW / 32; ++c) qv[r][c] = qp[16 * c + (lane & 15)];
    }
    if constexpr (ROPE) qlen = WIN ? len_of(a, bq) : seq_len(bq);  // absolute positions
    if constexpr (RSTAGE) {
      const int64_t tb = (int64_t)a.rope_max_pos * D * 4;
      const __amdgpu_buffer_rsrc_t rr =
          block_rsrc(reinterpret_cast<const uint8_t *>(a.rope_cs), (int)(tb < INT32_MAX ? tb : INT32_MAX));
      for (int j = 0; j < (SEQ ? 1 : a.Lq); ++j) {
        const int p = min(max(qlen - a.Lq + j, 0), a.rope_max_pos - 1);  // as rope_row clamps
#pragma unroll
        for (int c = 0; c < D / 64; ++c)
          __builtin_amdgcn_raw_ptr_buffer_load_lds(rr, (lds_void_t *)(rope_w + j * D + 64 * c), 4,
                                                   (p * D + 64 * c + lane) * 4, 0, 0, 0);
      }
    }
    qseq = bq;
  };
  auto finish_q = [&]() {
    if constexpr (ROPE && DS == 1) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // the staged cos/sin rows (see prepare)
      // row r (query position j = r / R, token qlen - Lq + j): pair words
      // 16 c + (lane & 15) of the first half turn with their partners
      // D/64 columns on
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float *crow = rope_w + (r / a.R) * D;  // position qlen - Lq + r / R
#pragma unroll
        for (int c = 0; c < D / 64; ++c) {
          const int d = 2 * (16 * c + (lane & 15));
          const float2 c2 = *reinterpret_cast<const float2 *>(crow + d);
          const float2 s2 = *reinterpret_cast<const float2 *>(crow + D / 2 + d);
          if (q_bf16)
            rope_pair_words<DT_BF16>(qv[r][c], qv[r][c + D / 64], c2, s2);
          else
            rope_pair_words<DT_F16>(qv[r][c], qv[r][c + D / 64], c2, s2);
        }
      }
    } else if constexpr (ROPE) {
      // d-slices: the partner of dim e is e +- D/2, in slice wsl ^ (DS/2);
      // its raw pair words are read here (once per segment) and the pair
      // turns by cos/sin index e mod D/2
      const bool low = wsl < DS / 2;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int hq = hk * a.R + (r0 + r) % a.R, j = (r0 + r) / a.R;
        const uint32_t *pp = reinterpret_cast<const uint32_t *>(q_row(a, qseq, hq, j)) + (wsl ^ (DS / 2)) * (DW / 2);
        const float *crow = rope_row(a, qlen - a.Lq + (r0 + r) / a.R, D);
#pragma unroll
        for (int c = 0; c < DW / 32; ++c) {
          const int i = (wsl % (DS / 2)) * DW + 2 * (16 * c + (lane & 15));
          const float2 c2 = *reinterpret_cast<const float2 *>(crow + i);
          const float2 s2 = *reinterpret_cast<const float2 *>(crow + D / 2 + i);
          const uint32_t part = pp[16 * c + (lane & 15)];
          uint32_t lo = low ? qv[r][c] : part, hi = low ? part : qv[r][c];
          if (q_bf16)
            rope_pair_words<DT_BF16>(lo, hi, c2, s2);
          else
            rope_pair_words<DT_F16>(lo, hi, c2, s2);
          qv[r][c] = low ? lo : hi;
        }
      }
    }
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      // bf16 pairs are widened to fp32 and rounded to fp16 (rows at the
      // fp16 range limit scaled by 2^-k first, q_range_scale); fp16 pairs
      // pass through
      float down = 1.0f, up = 1.0f;
      if (q_bf16) {
        float mx = 0.0f;
#pragma unroll
        for (int c = 0; c < DW / 32; ++c) {
          const uint32_t w = qv[r][c];
          mx = fmaxf(mx, fmaxf(fabsf(__builtin_bit_cast(float, w << 16)),
                               fabsf(__builtin_bit_cast(float, w & 0xffff0000u))));
        }
        down = q_range_scale(uniform_f32(row_allmax(mx)), up);
      }
      q_up[r] = DS > 1 ? up : a.scale_log2 * up;
#pragma unroll
      for (int c = 0; c < DW / 32; ++c) {
        const uint32_t w = qv[r][c];
        const half2_t hb = half2_t{(_Float16)(__builtin_bit_cast(float, w << 16) * down),
                                   (_Float16)(__builtin_bit_cast(float, w & 0xffff0000u) * down)};
        qv[r][c] = q_bf16 ? h2_as_u32(hb) : w;
      }
      if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const half2_t h0 = u32_as_h2(qv[r][2 * g]), h1 = u32_as_h2(qv[r][2 * g + 1]);
          qs[r][g] = uniform_f32(row_allsum(((float)h0.x + (float)h0.y) + ((float)h1.x + (float)h1.y)));
        }
      } else {
#pragma unroll
        for (int g = 0; g < GW; ++g) qs[r][g] = 0.0f;
      }
    }
    if constexpr (MSC) {
      // the query operands, through the wave's LDS (its lanes only)
      uint32_t *const ql = reinterpret_cast<uint32_t *>(msc_lds[SEQ ? wid : wsl]);
      if (lane < 16) {
#pragma unroll
        for (int r = 0; r < NR; ++r)
#pragma unroll
          for (int c = 0; c < DW / 32; ++c) ql[r * 64 + 16 * c + lane] = qv[r][c];
      }
      const int n = lane & 15, q4 = lane >> 4;
#pragma unroll
      for (int c = 0; c < KPN; ++c)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint4 w = uint4{0u, 0u, 0u, 0u};
          if (n < NR) w = *reinterpret_cast<const uint4 *>(ql + n * 64 + 32 * c + 8 * q4 + 4 * h);
          qB[c][h] = __builtin_bit_cast(half8_t, w);
        }
    }
  };

  // Loads of block n+1 are issued in a fixed order inside the loop: K bytes
  // and metadata once block n's K registers are consumed, V bytes once its V
  // registers are; waits on a load never cover a younger prefetch.  The
  // first block's loads (and the first segment's queries, issued ahead of
  // them) are settled before the loop so the loop-head waits follow the
  // steady-state order only.
  load_q(b);
  {
    const __amdgpu_buffer_rsrc_t r0 = rsrc_of(i0);
    load_k(r0);
    load_meta(r0, km, vm);
    load_v(r0);
  }
  if (own) prepare(b, s + nblk(seq_len(b)) - 1);
#pragma unroll
  for (int p = 0; p < NP; ++p) settle(kr[p]);
#pragma unroll
  for (int k = 0; k < NV; ++k) settle(vr[k]);
#pragma unroll
  for (int g = 0; g < GW; ++g) {
    settle(km[g]);
    settle(vm[g]);
  }
  finish_q();
#ifdef KRILL_WAVE_STAMPS
  st_t1 = __builtin_amdgcn_s_memrealtime();
#endif

  int i = i0;
  // Issue priority falls as the wave works through its range (3 in its
  // first quarter .. 0 in its last), so a wave that is ahead yields to the
  // other waves of its SIMD and the SIMD's waves finish together.
  const int nrange = iend_eff - i0;
  const int pq1 = i0 + (nrange + 3) / 4, pq2 = i0 + (nrange + 1) / 2, pq3 = i0 + (3 * nrange + 3) / 4;
  __builtin_amdgcn_s_setprio(3);
  // one pass per sequence segment [max(s, i0), min(s + nb, iend)); the
  // queries of sequence b are ready on entry
  while (true) {
    const int len = seq_len(b);
    const int e = s + nblk(len);
    const int seg_start = i, seg_end = min(e, iend_eff);

    int lim[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) lim[r] = key_limit(a, len, (r0 + r) / a.R);
    int lo[NR], wst = 0;  // sliding window: first key each row sees, first retained key
    if constexpr (WIN) {
      wst = win_view_start(a, b);
#pragma unroll
      for (int r = 0; r < NR; ++r) lo[r] = max(wst, len - a.Lq + (r0 + r) / a.R - a.window + 1);
    }

    // acc[dt]: O^T tile dt, lane l: query row l & 15, d = tile_d(dt, 4 (l >> 4) + j)
    float m_run[NR], l_part[NR], c_part[NR][GW];
    float4_t acc[PVM ? ND : 1];          // matrix-core P.V
    float accv[PVM ? 1 : NR][DPL];       // VALU P.V: row r, d = DPL lane + e
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      m_run[r] = -INFINITY;
      l_part[r] = 0.0f;
#pragma unroll
      for (int g = 0; g < GW; ++g) c_part[r][g] = 0.0f;
    }
#pragma unroll
    for (int dt = 0; dt < (PVM ? ND : 1); ++dt) acc[dt] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < (PVM ? 1 : NR); ++r)
#pragma unroll
      for (int e2 = 0; e2 < DPL; ++e2) accv[r][e2] = 0.0f;

  for (; i < seg_end; ++i) {
    if (i == pq1) __builtin_amdgcn_s_setprio(2);
    if (i == pq2) __builtin_amdgcn_s_setprio(1);
    if (i == pq3) __builtin_amdgcn_s_setprio(0);
    const int tbase = (i - s) << 6;
    const __amdgpu_buffer_rsrc_t nrs = rsrc_of(i + 1);
    if (i == patch_i) {
      // the block holding the segment's newest token: its K row and both
      // (scale, zero) words go to lane patch_t (MSC: its chunk 4 c + q4 to
      // lane (patch_t & 15) + 16 q4, register (patch_t / 16) KPN + c)
      if constexpr (MSC) {
        const bool mine = (lane & 15) == (patch_t & 15);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int c = 0; c < KPN; ++c) {
            const uint4 x = *reinterpret_cast<const uint4 *>(newrow + 16 * (p0 + 4 * c + (lane >> 4)));
            if (mine && (patch_t >> 4) == j) kr[j * KPN + c] = x;
          }
      } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
          const uint4 x = *reinterpret_cast<const uint4 *>(newrow + 16 * (p0 + p));
          if (lane == patch_t) kr[p] = x;
        }
      }
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        if (lane == patch_t) {
          km[g] = pkm[g0 + g];
          vm[g] = pvm[g0 + g];
        }
      }
    }

    // ---- scores: this lane's token against every query row; the query
    // pair of each dot comes from lane (pair & 15) of the lane's 16-lane row
    // through the DPP broadcast of v_dot2c.
    float accg[NR][GW];
    if constexpr (MSC) {
      float4_t sacc[4][GW];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int g = 0; g < GW; ++g) sacc[j][g] = float4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        half2_t ks2 = m1024, kz2 = m1024;
        if constexpr (MODE == MODE_REF) {
          // the (scale, zero) word of this lane's token of tile j
          const uint32_t kmj = (uint32_t)__shfl((int)km[0], 16 * j + (lane & 15));
          const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(kmj & 0xffffu));
          const _Float16 z = __builtin_bit_cast(_Float16, (uint16_t)(kmj >> 16));
          ks2 = half2_t{s, s};
          kz2 = half2_t{z, z};
        }
        half8_t A[KPN][2];
#pragma unroll
        for (int c = 0; c < KPN; ++c) {
          const int p = j * KPN + c;
          const uint32_t w4[4] = {kr[p].x, kr[p].y, kr[p].z, kr[p].w};
          half2_t kp[8];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kp[2 * e] = bytes01_plus1024(w4[e]);
            kp[2 * e + 1] = bytes23_plus1024(w4[e]);
          }
          if constexpr (MODE == MODE_REF) {
#pragma unroll
            for (int e = 0; e < 8; ++e) kp[e] = (kp[e] + m1024) * ks2 + kz2;
          } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) kp[e] = kp[e] + m1152;  // u - 128, exact
          }
          // the piece is converted: its register takes the next block's piece
          kr[p] = ld_stream16(nrs, k_off(p));
          A[c][0] = half8_t{kp[0][0], kp[0][1], kp[1][0], kp[1][1], kp[2][0], kp[2][1], kp[3][0], kp[3][1]};
          A[c][1] = half8_t{kp[4][0], kp[4][1], kp[5][0], kp[5][1], kp[6][0], kp[6][1], kp[7][0], kp[7][1]};
        }
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int c = 0; c < KPN; ++c) {
            const int g = MODE == MODE_AFFINE ? c : 0;
            sacc[j][g] = mfma16x16x32(A[c][h], qB[c][h], sacc[j][g]);
          }
      }
      // lane (n, q4) holds the sums of tokens 16 j + 4 q4 .. +3 for row n:
      // back to one token per lane through the wave's LDS
      float *const ml = msc_lds[SEQ ? wid : wsl];
      const int n = lane & 15, q4 = lane >> 4;
      if (n < NR) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int g = 0; g < GW; ++g)
            *reinterpret_cast<float4_t *>(ml + (g * NR + n) * ATS + 16 * j + 4 * q4) = sacc[j][g];
      }
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int g = 0; g < GW; ++g) accg[r][g] = ml[(g * NR + r) * ATS + lane];
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r)
#pragma unroll
        for (int g = 0; g < GW; ++g) accg[r][g] = 0.0f;
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
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) kp[i] = kp[i] + m1152;  // u - 128, exact
        }
        // the piece is converted: its register takes the next block's piece
        if constexpr (!LOAD_TOGETHER) kr[p] = ld_stream16(nrs, k_byte(lane, 16 * (p0 + p)));
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
    }
    // The K registers are consumed: the next block's K bytes and metadata
    // are fetched now, in flight through the softmax and P.V.
    uint32_t km_next[GW], vm_next[GW];
    if constexpr (!LOAD_TOGETHER) load_meta(nrs, km_next, vm_next);

    float s[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      float v;
      if constexpr (MODE == MODE_AFFINE) {
        v = 0.0f;
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const float kss = f16_bits_to_f32((uint16_t)(km[g] & 0xffffu));
          const float kzz = f16_bits_to_f32((uint16_t)(km[g] >> 16));
          v += kss * accg[r][g] + (kzz + 128.0f * kss) * qs[r][g];
        }
      } else {
        v = accg[r][0];
      }
      if constexpr (DS > 1) {
        sc_lds[sbuf][wsl][r * 64 + lane] = v * q_up[r];  // this slice's part of the score
      } else {
        bool seen = tbase + lane < lim[r];
        if constexpr (WIN) seen = seen && tbase + lane >= lo[r];
        s[r] = seen ? v * q_up[r] : -INFINITY;
      }
    }
    if constexpr (DS > 1) {
      // every slice's part in: the whole score, summed in slice order (the
      // same sum in every wave)
      __syncthreads();
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        float v = sc_lds[sbuf][0][r * 64 + lane];
#pragma unroll
        for (int w = 1; w < DS; ++w) v += sc_lds[sbuf][w][r * 64 + lane];
        bool seen = tbase + lane < lim[r];
        if constexpr (WIN) seen = seen && tbase + lane >= lo[r];
        s[r] = seen ? v * a.scale_log2 : -INFINITY;
      }
      sbuf ^= 1;
    }

    // ---- online softmax with a lazily raised running max
    bool raise = i == seg_start;
    if (!raise) {
      bool over = false;
#pragma unroll
      for (int r = 0; r < NR; ++r) over |= s[r] > m_run[r] + 8.0f;
      raise = __any(over);
    }
    if (raise) {
      float aln = 1.0f;  // the factor of this lane's accumulator row
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float mb = wave_allmax(s[r]);
        const float mn = fmaxf(m_run[r], mb);
        const float al = m_run[r] == -INFINITY ? 0.0f : fast_exp2(m_run[r] - mn);
        m_run[r] = uniform_f32(mn);
        l_part[r] *= al;
#pragma unroll
        for (int g = 0; g < GW; ++g) c_part[r][g] *= al;
        aln = (lane & 15) == r ? al : aln;
        if constexpr (!PVM) {
#pragma unroll
          for (int e2 = 0; e2 < DPL; ++e2) accv[r][e2] *= al;
        }
      }
      if constexpr (PVM) {
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) acc[dt] *= aln;
      }
    }
    float pr[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      pr[r] = fast_exp2(s[r] - (m_run[r] == -INFINITY ? 0.0f : m_run[r]));
      l_part[r] += pr[r];
    }

    // ---- weights to LDS in V storage order
    bool valid = tbase + lane < len;
    if constexpr (WIN) valid = valid && tbase + lane >= wst;  // rows below the window are not data
    // The weights stay binary32 (p * s_v rounded once): an fp16 weight
    // would carry a relative error of 2^-11 into p * s_v * u, up to 2^-11 of
    // the group's value range in the output when a few keys hold the weight.
    if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
      for (int g = 0; g < GW; ++g) {
        const float vsf = valid ? f16_bits_to_f32((uint16_t)(vm[g] & 0xffffu)) : 0.0f;
        const float vzf = valid ? f16_bits_to_f32((uint16_t)(vm[g] >> 16)) : 0.0f;
#pragma unroll
        for (int r = 0; r < NR; ++r) {
          w_lds[(r * GW + g) * 64 + pos] = pr[r] * vsf;
          // the zero point, plus on the matrix cores the 128 taken off the V
          // bytes: p (z + 128 s); the VALU takes the bytes as they are: p z
          c_part[r][g] = fmaf(pr[r], PVM ? fmaf(128.0f, vsf, vzf) : vzf, c_part[r][g]);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < NR; ++r) w_lds[r * 64 + pos] = pr[r];
      sz_lds[pos] = valid ? (uint16_t)(vm[0] & 0xffffu) : (uint16_t)0;
      sz_lds[64 + pos] = valid ? (uint16_t)(vm[0] >> 16) : (uint16_t)0;
    }
    // (each wave has its own weights; a workgroup barrier here would pair up
    // with other waves' barriers once the waves of a windowed workgroup,
    // whose block counts differ, leave the loop at different times)
    if constexpr (DS > 1 || SEQ)
      wave_lds_sync();
    else
      __syncthreads();
    if constexpr (PVM) {
    if (i == patch_i) {
      // the newest token's V bytes: storage position p of group tg is byte
      // p % 16 of every tile register of the lanes of quarter 2 tg + p / 16
      const int tg = patch_t >> 5, p = vpos(patch_t & 31), bp = p & 15;
      const int sh = 8 * (bp & 3);
      const uint32_t keep = ~(0xffu << sh);
      const bool mine = (lane >> 4) == 2 * tg + (p >> 4);
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) {
        const uint32_t nv = (uint32_t)newrow[D + tile_d(dt0 + vr_tile(dt, lane & 15), vr_row(dt, lane & 15))] << sh;
        uint4 &x = vr[dt];
        if (mine) {
          if ((bp >> 2) == 0) x.x = (x.x & keep) | nv;
          else if ((bp >> 2) == 1) x.y = (x.y & keep) | nv;
          else if ((bp >> 2) == 2) x.z = (x.z & keep) | nv;
          else x.w = (x.w & keep) | nv;
        }
      }
    }

    } else {
    if (i == patch_i) {
      // the newest token's V bytes: position p of group tg, byte p % 16 of the
      // piece (2 (d % DPL) + p / 16) of every lane's d rows
      const int tg = patch_t >> 5, p = vpos(patch_t & 31), hi = p >> 4, bp = p & 15;
      const int sh = 8 * (bp & 3);
      const uint32_t keep = ~(0xffu << sh);
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const uint32_t nv = (uint32_t)newrow[D + DPL * lane + e] << sh;
#pragma unroll
        for (int tgi = 0; tgi < 2; ++tgi)
#pragma unroll
          for (int h2 = 0; h2 < 2; ++h2)
            if (tgi == tg && h2 == hi) {
              uint4 &x = vr[tgi * 2 * DPL + 2 * e + h2];
              if ((bp >> 2) == 0) x.x = (x.x & keep) | nv;
              else if ((bp >> 2) == 1) x.y = (x.y & keep) | nv;
              else if ((bp >> 2) == 2) x.z = (x.z & keep) | nv;
              else x.w = (x.w & keep) | nv;
            }
      }
    }

    }
    if constexpr (PVM) {
    // ---- P.V on the matrix cores: O^T += V^T . P^T per 16-row d tile, two
    // 32-position sub-steps per block.  Sub-step sh of lane quarter q covers
    // positions 16 q + 8 sh .. +7: A = those bytes of the lane's tile row
    // (affine: exact fp16 u - 128; row mode: dequantized as the reference
    // does, f16(f16(u * s) + z)), B = the same positions' weights of query
    // row l & 15 (rows beyond NR repeat the last one; their outputs are never
    // read), each binary32 weight as an fp16 high part and the fp16 rounding
    // of its remainder (about 2^-22 relative left), two MFMAs per tile.
    if constexpr (VRM) {
      // head_dim 512: each regrouped tile lies in one scale group, whose
      // weights it takes in B
      const int nb = (lane & 15) < NR ? (lane & 15) : NR - 1, q = lane >> 4;
#pragma unroll
      for (int sh = 0; sh < 2; ++sh) {
        half8_t bh[2], bl[2];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
          const float *wp = w_lds + (nb * GW + g) * 64 + 16 * q + 8 * sh;
          split_hi_lo(*reinterpret_cast<const float4 *>(wp), *reinterpret_cast<const float4 *>(wp + 4), bh[g], bl[g]);
        }
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
          const uint4 v = vr[dt];
          const half8_t av = bytes8_centred(sh ? uint2{v.z, v.w} : uint2{v.x, v.y});
          const int g = dt / (ND / GW);
          acc[dt] = mfma16x16x32(av, bh[g], acc[dt]);
          acc[dt] = mfma16x16x32(av, bl[g], acc[dt]);
        }
      }
      // the tiles are consumed: their registers take the next block's
      const int tg = lane >> 5, h = (lane >> 4) & 1, m = lane & 15;
#pragma unroll
      for (int dt = 0; dt < ND; ++dt) vr[dt] = ld_stream16(nrs, v_tile_off(dt0 + vr_tile(dt, m), tg, h, vr_row(dt, m)));
    } else {
      const int nb = (lane & 15) < NR ? (lane & 15) : NR - 1, q = lane >> 4;
#pragma unroll
      for (int g = 0; g < GW; ++g) {
#pragma unroll
        for (int sh = 0; sh < 2; ++sh) {
          const float *wp = w_lds + (nb * GW + g) * 64 + 16 * q + 8 * sh;
          half8_t bh, bl;
          split_hi_lo(*reinterpret_cast<const float4 *>(wp), *reinterpret_cast<const float4 *>(wp + 4), bh, bl);
          uint4 sc = {0u, 0u, 0u, 0u}, zc = {0u, 0u, 0u, 0u};
          if constexpr (MODE == MODE_REF) {
            sc = *reinterpret_cast<const uint4 *>(sz_lds + 16 * q + 8 * sh);
            zc = *reinterpret_cast<const uint4 *>(sz_lds + 64 + 16 * q + 8 * sh);
          }
#pragma unroll
          for (int t = 0; t < ND / GW; ++t) {
            const int dt = g * (ND / GW) + t;
            const uint4 v = vr[dt];
            const uint2 w8 = sh ? uint2{v.z, v.w} : uint2{v.x, v.y};
            half8_t av;
            if constexpr (MODE == MODE_AFFINE)
              av = bytes8_centred(w8);
            else
              av = bytes8_dequant_ref(w8, sc, zc);
            acc[dt] = mfma16x16x32(av, bh, acc[dt]);
            acc[dt] = mfma16x16x32(av, bl, acc[dt]);
          }
        }
        // the group's tiles are consumed: their registers take the next block's
        {
          const int tg = lane >> 5, h = (lane >> 4) & 1, m = lane & 15;
#pragma unroll
          for (int t = 0; t < ND / GW; ++t) {
            const int dt = g * (ND / GW) + t;
            vr[dt] = ld_stream16(nrs, v_tile_off(dt0 + dt, tg, h, m));
          }
        }
      }
    }
    } else {
    // ---- P.V: lane owns V^T rows d = DPL*lane .. +DPL.  Steps of 4 tokens
    // (one V word per row d): affine mode turns the 4 bytes into exact
    // binary32 values u (v_cvt_f32_ubyte) and accumulates w * u with fp32
    // FMAs, the bias term sum p * z coming per (row, group) at the end; row
    // mode dequantizes as the reference does, f16(f16(u * s) + z), and
    // accumulates p * v.  The 4 weights of one (step, row) are one 16-byte
    // LDS read, issued two steps ahead of their use.
    constexpr int NSTEP = 16 * NR;  // (tg, chunk, half, row) steps
    auto wread = [&](int k) -> float4 {
      const int r = k % NR, c = k / NR;  // c = 2 * (tg * 4 + chunk) + half: positions 4c .. 4c + 3
      return *reinterpret_cast<const float4 *>(w_lds + (r * G + gl) * 64 + 4 * c);
    };
    float4 wq0 = wread(0), wq1 = wread(1 < NSTEP ? 1 : 0);
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const int tg = c >> 3, ch = (c >> 1) & 3, hf = c & 1;
      float vf[DPL][4];
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        // conversion of this step waits for the previous step's FMAs
        if (c > 0) order_after(vr[tg * 2 * DPL + 2 * e + (ch >> 1)], accv[NR - 1][DPL - 1]);
        const uint4 w = vr[tg * 2 * DPL + 2 * e + (ch >> 1)];
        const uint32_t wd = (ch & 1) ? (hf ? w.w : w.z) : (hf ? w.y : w.x);
        if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
          for (int i = 0; i < 4; ++i) vf[e][i] = (float)((wd >> (8 * i)) & 0xffu);
        } else {
          const half2_t lo = bytes01_plus1024(wd), hi = bytes23_plus1024(wd);
          const uint2 sp2 = *reinterpret_cast<const uint2 *>(sz_lds + 4 * c);
          const uint2 zp2 = *reinterpret_cast<const uint2 *>(sz_lds + 64 + 4 * c);
          const half2_t v0 = (lo + m1024) * u32_as_h2(sp2.x) + u32_as_h2(zp2.x);
          const half2_t v1 = (hi + m1024) * u32_as_h2(sp2.y) + u32_as_h2(zp2.y);
          vf[e][0] = (float)v0.x;
          vf[e][1] = (float)v0.y;
          vf[e][2] = (float)v1.x;
          vf[e][3] = (float)v1.y;
        }
      }
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int k = c * NR + r;
        const float4 wc = wq0;
        asm volatile("" ::: "memory");
        wq0 = wq1;
        if (k + 2 < NSTEP) wq1 = wread(k + 2);
        const float ww[4] = {wc.x, wc.y, wc.z, wc.w};
#pragma unroll
        for (int e = 0; e < DPL; ++e)
#pragma unroll
          for (int i = 0; i < 4; ++i) accv[r][e] = __builtin_fmaf(ww[i], vf[e][i], accv[r][e]);
      }
    }
    }
    // The V registers are free: the next block's V bytes (with three waves
    // per SIMD on the VALU path, its K bytes and metadata too, one pass over
    // the region).  Unconditional on purpose (after the wave's last block the
    // resource is empty and the loads return zeros without a memory access):
    // a conditional load would keep the consumed registers alive through the
    // loop header.
    if constexpr (LOAD_TOGETHER) load_k(nrs);
    if constexpr (!PVM) load_v(nrs);
    if constexpr (LOAD_TOGETHER) load_meta(nrs, km_next, vm_next);
#pragma unroll
    for (int g = 0; g < GW; ++g) {
      km[g] = km_next[g];
      vm[g] = vm_next[g];
    }
    if constexpr (DS > 1 || SEQ)
      wave_lds_sync();
    else
      __syncthreads();
  }

    // the segment's newest token goes to the pool with the segment's output
    // (the whole row, by the first slice's wave of row group 0; the other
    // row groups read the token from their registers, never from memory)
    if (patch_i >= 0 && wsl == 0 && rg == 0)
      store_newest<D, MODE>(a, hk, __builtin_amdgcn_readlane(tab, patch_i - i0), patch_t, newrow, pkm, pvm);

    if constexpr (PVM) {
    // ---- end of the segment: the whole sequence in this wave -> output;
    // otherwise a partial in slot hk * (waves + B) + wave + b.  Lane l holds
    // query row n = l & 15 (rows n >= NR are padding).
    const int n = lane & 15, q4 = 4 * (lane >> 4);
    float lsum_n = 0.0f, m_n = 0.0f, cg[GW];
#pragma unroll
    for (int g = 0; g < GW; ++g) cg[g] = 0.0f;
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      const float ls = uniform_f32(wave_allsum(l_part[r]));
      lsum_n = n == r ? ls : lsum_n;
      m_n = n == r ? m_run[r] : m_n;
      if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const float c = wave_allsum(c_part[r][g]);
          cg[g] = n == r ? c : cg[g];
        }
      }
    }
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) acc[dt] += cg[dt / (ND / GW)];
    // The lane's values of tiles DPL k .. DPL k + DPL - 1 form one run of
    // 4 DPL consecutive d: d = DPL (16 k + q4 + j) + e for j < 4, e < DPL
    // (k counted over the whole row: the slice's tiles start at dt0).
    if (n < NR) {
      const bool whole = !SEQ && !a.partial_only && s >= i0 && e <= iend;
      const float mul = !whole ? 1.0f : lsum_n > 0.0f ? 1.0f / lsum_n : 0.0f;
      const int64_t hslot = DS > 1 ? (int64_t)hk * a.row_groups + rg : (int64_t)hk;
      const int64_t pi = (hslot * (a.waves + a.B) + wv + b) * NR + n;
      const int64_t ob = whole ? out_row_base(a, b, hk, r0 + n, D) : SEQ ? (int64_t)n * PST : pi * D;
      if constexpr (VRM) {
        // regrouped tiles: d = DW wsl + 64 gv + 32 uh + 8 (lane >> 4) + 4 ul + j
        // for tile 4 gv + 2 uh + ul, element j -- four runs of 8
#pragma unroll
        for (int gv = 0; gv < 2; ++gv)
#pragma unroll
          for (int uh = 0; uh < 2; ++uh) {
            float run[8];
#pragma unroll
            for (int ul = 0; ul < 2; ++ul)
#pragma unroll
              for (int j2 = 0; j2 < 4; ++j2) run[4 * ul + j2] = acc[4 * gv + 2 * uh + ul][j2] * mul;
            store_run<8>(whole ? a.out : (void *)a.ws_o, ob + DW * wsl + 64 * gv + 32 * uh + 2 * q4, run,
                         whole ? a.out_dtype : DT_F32);
          }
      } else {
#pragma unroll
        for (int k = 0; k < ND / DPL; ++k) {
          float run[4 * DPL];
#pragma unroll
          for (int j2 = 0; j2 < 4; ++j2)
#pragma unroll
            for (int e2 = 0; e2 < DPL; ++e2) run[DPL * j2 + e2] = acc[DPL * k + e2][j2] * mul;
          store_run<4 * DPL>(SEQ ? (void *)part_lds[wid] : whole ? a.out : (void *)a.ws_o,
                             ob + DPL * (16 * (dt0 / DPL + k) + q4), run, whole ? a.out_dtype : DT_F32);
        }
      }
      if constexpr (SEQ) {
        if (lane < 16) {
          part_lds[wid][n * PST + D] = m_n;
          part_lds[wid][n * PST + D + 1] = lsum_n;
        }
      } else if (!whole && lane < 16 && wsl == 0) {
        reinterpret_cast<float2 *>(a.ws_ml)[pi] = float2{m_n, lsum_n};
      }
    }
    } else {
    // ---- end of the segment: the whole sequence in this wave -> output;
    // otherwise a partial in slot hk * (waves + B) + wave + b
    float lsum[NR];
#pragma unroll
    for (int r = 0; r < NR; ++r) {
      lsum[r] = uniform_f32(wave_allsum(l_part[r]));
      float cg = 0.0f;
      if constexpr (MODE == MODE_AFFINE) {
#pragma unroll
        for (int g = 0; g < GW; ++g) {
          const float c = wave_allsum(c_part[r][g]);
          cg = g == gl ? c : cg;
        }
      }
#pragma unroll
      for (int e2 = 0; e2 < DPL; ++e2) accv[r][e2] += cg;
    }
    if constexpr (SEQ) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
#pragma unroll
        for (int e2 = 0; e2 < DPL; ++e2) part_lds[wid][r * PST + DPL * lane + e2] = accv[r][e2];
        if (lane == 0) {
          part_lds[wid][r * PST + D] = m_run[r];
          part_lds[wid][r * PST + D + 1] = lsum[r];
        }
      }
    } else if (!a.partial_only && s >= i0 && e <= iend) {
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const float inv = lsum[r] > 0.0f ? 1.0f / lsum[r] : 0.0f;
        const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
        for (int e2 = 0; e2 < DPL; ++e2) store_out(a.out, ob + DPL * lane + e2, accv[r][e2] * inv, a.out_dtype);
      }
    } else {
      const int64_t slot = (int64_t)hk * (a.waves + a.B) + wv + b;
#pragma unroll
      for (int r = 0; r < NR; ++r) {
        const int64_t pi = slot * NR + r;
#pragma unroll
        for (int e2 = 0; e2 < DPL; ++e2) a.ws_o[pi * D + DPL * lane + e2] = accv[r][e2];
        if (lane == 0) reinterpret_cast<float2 *>(a.ws_ml)[pi] = float2{m_run[r], lsum[r]};
      }
    }
    }
#ifdef KRILL_WAVE_STAMPS
    ++st_seg;
#endif
    if (i >= iend_eff) break;
    // next sequence with blocks (empty ones get zeros from the merge)
    ++b;
    s = e;
    while (b < a.B && nblk(seq_len(b)) == 0) ++b;
    if (b >= a.B) break;
    load_q(b);
    patch_i = -1;
    if (a.k_new) {
      const int len2 = seq_len(b), nb2 = nblk(len2);
      if (s + nb2 <= iend && ((len2 - 1) >> 6) == nb2 - 1) {
        load_new_rows<D>(a, b, hk, rk, rv);
        prepare(b, s + nb2 - 1);
      }
    }
    finish_q();
  }
  if constexpr (SEQ) {
    // Every wave's partial of the sequence is in LDS: wave w combines rows
    // w, w + SW, ... (the softmax merge of k_attn_merge_flat over the SW
    // partials in wave order; a wave without blocks left m = -inf, l = 0)
    // and writes them out.
    __syncthreads();
    for (int r = wid; r < NR; r += SW) {
      const float mk = lane < SW ? part_lds[lane][r * PST + D] : -INFINITY;
      const float lk = lane < SW ? part_lds[lane][r * PST + D + 1] : 0.0f;
      const float M = uniform_f32(wave_allmax(mk));
      const float wk = lane < SW && mk != -INFINITY ? fast_exp2(mk - M) : 0.0f;
      const float L = uniform_f32(wave_allsum(wk * lk));
      const float inv = (M == -INFINITY || !(L > 0.0f)) ? 0.0f : 1.0f / L;
      const int64_t ob = out_row_base(a, b, hk, r, D);
#pragma unroll
      for (int e2 = 0; e2 < DPL; ++e2) {
        const int d = lane + 64 * e2;
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < SW; ++k) acc += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wk), k)) * part_lds[k][r * PST + d];
        store_out(a.out, ob + d, acc * inv, a.out_dtype);
      }
    }
  }
#ifdef KRILL_WAVE_STAMPS
  {
    const unsigned long long t2 = __builtin_amdgcn_s_memrealtime();
    const unsigned hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);    // HW_REG_HW_ID
    const unsigned xcc = __builtin_amdgcn_s_getreg((31 << 11) | 20);  // HW_REG_XCC_ID
    const int64_t idx = (((int64_t)blockIdx.z * gridDim.y + blockIdx.y) * gridDim.x + blockIdx.x) * (SEQ ? SW : 1) + wid;
    if (lane == 0 && wsl == 0 && idx < kStampWaves) {
      unsigned long long *o = g_wave_stamps + idx * 6;
      o[0] = st_t0;
      o[1] = st_t1;
      o[2] = t2;
      o[3] = 0;
      o[4] = (unsigned long long)hw | ((unsigned long long)xcc << 32);
      o[5] = (unsigned long long)(unsigned)(iend_eff - i0) | ((unsigned long long)(unsigned)st_seg << 32);
    }
  }
#endif
}

template <int D, int MODE, int NR>
static hipError_t launch_one(const AttnArgs &args, int B, dim3 grid, hipStream_t st) {
  const dim3 block(64 * d_slices<D>());
  // windowed, whole head per wave: one workgroup of seq_waves per (sequence,
  // KV head), each wave at most 64 of the sequence's blocks
  auto seq_launch = [&](auto var) -> bool {
    constexpr int SW = seq_waves<D, NR, MODE, decltype(var)::value>();
    if constexpr (SW > 0) {
      if (args.nb_cap > 64 * SW) return false;
      k_attn_valu<D, NR, MODE, decltype(var)::value><<<dim3((unsigned)B, grid.y, 1), dim3(64 * SW), 0, st>>>(args);
    } else {
      k_attn_valu<D, NR, MODE, decltype(var)::value><<<grid, block, 0, st>>>(args);
    }
    return true;
  };
  if (args.rope_cs && args.window > 0) {
    // sliding-window layers with RoPE: head_dim <= 256
    if constexpr (D <= 256) {
      if (!seq_launch(std::integral_constant<int, 3>{})) return hipErrorInvalidValue;
    } else {
      return hipErrorInvalidValue;
    }
  } else if (args.rope_cs) {
    k_attn_valu<D, NR, MODE, 1><<<grid, block, 0, st>>>(args);
  } else if (args.window > 0) {
    if (!seq_launch(std::integral_constant<int, 2>{})) return hipErrorInvalidValue;
  } else {
    k_attn_valu<D, NR, MODE, 0><<<grid, block, 0, st>>>(args);
  }
  return hipSuccess;
}

template <int D, int MODE>
static hipError_t launch_valu_nr(const AttnArgs &args, int NR, int B, dim3 grid, hipStream_t st) {
  hipError_t e;
  switch (NR) {
    case 1: e = launch_one<D, MODE, 1>(args, B, grid, st); break;
    case 2: e = launch_one<D, MODE, 2>(args, B, grid, st); break;
    case 3: e = launch_one<D, MODE, 3>(args, B, grid, st); break;
    case 4: e = launch_one<D, MODE, 4>(args, B, grid, st); break;
    case 5: e = launch_one<D, MODE, 5>(args, B, grid, st); break;
    case 6: e = launch_one<D, MODE, 6>(args, B, grid, st); break;
    case 7: e = launch_one<D, MODE, 7>(args, B, grid, st); break;
    case 8: e = launch_one<D, MODE, 8>(args, B, grid, st); break;
    default: return hipErrorInvalidValue;
  }
  if (e != hipSuccess) return e;
  return hipGetLastError();
}

template <int D, int MODE>
static int32_t occupancy_nr(int NR) {
  int n = 0;
  hipError_t e = hipErrorInvalidValue;
  switch (NR) {
#define KRILL_OCC(N)                                                                                        \
  case N:                                                                                                   \
    e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, reinterpret_cast<const void *>(&k_attn_valu<D, N, MODE, 0>), \
                                                     64 * d_slices<D>(), 0);                                \
    if (e != hipSuccess || n <= 0)                                                                          \
      n = 4 * valu_waves_per_simd<D, N>();                                                                  \
    else                                                                                                    \
      n *= d_slices<D>();                                                                                   \
    break;
    KRILL_OCC(1) KRILL_OCC(2) KRILL_OCC(3) KRILL_OCC(4) KRILL_OCC(5) KRILL_OCC(6) KRILL_OCC(7) KRILL_OCC(8)
#undef KRILL_OCC
    default: n = 8;
  }
  if (e != hipSuccess) (void)hipGetLastError();
  return n;
}

// Resident waves per CU (for head_dim 512: workgroups x 4 waves).
int32_t valu_waves_per_cu(const PoolGeometry &g, int32_t NR) {
  const int dsel = g.D == 64 ? 0 : g.D == 128 ? 1 : g.D == 256 ? 2 : 3;
  if (NR < 1 || NR > 8) return 8;
  if (g.num_cus <= 0) {  // host-only pool: the design point
    static const int est[4][9] = {{0, 12, 12, 12, 12, 12, 12, 12, 12},
                                  {0, 12, 12, 12, 12, 12, 8, 8, 8},
                                  {0, 8, 8, 8, 8, 8, 8, 8, 8},
                                  {0, 8, 8, 8, 8, 8, 8, 8, 8}};
    return est[dsel][NR];
  }
  static int cache[2][4][9] = {};  // [mode][D][NR], filled on first use per process
  int &c = cache[g.mode == MODE_AFFINE][dsel][NR];
  if (c == 0) {
    int n = 8;
    if (g.D == 64) n = g.mode == MODE_REF ? occupancy_nr<64, MODE_REF>(NR) : occupancy_nr<64, MODE_AFFINE>(NR);
    else if (g.D == 128) n = g.mode == MODE_REF ? occupancy_nr<128, MODE_REF>(NR) : occupancy_nr<128, MODE_AFFINE>(NR);
    else if (g.D == 256) n = g.mode == MODE_REF ? occupancy_nr<256, MODE_REF>(NR) : occupancy_nr<256, MODE_AFFINE>(NR);
    else n = g.mode == MODE_REF ? occupancy_nr<512, MODE_REF>(NR) : occupancy_nr<512, MODE_AFFINE>(NR);
    c = n;
  }
  return c;
}

// Longest windowed view (tokens) the decode kernel's per-sequence workgroups
// take at head_dim <= 256 (64 blocks per wave); 0 where the flat split runs.
template <int D, int MODE>
static int32_t window_limit_nr(int NR, bool rope) {
  switch (NR) {
#define KRILL_WL(N)                                                                        \
  case N:                                                                                  \
    return 64 * (rope ? seq_max_blocks<D, N, MODE, 3>() : seq_max_blocks<D, N, MODE, 2>());
    KRILL_WL(1) KRILL_WL(2) KRILL_WL(3) KRILL_WL(4) KRILL_WL(5) KRILL_WL(6) KRILL_WL(7) KRILL_WL(8)
#undef KRILL_WL
    default: return 0;
  }
}
int32_t valu_window_limit(const PoolGeometry &g, int32_t NR, bool rope) {
  const bool aff = g.mode == MODE_AFFINE;
  switch (g.D) {
    case 64: return aff ? window_limit_nr<64, MODE_AFFINE>(NR, rope) : window_limit_nr<64, MODE_REF>(NR, rope);
    case 128: return aff ? window_limit_nr<128, MODE_AFFINE>(NR, rope) : window_limit_nr<128, MODE_REF>(NR, rope);
    case 256: return aff ? window_limit_nr<256, MODE_AFFINE>(NR, rope) : window_limit_nr<256, MODE_REF>(NR, rope);
    default: return 0;
  }
}

// Copies the stamps of the last decode launch (diagnostic build), up to
// max_waves rows of 6 words; returns the rows copied, or -1 if this build
// has no stamps.
int32_t wave_stamps(unsigned long long *host, int32_t max_waves) {
#ifdef KRILL_WAVE_STAMPS
  const int32_t n = max_waves < kStampWaves ? max_waves : kStampWaves;
  if (hipMemcpyFromSymbol(host, HIP_SYMBOL(g_wave_stamps), (size_t)n * 6 * 8, 0, hipMemcpyDeviceToHost) != hipSuccess)
    return -2;
  return n;
#else
  (void)host;
  (void)max_waves;
  return -1;
#endif
}

hipError_t launch_attn_valu(const PoolGeometry &g, int32_t layer, const AttnLaunch &a, const AttnPlan &p,
                            hipStream_t st) {
  // one VGPR of block-table entries per wave
  if (p.waves < 1 || (int64_t)p.waves * 64 < (int64_t)a.B * p.nb_cap) return hipErrorInvalidValue;
  // rows beyond 8 per KV head run in row groups on head_dim 512 only
  if (p.row_groups < 1 || p.row_groups * p.rows_per_group != p.NR || (g.D <= 256 && p.row_groups != 1))
    return hipErrorInvalidValue;
  const AttnArgs args = make_attn_args(g, layer, a, p);
  const dim3 grid((unsigned)p.waves, (unsigned)g.Hkv, (unsigned)p.row_groups);
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
    case 512:
      return g.mode == MODE_REF ? launch_valu_nr<512, MODE_REF>(args, p.rows_per_group, a.B, grid, st)
                                : launch_valu_nr<512, MODE_AFFINE>(args, p.rows_per_group, a.B, grid, st);
    default:
      return hipErrorInvalidValue;
  }
}

}  // namespace krill
