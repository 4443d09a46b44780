// Device-side definitions shared by the gfx950 kernels of libkrillhip:
// pool layout, dtype conversions and wave64 helpers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace krill {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

enum { DT_F16 = 0, DT_BF16 = 1, DT_F32 = 2 };
enum { MODE_REF = 0, MODE_AFFINE = 1 };

constexpr int kBlockTokens = 64;

// Layout of one (layer, block, kv-head) region of the pool, D = head_dim,
// G = scale/zero groups per token (1 in the reference's row mode, D/64 in the
// affine group-64 mode).  Every piece is laid out so that a wave64 load of
// 16 bytes per lane (4*G bytes for metadata) reads one contiguous run:
//   [0, 64*D)          K bytes in 16-byte d-chunks, chunk major:
//                        ((d/16)*64 + t)*16 + d%16
//                      (lane = token reads chunk c of all 64 tokens at once)
//   [64*D, 128*D)      V bytes, per 32-token group tg (32*D bytes each) in
//                      16-byte pieces of 16 token positions of one d:
//                        tg*32*D + ((2*(d%DPL) + p/16)*64 + d/DPL)*16 + p%16
//                      with DPL = D/64 and p = vpos(t%32) the token's
//                      position (lane l, owning d = DPL*l .. DPL*l+DPL-1,
//                      reads piece i of all lanes at once)
//   [128*D, +256*G)    K (scale, zero) fp16 pairs:  (t*G + g)*4
//   [128*D+256*G, ..)  V (scale, zero) fp16 pairs
// The 16-byte K chunks also hold the 8 consecutive d of a 16x16x32 MFMA A
// operand contiguously.  Token positions inside a V group follow the MFMA P.V
// B operand (lane quarter q holds tokens 4q..4q+3 and 16+4q..16+4q+3 as
// positions 8q..8q+7, contiguous), so P never has to be transposed.
__host__ __device__ constexpr int head_region_bytes(int D, int G) { return 128 * D + 512 * G; }
__host__ __device__ constexpr int v_offset(int D) { return 64 * D; }
__host__ __device__ constexpr int km_offset(int D) { return 128 * D; }
__host__ __device__ constexpr int vm_offset(int D, int G) { return 128 * D + 256 * G; }
__host__ __device__ constexpr int k_byte(int t, int d) { return (((d >> 4) * 64 + t) << 4) + (d & 15); }
// position of token tt (0..31) inside its 32-token group of a V row
__host__ __device__ constexpr int vpos(int tt) {
  return (((tt & 15) >> 2) << 3) + (tt & 3) + ((tt >> 4) << 2);
}
// inverse of vpos
__host__ __device__ constexpr int vtok(int p) { return ((p >> 3) << 2) + (p & 3) + (((p >> 2) & 1) << 4); }
// byte of V row d, token group tg, position p (0..31)
__host__ __device__ constexpr int v_pos_byte(int D, int tg, int d, int p) {
  return 64 * D + tg * 32 * D + (((2 * (d % (D / 64)) + (p >> 4)) * 64 + d / (D / 64)) << 4) + (p & 15);
}
__host__ __device__ constexpr int v_byte(int D, int t, int d) { return v_pos_byte(D, t >> 5, d, vpos(t & 31)); }

// Device view of one layer of the pool.
struct LayerView {
  uint8_t *base;         // layer base
  int64_t block_stride;  // bytes per block (all heads)
  int32_t head_bytes;    // bytes per (block, head)
  int32_t num_blocks;
};

__device__ __forceinline__ uint8_t *head_region(const LayerView &lv, int32_t block, int32_t h) {
  return lv.base + (int64_t)block * lv.block_stride + (int64_t)h * lv.head_bytes;
}

// Block region of the pool as a buffer resource: loads past `bytes` return
// zero without touching memory, so the prefetch after a wave's last block is
// free (bytes = 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t block_rsrc(const uint8_t *p, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(p), (short)0, bytes, 0x00020000);
}

// ---------------------------------------------------------------- dtypes

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  return (float)__builtin_bit_cast(_Float16, h);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, round to nearest even
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) {
  return __builtin_bit_cast(float, (uint32_t)b << 16);
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t x = __builtin_bit_cast(uint32_t, f);
  if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
  x += 0x7fffu + ((x >> 16) & 1u);
  return (uint16_t)(x >> 16);
}
template <int DT>
__device__ __forceinline__ float load_elem(const uint16_t *p) {
  return DT == DT_BF16 ? bf16_bits_to_f32(*p) : f16_bits_to_f32(*p);
}
template <int DT>
__device__ __forceinline__ float elem_to_f32(uint16_t v) {
  return DT == DT_BF16 ? bf16_bits_to_f32(v) : f16_bits_to_f32(v);
}
// Round a binary32 value to the element dtype and back (round to nearest even).
template <int DT>
__device__ __forceinline__ float round_dt(float f) {
  return DT == DT_BF16 ? bf16_bits_to_f32(f32_to_bf16_bits(f)) : f16_bits_to_f32(f32_to_f16_bits(f));
}

__device__ __forceinline__ void store_out(void *out, int64_t idx, float v, int dt) {
  if (dt == DT_F32)
    reinterpret_cast<float *>(out)[idx] = v;
  else if (dt == DT_F16)
    reinterpret_cast<uint16_t *>(out)[idx] = f32_to_f16_bits(v);
  else
    reinterpret_cast<uint16_t *>(out)[idx] = f32_to_bf16_bits(v);
}

// N consecutive outputs (N a multiple of 4; idx a multiple of N) in 16-byte
// stores where they fill them.
template <int N>
__device__ __forceinline__ void store_run(void *out, int64_t idx, const float (&v)[N], int dt) {
  static_assert(N % 4 == 0, "runs of 4k values");
  if (dt == DT_F32) {
#pragma unroll
    for (int k = 0; k < N; k += 4)
      *reinterpret_cast<float4 *>(reinterpret_cast<float *>(out) + idx + k) = float4{v[k], v[k + 1], v[k + 2], v[k + 3]};
    return;
  }
  uint32_t w[N / 2];
#pragma unroll
  for (int k = 0; k < N / 2; ++k) {
    const uint32_t lo = dt == DT_F16 ? f32_to_f16_bits(v[2 * k]) : f32_to_bf16_bits(v[2 * k]);
    const uint32_t hi = dt == DT_F16 ? f32_to_f16_bits(v[2 * k + 1]) : f32_to_bf16_bits(v[2 * k + 1]);
    w[k] = lo | (hi << 16);
  }
  uint16_t *o = reinterpret_cast<uint16_t *>(out) + idx;
  if constexpr (N % 8 == 0) {
#pragma unroll
    for (int k = 0; k < N / 2; k += 4) *reinterpret_cast<uint4 *>(o + 2 * k) = uint4{w[k], w[k + 1], w[k + 2], w[k + 3]};
  } else {
#pragma unroll
    for (int k = 0; k < N / 2; k += 2) *reinterpret_cast<uint2 *>(o + 2 * k) = uint2{w[k], w[k + 1]};
  }
}

// ---------------------------------------------------------- byte unpacking

// Two bytes of `w` as fp16 (1024 + byte): byte values ride in the mantissa of
// 0x64XX, so one v_perm_b32 turns two bytes into two exact fp16 values.
__device__ __forceinline__ half2_t bytes01_plus1024(uint32_t w) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x04010400u));
}
__device__ __forceinline__ half2_t bytes23_plus1024(uint32_t w) {
  return __builtin_bit_cast(half2_t, __builtin_amdgcn_perm(0x64646464u, w, 0x04030402u));
}

__device__ __forceinline__ float dot2(half2_t a, half2_t b, float c) {
  return __builtin_amdgcn_fdot2(a, b, c, false);
}

__device__ __forceinline__ half2_t u32_as_h2(uint32_t u) { return __builtin_bit_cast(half2_t, u); }
__device__ __forceinline__ uint32_t h2_as_u32(half2_t h) { return __builtin_bit_cast(uint32_t, h); }

// LDS address space (destination of the direct-to-LDS buffer loads)
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ float4_t mfma16x16x32(half8_t a, half8_t b, float4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
// Eight bytes as exact fp16 u - 128.
__device__ __forceinline__ half8_t bytes8_centred(uint2 w) {
  const half2_t m1152 = half2_t{(_Float16)-1152.0f, (_Float16)-1152.0f};
  const half2_t a = bytes01_plus1024(w.x) + m1152, b = bytes23_plus1024(w.x) + m1152;
  const half2_t c = bytes01_plus1024(w.y) + m1152, d = bytes23_plus1024(w.y) + m1152;
  return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// Eight bytes dequantized as the reference does, f16(f16(u * s) + z), with
// the eight positions' fp16 scales `sc` and zero points `zc` (pairs per word).
__device__ __forceinline__ half8_t bytes8_dequant_ref(uint2 w, uint4 sc, uint4 zc) {
  const half2_t m1024 = half2_t{(_Float16)-1024.0f, (_Float16)-1024.0f};
  const half2_t a = (bytes01_plus1024(w.x) + m1024) * u32_as_h2(sc.x) + u32_as_h2(zc.x);
  const half2_t b = (bytes23_plus1024(w.x) + m1024) * u32_as_h2(sc.y) + u32_as_h2(zc.y);
  const half2_t c = (bytes01_plus1024(w.y) + m1024) * u32_as_h2(sc.z) + u32_as_h2(zc.z);
  const half2_t d = (bytes23_plus1024(w.y) + m1024) * u32_as_h2(sc.w) + u32_as_h2(zc.w);
  return half8_t{a[0], a[1], b[0], b[1], c[0], c[1], d[0], d[1]};
}
// Eight binary32 weights as fp16 high parts (round to nearest) and the fp16
// rounding of their remainders: hi + lo is within about 2^-22 of each weight.
__device__ __forceinline__ void split_hi_lo(float4 a, float4 b, half8_t &hi, half8_t &lo) {
  typedef float f2_t __attribute__((ext_vector_type(2)));
  const f2_t f[4] = {f2_t{a.x, a.y}, f2_t{a.z, a.w}, f2_t{b.x, b.y}, f2_t{b.z, b.w}};
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const half2_t h = __builtin_convertvector(f[k], half2_t);
    const f2_t back = __builtin_convertvector(h, f2_t);
    const half2_t l = __builtin_convertvector(f2_t{f[k].x - back.x, f[k].y - back.y}, half2_t);
    hi[2 * k] = h[0];
    hi[2 * k + 1] = h[1];
    lo[2 * k] = l[0];
    lo[2 * k + 1] = l[1];
  }
}

// ---------------------------------------------------------- wave helpers

__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }

template <int FIRST, int LAST>
__device__ __forceinline__ float wave_sum_range(float v) {
#pragma unroll
  for (int m = FIRST; m <= LAST; m <<= 1) v += shfl_xor(v, m);
  return v;
}
template <int FIRST, int LAST>
__device__ __forceinline__ float wave_max_range(float v) {
#pragma unroll
  for (int m = FIRST; m <= LAST; m <<= 1) v = fmaxf(v, shfl_xor(v, m));
  return v;
}
template <int FIRST, int LAST>
__device__ __forceinline__ float wave_min_range(float v) {
#pragma unroll
  for (int m = FIRST; m <= LAST; m <<= 1) v = fminf(v, shfl_xor(v, m));
  return v;
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Whole-wave all-reductions without LDS: DPP inside each 16-lane row
// (quad xor 1, quad xor 2, row rotate 4, row rotate 8), then the gfx950
// row-pair and half-wave swaps (v_permlane16_swap / v_permlane32_swap).
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0u, __builtin_bit_cast(unsigned, v), CTRL, 0xf, 0xf,
                                                               false));
}
// The row swaps are issued as inline asm with both registers as in/out
// operands: through __builtin_amdgcn_permlane{16,32}_swap this compiler
// reads only the first register after the swap and uses it for both
// results.  With a == b on entry, v_permlane16_swap leaves rows {0,0,2,2} of
// the value in `a` and rows {1,1,3,3} in `b`; v_permlane32_swap leaves rows
// {0,1,0,1} and {2,3,2,3}.  The s_nop covers the VALU-write -> permlane-read
// hazard of the copy the compiler makes to split a from b.
__device__ __forceinline__ void row_swap16(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ void row_swap32(float &a, float &b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1" : "+v"(a), "+v"(b));
}
__device__ __forceinline__ float swap16_sum(float v) {
  float a = v, b = v;
  row_swap16(a, b);
  return a + b;
}
__device__ __forceinline__ float swap32_sum(float v) {
  float a = v, b = v;
  row_swap32(a, b);
  return a + b;
}
__device__ __forceinline__ float swap16_max(float v) {
  float a = v, b = v;
  row_swap16(a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float swap32_max(float v) {
  float a = v, b = v;
  row_swap32(a, b);
  return fmaxf(a, b);
}
// Sum over the 16 lanes of each DPP row, left in every lane of the row.
__device__ __forceinline__ float row_allsum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
  v += dpp_f32<0x124>(v);  // row_ror:4
  v += dpp_f32<0x128>(v);  // row_ror:8
  return v;
}
// Maximum over the 16 lanes of each DPP row, left in every lane of the row.
__device__ __forceinline__ float row_allmax(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  v = fmaxf(v, dpp_f32<0x128>(v));
  return v;
}
// Queries reach the matrix and dot-product instructions as fp16.  A bf16 row
// whose largest |q| is at or above 65504 (where the fp16 rounding overflows)
// is scaled by 2^-k first, k the smallest power that brings it below 2^15,
// and its scores by 2^k; both are exact.  Returns 2^-k (1 for every other
// row, non-finite maxima included) and sets `up` to 2^k.
__device__ __forceinline__ float q_range_scale(float absmax, float &up) {
  const int e = (int)((__builtin_bit_cast(uint32_t, absmax) >> 23) & 0xffu);  // biased exponent
  const int k = (absmax >= 65504.0f && e < 255) ? e - 141 : 0;              // 2^15 has e = 142
  up = __builtin_bit_cast(float, (uint32_t)(127 + k) << 23);
  return __builtin_bit_cast(float, (uint32_t)(127 - k) << 23);
}
// A value known to be the same in every lane, moved to a scalar register.
__device__ __forceinline__ float uniform_f32(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readfirstlane(__builtin_bit_cast(int, v)));
}
__device__ __forceinline__ float wave_allsum(float v) { return swap32_sum(swap16_sum(row_allsum(v))); }
__device__ __forceinline__ float wave_allmax(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x124>(v));
  v = fmaxf(v, dpp_f32<0x128>(v));
  return swap32_max(swap16_max(v));
}

// A zero the compiler cannot see through: loads addressed with it stay below
// the point where it is produced (used to keep scalar loads from being
// hoisted all at once).
__device__ __forceinline__ int opaque_zero() {
  int z;
  asm volatile("s_mov_b32 %0, 0" : "=s"(z));
  return z;
}
// Register fence: `x` is treated as rewritten after `after` is available, so
// work on `x` cannot be scheduled ahead of the work that produced `after`
// (bounds register live ranges the scheduler would otherwise stretch).
// The 16 bytes go in as one 128-bit register tuple: split into four 32-bit
// operands, the register allocator may give the components of a loop-carried
// load different registers on the two sides of the back edge, and the copies
// it then adds on the latch must wait for the load.
typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void order_after(uint4 &x, float after) {
  u32x4_t v = __builtin_bit_cast(u32x4_t, x);
  asm volatile("; order %0 after %1" : "+v"(v) : "v"(after));
  x = __builtin_bit_cast(uint4, v);
}
// Register settle: `x` counts as read and rewritten here, so a load into it
// completes before this point and later waits no longer track it.
__device__ __forceinline__ void settle(uint4 &x) {
  u32x4_t v = __builtin_bit_cast(u32x4_t, x);
  asm volatile("; settle %0" : "+v"(v));
  x = __builtin_bit_cast(uint4, v);
}
__device__ __forceinline__ void settle(uint32_t &x) { asm volatile("; settle %0" : "+v"(x)); }

// ---------------------------------------------------------- row quantizer
// Wave-collective quantization of one token row (K or V of one head): lane l
// owns the E = D/64 consecutive values d = l*E .. l*E+E-1, given as fp32
// widened from the input dtype DT.  Every kernel that writes new tokens into
// the pool goes through this function, so all of them store the same bytes.
// MODE_REF: QuantizedKVCache.quantizePerHead
// (Sources/KrillCache/QuantizedKVCache.swift:181-197):
//   mn, mx = min/max over D; scale = f32(dt(mx - mn)) / 255; safe = max(scale, 1e-8)
//   q = u8(trunc(clip(f32(dt(x - mn)) / safe, 0, 255))); (scale, zero) = (safe, mn)
// MODE_AFFINE (group 64): values cast to fp16, per group
//   s = max((max-min)/255, 1e-7) signed toward the larger-magnitude edge,
//   q0 = rint(edge/s), s = edge/q0 and bias = edge when q0 != 0 (else bias 0),
//   q = clip(rint((w - bias)/s), 0, 255); (scale, zero) = (s, bias).
// Scalar steps of the two quantizers, shared by the wave-collective and the
// lane-local forms so both produce the same bytes.
template <int DT>
__device__ __forceinline__ float ref_safe_scale(float mn, float mx) {
  const float sc = round_dt<DT>(mx - mn) / 255.0f;
  return sc > 1e-8f ? sc : 1e-8f;
}
template <int DT>
__device__ __forceinline__ uint8_t ref_q(float x, float mn, float safe) {
  float n = round_dt<DT>(x - mn) / safe;
  if (n < 0.0f) n = 0.0f;
  if (n > 255.0f) n = 255.0f;
  return (uint8_t)(uint32_t)n;
}
// affine input: the element rounded to fp16 (bf16 inputs are cast first)
template <int DT>
__device__ __forceinline__ float affine_w(float x) {
  return DT == DT_F16 ? x : f16_bits_to_f32(f32_to_f16_bits(x));
}
__device__ __forceinline__ void affine_params(float wmin, float wmax, float &s_out, float &bias_out) {
  const bool side = fabsf(wmin) > fabsf(wmax);
  float s = (wmax - wmin) / 255.0f;
  if (!(s > 1e-7f)) s = 1e-7f;
  s = side ? s : -s;
  const float edge = side ? wmin : wmax;
  const float q0 = rintf(edge / s);
  float bias = 0.0f;
  if (q0 != 0.0f) {
    s = edge / q0;
    bias = edge;
  }
  s_out = s;
  bias_out = bias;
}
__device__ __forceinline__ uint8_t affine_q(float w, float s, float bias) {
  float n = rintf((w - bias) / s);
  if (n > 255.0f) n = 255.0f;
  if (n < 0.0f) n = 0.0f;
  return (uint8_t)(uint32_t)n;
}

// The two quantizers' per-element division q = x / s done as x * r, with r
// = v_rcp_f32(s) (within one ulp of 1/s), wherever that provably gives the
// same byte: |fl(x r) - fl(x / s)| <= (2^-23 + 2^-24 + 2^-24) |x / s| =
// 2^-22 |x / s| < 2^-13 for |x / s| < 512 (the quotients here stay within
// about [-1, 256]), so when x r lies more than 2^-12 from every rounding
// boundary of the step that follows (k + 1/2 for rint, k for truncation)
// both round to the same integer; otherwise the exact division decides.
// (About 2^-11 of uniformly spread quotients take the division.)

// affine_q for four elements (byte e = element e of the word), with the
// division y = (w - bias) / s done as (w - bias) * r, r = v_rcp_f32(s),
// wherever that provably gives the same byte.  Off a rounding tie (ties sit
// at k + 1/2, at distance |fract(y) - 1/2|) by more than 2^-12, rint(y) =
// floor(y + 1/2), which v_cvt_rpi_i32_f32 gives as an integer in one step
// (y + 1/2 is exact for |y| < 512), clamped as an integer.  No branch per
// element: when any of the four is near a tie (or |y| >= 512, or NaN) all
// four take the exact division, which gives the same bytes where the fast
// path held.
__device__ __forceinline__ uint32_t affine_q4(const float (&w)[4], float s, float bias, float r) {
  float a[4];
  int n[4];
  int ok = 1;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    a[e] = w[e] - bias;
    const float y = a[e] * r;
    asm("v_cvt_rpi_i32_f32 %0, %1" : "=v"(n[e]) : "v"(y));
    ok &= (int)(fabsf(y) < 512.0f) & (int)(fabsf(__builtin_amdgcn_fractf(y) - 0.5f) > 0x1p-12f);
  }
  if (!ok) {
#pragma unroll
    for (int e = 0; e < 4; ++e) n[e] = (int)rintf(a[e] / s);
  }
  uint32_t q = 0;
#pragma unroll
  for (int e = 0; e < 4; ++e) q |= (uint32_t)min(max(n[e], 0), 255) << (8 * e);
  return q;
}
template <int DT>
__device__ __forceinline__ uint8_t ref_q_r(float x, float mn, float safe, float r) {
  const float a = round_dt<DT>(x - mn);
  float n = a * r;
  if (!(fabsf(n) < 512.0f && fabsf(n - rintf(n)) > 0x1p-12f)) n = a / safe;
  if (n < 0.0f) n = 0.0f;
  if (n > 255.0f) n = 255.0f;
  return (uint8_t)(uint32_t)n;
}

template <int D, int MODE, int DT>
__device__ __forceinline__ void quantize_row(const float (&x)[D / 64], uint8_t (&qb)[D / 64], float &scale,
                                             float &zero) {
  constexpr int E = D / 64;
  if constexpr (MODE == MODE_REF) {
    float mn = x[0], mx = x[0];
#pragma unroll
    for (int e = 1; e < E; ++e) {
      mn = fminf(mn, x[e]);
      mx = fmaxf(mx, x[e]);
    }
    mn = wave_min_range<1, 32>(mn);
    mx = wave_max_range<1, 32>(mx);
    const float safe = ref_safe_scale<DT>(mn, mx);
#pragma unroll
    for (int e = 0; e < E; ++e) qb[e] = ref_q<DT>(x[e], mn, safe);
    scale = safe;
    zero = mn + 0.0f;  // a zero minimum is stored as +0 (min over +-0 depends on order)
  } else {
    constexpr int LPG = 64 / E;  // lanes per group of 64
    float w[E];
#pragma unroll
    for (int e = 0; e < E; ++e) w[e] = affine_w<DT>(x[e]);
    float wmin = w[0], wmax = w[0];
#pragma unroll
    for (int e = 1; e < E; ++e) {
      wmin = fminf(wmin, w[e]);
      wmax = fmaxf(wmax, w[e]);
    }
    wmin = wave_min_range<1, LPG / 2>(wmin);
    wmax = wave_max_range<1, LPG / 2>(wmax);
    affine_params(wmin, wmax, scale, zero);
#pragma unroll
    for (int e = 0; e < E; ++e) qb[e] = affine_q(w[e], scale, zero);
  }
}

// Stores a row quantized by quantize_row (kv 0: K, 1: V) as token t of the
// head region `reg`, with its fp16 (scale, zero) pair(s).
template <int D, int MODE>
__device__ __forceinline__ void store_row(uint8_t *reg, int kv, int t, int lane, const uint8_t (&qb)[D / 64],
                                          float scale, float zero) {
  constexpr int E = D / 64;
  constexpr int G = MODE == MODE_AFFINE ? D / 64 : 1;
  const int d0 = lane * E;
  if (kv == 0) {
    uint8_t *dst = reg + k_byte(t, d0);
    if constexpr (E == 1) {
      dst[0] = qb[0];
    } else if constexpr (E == 2) {
      *reinterpret_cast<uint16_t *>(dst) = (uint16_t)(qb[0] | (qb[1] << 8));
    } else if constexpr (E == 4) {
      *reinterpret_cast<uint32_t *>(dst) =
          (uint32_t)qb[0] | ((uint32_t)qb[1] << 8) | ((uint32_t)qb[2] << 16) | ((uint32_t)qb[3] << 24);
    } else {
      static_assert(E == 8, "head_dim 64, 128, 256 or 512");
      // d0 = 8 lane: the 8 bytes sit in one 16-byte K chunk
      *reinterpret_cast<uint2 *>(dst) =
          uint2{(uint32_t)qb[0] | ((uint32_t)qb[1] << 8) | ((uint32_t)qb[2] << 16) | ((uint32_t)qb[3] << 24),
                (uint32_t)qb[4] | ((uint32_t)qb[5] << 8) | ((uint32_t)qb[6] << 16) | ((uint32_t)qb[7] << 24)};
    }
  } else {
#pragma unroll
    for (int e = 0; e < E; ++e) reg[v_byte(D, t, d0 + e)] = qb[e];
  }
  const int g = MODE == MODE_AFFINE ? d0 / 64 : 0;
  if ((d0 & (MODE == MODE_AFFINE ? 63 : (D - 1))) == 0) {
    const uint32_t meta = (uint32_t)f32_to_f16_bits(scale) | ((uint32_t)f32_to_f16_bits(zero) << 16);
    const int off = (kv ? vm_offset(D, G) : km_offset(D)) + ((t * G + g) << 2);
    *reinterpret_cast<uint32_t *>(reg + off) = meta;
  }
}

}  // namespace krill
