"""Python face of the CPU oracle (oracle/krill_oracle.c).

TEST INFRASTRUCTURE.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of bench.py import this module, and only as the checker
(or the timed CPU baseline).  The product package ``krill_amd`` never imports
it; the GPU path fails loudly instead of falling back to anything here.

How each oracle function is pinned (checked by something other than itself):

==========================  ====================================================
function                    pin
==========================  ====================================================
f16/bf16 conversions        exhaustive: all 65536 binary16 patterns round-trip;
                            binary32 -> binary16 against numpy's IEEE cast on
                            random and boundary values; bf16 against torch's
                            CPU RNE cast (tests/test_oracle.py).
quantize_ref (a1)           (1) tiny-input brute force with exact rational
                            arithmetic (fractions.Fraction) of every rounding
                            step; (2) the reference's own unit tests:
                            Weyl-sequence tensors round-trip within 1.5 steps
                            + 1e-3 / 1e-2 (QuantizedKVCacheUnitTests.swift
                            :38-84); (3) closed-form special cases (constant
                            row -> scale 0 after fp16 rounding, q = 0, zero =
                            value; the row minimum always maps to q = 0);
                            (4) committed golden vectors (tests/golden/).
                            A zero row minimum is returned as +0 (which of
                            +-0 a minimum returns depends on comparison order).
quantize_mlx (a1')          MLX's CPU affine quantize (third-party mlx 0.31
                            via mlx-swift 0.31.4, absent here) restated from
                            its published algorithm and pinned choice by
                            choice: groups built so that each plausible
                            alternative changes a byte, with the bytes derived
                            by hand -- ties round half to even, the scale is
                            negative and the bias is the max when |max| >=
                            |min|, constant groups store fp16(-1e-7) and the
                            constant (0 -> bias 0), q uses the binary32
                            scale edge/q0 (not its fp16 rounding) and divides
                            (not a reciprocal multiply); an exact-rational
                            restatement with explicit binary32 rounding on 240
                            random groups; invariants (q in [0,255], round
                            trip within half a step + fp16 rounding).
dequant_ref (a3)            exhaustive check of the two-rounding formula for
                            every q byte against numpy float16 arithmetic.
attention_f64 (a7/a8)       closed forms: one key -> output = that value row;
                            equal keys -> output = mean of values; huge masked
                            tail has no effect; brute force against an
                            independent numpy softmax on tiny shapes.
attention_mlx_composed      MLX's op-by-op SDPA (the reference's CPU path):
(a7, second oracle)         closed forms (one key -> the value row exactly,
                            equal keys -> the mean within fp16 rounding);
                            within the roundings it adds of attention_f64
                            (its unrounded-query form within 1e-5).  Its exact
                            agreement with MLX is parity unpinned (MLX is
                            not in this tree).
stack_left_padded (a5)      closed form of BatchedDecode.swift:119-147 on
                            integer rows (tests/test_oracle.py).
prefix_key (a10)            FNV-1a 64 published test vectors ("" and "a").
sliding_window_rows         the reference's mask tests
(next row 4)                (SlidingWindowMaskTests.swift:17-53): the
                            visible sets of (4, 0, 2), (3, 0, 10) and
                            (1, 600, 512), key by key.
attention_window_f64        reduces to attention_f64 on the key slice; against
                            an independent numpy softmax with a -inf mask.
rotating_retained_start     the retained rows of RotatingKVCacheTests.swift
                            :115-161 (window 4: last min(t+1, 4) tokens after
                            t appends; truncate 10 -> 8 then one append keeps
                            tokens 6, 7, 8; below token 6 refused).
rope_rows (next row 3)      closed forms: position 0 of a cos/sin table is the
                            identity bit for bit; a quarter turn (cos 0,
                            sin 1) maps (x, y) -> (-y, x) exactly; against
                            the float64 rotation of each (i, i + D/2) pair
                            within one rounding of the element dtype; two
                            turns compose to their sum; pair norms kept.
==========================  ====================================================
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libkrill_oracle.so")
_lib = None

DT_F16 = 0
DT_BF16 = 1


def build() -> str:
    """Compile the oracle with its Makefile (gcc); returns the .so path."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        P = ctypes.c_void_p
        i32, i64, u64, f32, f64 = (ctypes.c_int32, ctypes.c_int64, ctypes.c_uint64,
                                   ctypes.c_float, ctypes.c_double)
        L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_f16_to_f32.restype = f32
        L.oracle_f32_to_f16.argtypes = [f32]
        L.oracle_f32_to_f16.restype = ctypes.c_uint16
        L.oracle_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.oracle_bf16_to_f32.restype = f32
        L.oracle_f32_to_bf16.argtypes = [f32]
        L.oracle_f32_to_bf16.restype = ctypes.c_uint16
        L.oracle_f16_to_f32_array.argtypes = [P, i64, P]
        L.oracle_f32_to_f16_array.argtypes = [P, i64, P]
        L.oracle_f32_to_bf16_array.argtypes = [P, i64, P]
        L.oracle_quantize_ref_rows.argtypes = [P, i32, i64, i32, P, P, P]
        L.oracle_quantize_mlx_affine.argtypes = [P, i32, i64, i32, i32, P, P, P]
        L.oracle_dequant_ref_rows.argtypes = [P, P, P, i64, i32, P]
        L.oracle_dequant_f64.argtypes = [P, P, P, i64, i32, i32, i32, P]
        L.oracle_attention_f64.argtypes = [P, P, P, i32, i32, i32, P, f64, P]
        L.oracle_stack_left_padded.argtypes = [P, P, P, P, i32, i32, i32, i32, i32, P, P, P]
        L.oracle_fnv1a64.argtypes = [P, i64, u64]
        L.oracle_fnv1a64.restype = u64
        L.oracle_prefix_key.argtypes = [ctypes.c_char_p, ctypes.c_char_p, i32, P, i64]
        L.oracle_prefix_key.restype = u64
        L.oracle_common_prefix_length.argtypes = [P, i64, P, i64]
        L.oracle_common_prefix_length.restype = i64
        L.oracle_baseline_create.argtypes = [i32, i32, i32, i32, i32, P, u64]
        L.oracle_baseline_create.restype = P
        L.oracle_baseline_destroy.argtypes = [P]
        L.oracle_baseline_threads.argtypes = [P]
        L.oracle_baseline_threads.restype = i32
        L.oracle_baseline_set_threads.argtypes = [P, i32]
        L.oracle_baseline_step.argtypes = [P, P, P, P, i32, f32, P, i32]
        _lib = L
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return a.ctypes.data_as(ctypes.c_void_p)


# --------------------------------------------------------------------------
# dtype helpers (bit patterns are carried as uint16 arrays)
# --------------------------------------------------------------------------

def f32_to_f16_bits(x) -> np.ndarray:
    """numpy's IEEE RNE cast (the C conversion is tested bit-equal to it)."""
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def f16_bits_to_f32(h) -> np.ndarray:
    return np.ascontiguousarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def c_f16_to_f32_array(h) -> np.ndarray:
    h = np.ascontiguousarray(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().oracle_f16_to_f32_array(_p(h), h.size, _p(out))
    return out


def c_f32_to_f16_array(f) -> np.ndarray:
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_f16_array(_p(f), f.size, _p(out))
    return out


def c_f32_to_bf16_array(f) -> np.ndarray:
    f = np.ascontiguousarray(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().oracle_f32_to_bf16_array(_p(f), f.size, _p(out))
    return out


def c_f32_to_f16(v: float) -> int:
    return int(lib().oracle_f32_to_f16(float(v)))


def c_f16_to_f32(h: int) -> float:
    return float(lib().oracle_f16_to_f32(int(h)))


def f32_to_bf16_bits(x) -> np.ndarray:
    """Vectorised RNE float32 -> bfloat16 bits (same rule as the C oracle)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_bits_to_f32(b) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def bits_to_f32(b, dt: int) -> np.ndarray:
    if dt == DT_BF16:
        return bf16_bits_to_f32(b)
    return np.ascontiguousarray(b, dtype=np.uint16).view(np.float16).astype(np.float32)


# --------------------------------------------------------------------------
# a1 / a1' / a3
# --------------------------------------------------------------------------

def quantize_ref(x_bits: np.ndarray, dt: int):
    """Reference row quantizer over the last axis (QuantizedKVCache.swift:181-197).

    Returns (q u8 [..., D], scale f16-bits [..., 1], zero f16-bits [..., 1])."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    D = x.shape[-1]
    n = x.size // D
    q = np.empty(x.shape, np.uint8)
    s = np.empty(x.shape[:-1] + (1,), np.uint16)
    z = np.empty(x.shape[:-1] + (1,), np.uint16)
    lib().oracle_quantize_ref_rows(_p(x), dt, n, D, _p(q), _p(s), _p(z))
    return q, s, z


def quantize_mlx(x_bits: np.ndarray, dt: int, group: int = 64):
    """MLX affine 8-bit group quantizer (mlx's CPU affine quantize; pins in the header)."""
    x = np.ascontiguousarray(x_bits, dtype=np.uint16)
    D = x.shape[-1]
    G = D // group
    n = x.size // D
    q = np.empty(x.shape, np.uint8)
    s = np.empty(x.shape[:-1] + (G,), np.uint16)
    b = np.empty(x.shape[:-1] + (G,), np.uint16)
    lib().oracle_quantize_mlx_affine(_p(x), dt, n, D, group, _p(q), _p(s), _p(b))
    return q, s, b


def quantize(x_bits: np.ndarray, dt: int, mode: int, group: int = 64):
    """mode 0 = reference rows, mode 1 = affine groups of `group`."""
    return quantize_ref(x_bits, dt) if mode == 0 else quantize_mlx(x_bits, dt, group)


def rope_rows(x_bits: np.ndarray, dt: int, positions, cos_sin) -> np.ndarray:
    """RoPE of rows [..., D] (MLX RoPE, traditional = false, all D dims) as
    krill_quantize_append_rope applies it to K: pair (i, i + D/2) of the row
    at position p turns by the table's angle i: x'[i] = x[i] c - x[i+D/2] s,
    x'[i+D/2] = x[i] s + x[i+D/2] c in float32 (each product and sum rounded
    once), then rounded to the element dtype.  positions: one per row
    (shape x.shape[:-1]); cos_sin: float32 [max_pos, D].  Returns dtype bits."""
    x = bits_to_f32(x_bits, dt)
    D = x.shape[-1]
    h = D // 2
    cs = np.asarray(cos_sin, np.float32)[np.asarray(positions)]
    c, s = cs[..., :h], cs[..., h:]
    x1, x2 = x[..., :h], x[..., h:]
    o1 = (x1 * c).astype(np.float32) - (x2 * s).astype(np.float32)
    o2 = (x1 * s).astype(np.float32) + (x2 * c).astype(np.float32)
    o = np.concatenate([o1, o2], axis=-1).astype(np.float32)
    return f32_to_bf16_bits(o) if dt == DT_BF16 else f32_to_f16_bits(o)


def dequant_ref_f16(q, s, z) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    z = np.ascontiguousarray(z, np.uint16)
    D = q.shape[-1]
    out = np.empty(q.shape, np.uint16)
    lib().oracle_dequant_ref_rows(_p(q), _p(s), _p(z), q.size // D, D, _p(out))
    return out


def dequant_f64(q, s, z, mode: int) -> np.ndarray:
    q = np.ascontiguousarray(q, np.uint8)
    s = np.ascontiguousarray(s, np.uint16)
    z = np.ascontiguousarray(z, np.uint16)
    D = q.shape[-1]
    G = s.shape[-1]
    out = np.empty(q.shape, np.float64)
    lib().oracle_dequant_f64(_p(q), _p(s), _p(z), q.size // D, D, G, mode, _p(out))
    return out


# --------------------------------------------------------------------------
# a7 / a8
# --------------------------------------------------------------------------

def attention_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, limits, scale: float) -> np.ndarray:
    """q [NR, D], k/v [T, D] (float64), row r sees keys [0, limits[r])."""
    q = np.ascontiguousarray(q, np.float64)
    k = np.ascontiguousarray(k, np.float64)
    v = np.ascontiguousarray(v, np.float64)
    NR, D = q.shape
    T = k.shape[0]
    lim = np.ascontiguousarray(np.broadcast_to(np.asarray(limits, np.int32), (NR,)), np.int32)
    out = np.empty((NR, D), np.float64)
    lib().oracle_attention_f64(_p(q), _p(k), _p(v), NR, T, D, _p(lim), float(scale), _p(out))
    return out


def attention_mlx_composed(q_bits: np.ndarray, q_dt: int, k_f16: np.ndarray, v_f16: np.ndarray, limits,
                           scale: float) -> np.ndarray:
    """MLX's composed SDPA on the dequantized cache, op by op: the arithmetic
    of the reference's decode SDPA (MLXFast.scaledDotProductAttention,
    Attention.swift:95-98, Gemma4Model.swift:516-517) where MLX runs it as
    separate ops (its CPU path): q scaled in its own dtype (the scale a
    scalar of that dtype), scores = q . K^T, softmax (precise: float32
    inside), out = P . V.  The dtype of the products is the promotion of
    the query dtype and fp16 (the dequantized K/V): fp16 for fp16 queries --
    scores, weights and output each rounded once to fp16 (float32
    accumulation inside each product) -- and float32 for bf16 queries.
    q_bits [NR, D] in q_dt; k_f16 / v_f16 [T, D] fp16 bits; row r sees keys
    [0, limits[r]).  Returns float64 copies of the output values.

    MLX (mlx-swift 0.31.4) is not in this tree: this restates its published
    op sequence; it is pinned by closed forms (one key, equal keys) and by
    its distance from attention_f64 (within the roundings it adds: the
    scaled query in its dtype, and in fp16 the scores, weights and output),
    not against MLX's own outputs."""
    qv = bits_to_f32(q_bits, q_dt)
    if q_dt == DT_BF16:
        sc = float(bf16_bits_to_f32(f32_to_bf16_bits(np.array([scale], np.float32)))[0])
        qs = bf16_bits_to_f32(f32_to_bf16_bits(qv * np.float32(sc)))
    else:
        sc = float(np.float16(scale))
        qs = (qv * np.float32(sc)).astype(np.float16).astype(np.float32)
    k = f16_bits_to_f32(k_f16)
    v = f16_bits_to_f32(v_f16)
    half = q_dt == DT_F16
    NR, D = qs.shape
    lim = np.broadcast_to(np.asarray(limits, np.int64), (NR,))
    out = np.empty((NR, D), np.float64)
    for r in range(NR):
        T = int(lim[r])
        s_ = k[:T] @ qs[r]  # float32 accumulation
        if half:
            s_ = s_.astype(np.float16).astype(np.float32)
        e = np.exp(s_ - s_.max())
        p = (e / e.sum(dtype=np.float32)).astype(np.float32)
        if half:
            p = p.astype(np.float16).astype(np.float32)
        o = p @ v[:T]
        if half:
            o = o.astype(np.float16).astype(np.float32)
        out[r] = o
    return out


def sliding_window_rows(new_len: int, cache_len: int, window: int):
    """Visible key range [lo, hi) of each of new_len query rows whose first
    row sits at absolute position cache_len: causal and q - k < window
    (createSlidingWindowCausalMask, Sources/KrillCore/LlamaModel.swift:216-230)."""
    rows = []
    for i in range(new_len):
        q = cache_len + i
        rows.append((max(0, q - window + 1), q + 1))
    return rows


def attention_window_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray, lo, hi, scale: float) -> np.ndarray:
    """q [NR, D], k/v [T, D]: row r attends keys [lo[r], hi[r]) -- attention_f64
    over that slice of the keys."""
    q = np.ascontiguousarray(q, np.float64)
    out = np.empty(q.shape, np.float64)
    for r in range(q.shape[0]):
        a, b = int(lo[r]), int(hi[r])
        out[r] = attention_f64(q[r: r + 1], k[a:b], v[a:b], [b - a], scale)[0]
    return out


def rotating_retained_start(ops, window: int) -> tuple[int, int]:
    """(total tokens, first retained token) after ops on a RotatingKVCache
    (Sources/KrillCache/RotatingKVCache.swift:70-75 trimForAppend before
    every append of L >= 1 rows, :130-138 truncate within the retained
    tail): ops = [("append", L) | ("truncate", n)]."""
    total = start = 0
    for op, x in ops:
        if op == "append":
            if x >= 1:
                if total - start > window - 1:
                    start = total - (window - 1)
                total += x
        elif op == "truncate":
            if x < total:
                if x < start:
                    raise ValueError("truncate below the retained range")
                total = x
    return total, start


# --------------------------------------------------------------------------
# a5
# --------------------------------------------------------------------------

def stack_left_padded(rows_q, rows_s, rows_z, lens, sMax=None):
    """rows_*[r]: [H, L_r, D] u8 / [H, L_r, G] f16 bits -> stacked right-aligned."""
    R = len(rows_q)
    H, _, D = rows_q[0].shape
    G = rows_s[0].shape[-1]
    lens = np.ascontiguousarray(lens, np.int32)
    if sMax is None:
        sMax = int(lens.max()) if R else 0
    rq = [np.ascontiguousarray(a, np.uint8) for a in rows_q]
    rs = [np.ascontiguousarray(a, np.uint16) for a in rows_s]
    rz = [np.ascontiguousarray(a, np.uint16) for a in rows_z]
    pq = (ctypes.c_void_p * R)(*[a.ctypes.data for a in rq])
    ps = (ctypes.c_void_p * R)(*[a.ctypes.data for a in rs])
    pz = (ctypes.c_void_p * R)(*[a.ctypes.data for a in rz])
    oq = np.empty((R, H, sMax, D), np.uint8)
    os_ = np.empty((R, H, sMax, G), np.uint16)
    oz = np.empty((R, H, sMax, G), np.uint16)
    lib().oracle_stack_left_padded(pq, ps, pz, _p(lens), R, H, D, G, sMax, _p(oq), _p(os_), _p(oz))
    return oq, os_, oz


# --------------------------------------------------------------------------
# a10
# --------------------------------------------------------------------------

def fnv1a64(data: bytes) -> int:
    buf = np.frombuffer(data, np.uint8).copy() if data else np.zeros(1, np.uint8)
    return int(lib().oracle_fnv1a64(_p(buf), len(data), 14695981039346656037))


def prefix_key(model_id: str, media_hash: str | None, dtype_tag: int, tokens) -> int:
    t = np.ascontiguousarray(tokens, np.int64)
    if t.size == 0:
        t = np.zeros(1, np.int64)
        n = 0
    else:
        n = t.size
    return int(lib().oracle_prefix_key(model_id.encode(), (media_hash or "").encode(),
                                       dtype_tag, _p(t), n))


def common_prefix_length(a, b) -> int:
    na, nb = len(a), len(b)
    a2 = np.ascontiguousarray(a, np.int64) if na else np.zeros(1, np.int64)
    b2 = np.ascontiguousarray(b, np.int64) if nb else np.zeros(1, np.int64)
    return int(lib().oracle_common_prefix_length(_p(a2), na, _p(b2), nb))


# --------------------------------------------------------------------------
# CPU baseline session (the reference's per-step algorithm, see the C file)
# --------------------------------------------------------------------------

class Baseline:
    def __init__(self, layers, B, Hkv, Hq, D, lens, seed=0):
        self.layers, self.B, self.Hkv, self.Hq, self.D = layers, B, Hkv, Hq, D
        self._lens = np.ascontiguousarray(lens, np.int32)
        self.h = lib().oracle_baseline_create(layers, B, Hkv, Hq, D, _p(self._lens), seed)

    @property
    def threads(self) -> int:
        return int(lib().oracle_baseline_threads(self.h))

    def set_threads(self, n: int):
        lib().oracle_baseline_set_threads(self.h, int(n))

    def step(self, q_bits, k_bits, v_bits, dt, scale, out, layers_to_run=0):
        lib().oracle_baseline_step(self.h, _p(q_bits), _p(k_bits), _p(v_bits), dt,
                                   float(scale), _p(out), layers_to_run)

    def close(self):
        if self.h:
            lib().oracle_baseline_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
