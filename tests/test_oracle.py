"""Pins of the CPU oracle: each oracle function is checked against something
other than itself -- IEEE conversions in numpy/torch, independent dtype
arithmetic, the reference's own unit-test tolerances and closed forms."""
import os

import numpy as np
import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


# --------------------------------------------------------------- conversions

def test_f16_exhaustive_round_trip(oracle):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = oracle.c_f16_to_f32_array(bits)
    np.testing.assert_array_equal(f.view(np.uint32), bits.view(np.float16).astype(np.float32).view(np.uint32))
    nan = np.isnan(f)
    back = oracle.c_f32_to_f16_array(f)
    np.testing.assert_array_equal(back[~nan], bits[~nan])
    assert np.all(np.isnan(back[nan].view(np.float16)))


def test_f32_to_f16_matches_numpy_ieee_cast(oracle):
    rng = np.random.default_rng(0)
    parts = [
        rng.standard_normal(200_000).astype(np.float32),
        (rng.standard_normal(100_000) * 1e-5).astype(np.float32),   # subnormal range
        (rng.standard_normal(100_000) * 1e-7).astype(np.float32),   # below half the smallest subnormal
        (rng.uniform(6.0e4, 7.0e4, 100_000) * rng.choice([-1, 1], 100_000)).astype(np.float32),  # overflow edge
        rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32),  # any pattern
    ]
    # exact ties of binary16 (round to even) and boundaries
    h = np.arange(0, 0x7BFF, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    parts.append(((lo + hi) / 2).astype(np.float32))
    parts.append(np.array([65504, 65519.99, 65520, 2.0**-24, 2.0**-25, 3 * 2.0**-26, 0.0, -0.0], np.float32))
    x = np.concatenate(parts)
    x = x[~np.isnan(x)]
    with np.errstate(over="ignore"):  # values past 65520 round to inf on purpose
        expect = x.astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(oracle.c_f32_to_f16_array(x), expect)


def test_f32_to_bf16_matches_torch_rne(oracle):
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(1)
    x = np.concatenate([
        rng.standard_normal(200_000).astype(np.float32),
        rng.integers(0, 2**32, 200_000, dtype=np.uint64).astype(np.uint32).view(np.float32),
    ])
    x = x[~np.isnan(x)]
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(oracle.c_f32_to_bf16_array(x), want)
    np.testing.assert_array_equal(oracle.f32_to_bf16_bits(x), want)


# --------------------------------------------------- reference row quantizer

def _numpy_ref_quantize(x_bits, dt):
    """Restatement of QuantizedKVCache.quantizePerHead with numpy/torch dtype
    arithmetic (independent of the oracle's bit-level code): dtype subtraction,
    float32 division by 255 and by the safe scale, clip, truncating cast."""
    torch = pytest.importorskip("torch")
    if dt == 0:
        x = x_bits.view(np.float16)
        mn = x.min(axis=-1, keepdims=True)
        mx = x.max(axis=-1, keepdims=True)
        d = (mx - mn).astype(np.float32)                  # float16 subtraction
        xm = (x - mn).astype(np.float32)
        zero = mn.view(np.uint16)
    else:
        t = torch.from_numpy(x_bits.view(np.int16)).view(torch.bfloat16)
        mn = t.min(dim=-1, keepdim=True).values
        mx = t.max(dim=-1, keepdim=True).values
        d = (mx - mn).float().numpy()                     # bfloat16 subtraction
        xm = (t - mn).float().numpy()
        zero = mn.float().numpy().astype(np.float16).view(np.uint16)
    scale = d / np.float32(255.0)
    safe = np.maximum(scale, np.float32(1e-8))
    n = np.clip(xm / safe, np.float32(0), np.float32(255))
    q = n.astype(np.uint8)                                 # truncation
    return q, safe.astype(np.float16).view(np.uint16), zero


@pytest.mark.parametrize("dt", [0, 1])
@pytest.mark.parametrize("D", [4, 7, 64, 128])
def test_quantize_ref_matches_independent_restatement(oracle, dt, D):
    rng = np.random.default_rng(10 + D + dt)
    x = rng.standard_normal((500, D)).astype(np.float32) * rng.choice([0.01, 1, 30], (500, 1)).astype(np.float32)
    bits = oracle.f32_to_bf16_bits(x) if dt == 1 else oracle.f32_to_f16_bits(x)
    q, s, z = oracle.quantize_ref(bits, dt)
    eq, es, ez = _numpy_ref_quantize(bits, dt)
    np.testing.assert_array_equal(q, eq)
    np.testing.assert_array_equal(s, es)
    np.testing.assert_array_equal(z, ez)


def test_quantize_ref_known_answers(oracle):
    # [0, 1]: scale = f32(1)/255 rounds up, so 1/scale truncates to 254
    q, s, z = oracle.quantize_ref(np.array([[0, 1]], np.float32).astype(np.float16).view(np.uint16), 0)
    assert q.tolist() == [[0, 254]]
    assert s[0, 0] == np.float16(np.float32(1) / np.float32(255)).view(np.uint16)
    # constant row: scale clamps to 1e-8, which rounds to fp16 zero; q = 0; zero = the value
    c = np.full((1, 16), 3.5, np.float32).astype(np.float16).view(np.uint16)
    q, s, z = oracle.quantize_ref(c, 0)
    assert not q.any() and s[0, 0] == 0 and z[0, 0] == np.float16(3.5).view(np.uint16)
    deq = oracle.dequant_ref_f16(q, s, z).view(np.float16)
    assert np.all(deq == np.float16(3.5))
    # the row minimum always maps to byte 0
    rng = np.random.default_rng(3)
    x = oracle.f32_to_bf16_bits(rng.standard_normal((200, 64)).astype(np.float32))
    q, _, _ = oracle.quantize_ref(x, 1)
    xf = oracle.bf16_bits_to_f32(x)
    assert np.all(q[np.arange(200), xf.argmin(axis=1)] == 0)


def _weyl(shape, lo, hi):
    """deterministicTensor of QuantizedKVCacheUnitTests.swift:17-27 in float32
    (Swift Float arithmetic, no fused multiply-add), then fp16."""
    total = int(np.prod(shape))
    span = np.float32(max(np.float32(hi) - np.float32(lo), np.float32(1e-3)))
    c = np.float32(0.6180339887)
    i = np.arange(total).astype(np.float32)
    prod = (i * c).astype(np.float32)
    frac = (prod - np.trunc(prod).astype(np.float32)).astype(np.float32)
    vals = (np.float32(lo) + (frac * span).astype(np.float32)).astype(np.float32)
    return vals.reshape(shape).astype(np.float16).view(np.uint16)


@pytest.mark.parametrize("lo,hi,extra", [(0.0, 10.0, 1e-3), (0.0, 5.0, 1e-3), (-64.0, 64.0, 1e-2),
                                         (-32.0, 64.0, 1e-2)])
def test_reference_unit_test_round_trip_tolerance(oracle, lo, hi, extra):
    """QuantizedKVCacheUnitTests.swift:38-84: round trip within 1.5 steps + slack."""
    x = _weyl([1, 4, 8, 16], lo, hi)
    q, s, z = oracle.quantize_ref(x, 0)
    deq = oracle.dequant_ref_f16(q, s, z).view(np.float16).astype(np.float32)
    err = np.abs(deq - x.view(np.float16).astype(np.float32)).max()
    assert err < (hi - lo) / 255.0 * 1.5 + extra


def test_golden_quantize_vectors(oracle):
    """Committed fixtures (tests/golden/make_golden.py) still reproduce."""
    path = os.path.join(HERE, "golden", "quantize_golden.npz")
    g = np.load(path, allow_pickle=False)
    for name in sorted({k.rsplit("__", 1)[0] for k in g.files}):
        x, dt, mode = g[name + "__x"], int(g[name + "__dt"]), int(g[name + "__mode"])
        q, s, z = oracle.quantize(x, dt, mode)
        np.testing.assert_array_equal(q, g[name + "__q"], err_msg=name)
        np.testing.assert_array_equal(s, g[name + "__s"], err_msg=name)
        np.testing.assert_array_equal(z, g[name + "__z"], err_msg=name)


# ------------------------------------------------------ affine group-64 mode

def _numpy_affine(w16):
    """The affine rule restated with numpy float32 arithmetic."""
    w = w16.view(np.float16).astype(np.float32)
    wmin, wmax = w.min(), w.max()
    side = abs(wmin) > abs(wmax)
    s = np.float32((wmax - wmin) / np.float32(255))
    s = s if s > np.float32(1e-7) else np.float32(1e-7)
    s = s if side else -s
    edge = wmin if side else wmax
    q0 = np.rint(np.float32(edge / s))
    bias = np.float32(0)
    if q0 != 0:
        s = np.float32(edge / q0)
        bias = edge
    q = np.minimum(np.rint((w - bias) / s), np.float32(255)).astype(np.uint8)
    return q, np.float16(s).view(np.uint16), np.float16(bias).view(np.uint16)


def test_affine_matches_restatement_and_invariants(oracle):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((300, 128)).astype(np.float32) * rng.choice([0.001, 1, 50], (300, 1)).astype(np.float32)
    x[:20, 5] = 0.0  # an exact zero in some groups
    bits = oracle.f32_to_f16_bits(x)
    q, s, b = oracle.quantize_mlx(bits, 0, 64)
    for r in range(0, 300, 7):
        for g in range(2):
            eq, es, eb = _numpy_affine(bits[r, 64 * g: 64 * (g + 1)])
            np.testing.assert_array_equal(q[r, 64 * g: 64 * (g + 1)], eq)
            assert s[r, g] == es and b[r, g] == eb
    sf = s.view(np.float16).astype(np.float64)
    bf = b.view(np.float16).astype(np.float64)
    w = bits.view(np.float16).astype(np.float64)
    deq = oracle.dequant_f64(q, s, b, 1)
    # half a step, plus the fp16 rounding of scale and bias (relative 2^-11,
    # or half the subnormal spacing 2^-25 when the scale is subnormal)
    ds = np.maximum(np.abs(sf) * 2.0**-11, 2.0**-25)
    db = np.maximum(np.abs(bf) * 2.0**-11, 2.0**-25)
    err = np.abs(deq - w)
    rnd = np.repeat(255 * ds + db + 1e-12, 64, axis=1)
    step = np.repeat(np.abs(sf), 64, axis=1)
    # interior codes round to the nearest grid point: half a step
    interior = (q > 0) & (q < 255)
    assert np.all(err[interior] <= 0.5 * step[interior] + rnd[interior])
    # the grid spans 255*|s| with |s| = |edge|/|q0|, which can fall short of
    # the group range by under one step, so a clamped end code is within a step
    assert np.all(err <= step + rnd)
    # the zero point is a grid point before the fp16 rounding of scale/bias:
    # 0 dequantizes to q0*ds + db at most
    assert np.all(np.abs(deq[:20, 5]) <= q[:20, 5] * ds[:20, 0] + db[:20, 0] + 1e-12)


# Pins of the affine rule's individual choices.  MLX's CPU affine quantize
# (mlx/backend/cpu/quantized.cpp, mlx 0.31 via mlx-swift 0.31.4; not in the
# reference tree) computes, per group, in binary32: the true min and max;
# scale = max((max - min) / 255, 1e-7), negated unless |min| > |max|; edge =
# min or max accordingly; q0 = rint(edge / scale); if q0 != 0 then
# scale = edge / q0 and bias = edge, else bias = 0; q = clamp(rint((w - bias)
# / scale), 0, 255); scale and bias stored in the input dtype (fp16 here).
# _affine_exact restates it with exact rationals and explicit binary32
# rounding of every operation; each _alt_* changes one choice.  The
# constructed groups below are ones where each alternative yields a
# different byte, with the expected bytes derived by hand in the comments.

from fractions import Fraction as _Fr


def _round_bin(x, mant_bits, emin):
    """x rounded to the nearest binary float with `mant_bits` significand
    bits and minimum normal exponent `emin` (ties to even), exactly."""
    if x == 0:
        return _Fr(0)
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if a < _Fr(2) ** e:
        e -= 1
    elif a >= _Fr(2) ** (e + 1):
        e += 1
    ulp = _Fr(2) ** (max(e, emin) - (mant_bits - 1))
    m = a / ulp
    fl = m.numerator // m.denominator
    r = m - fl
    if r > _Fr(1, 2) or (r == _Fr(1, 2) and fl % 2 == 1):
        fl += 1
    return (fl * ulp) if x > 0 else -(fl * ulp)


def _fl32(x):
    return _round_bin(x, 24, -126)


def _fl16(x):
    return _round_bin(x, 11, -14)


def _rint(x):
    fl = x.numerator // x.denominator
    r = x - fl
    return fl + 1 if r > _Fr(1, 2) or (r == _Fr(1, 2) and fl % 2 == 1) else fl


def _round_half_away(x):
    a = abs(x)
    n = (a + _Fr(1, 2)).numerator // (a + _Fr(1, 2)).denominator
    return n if x >= 0 else -n


_EPS32 = _fl32(_Fr(1, 10**7))


def _affine_exact(w, rnd=_rint, scale_for_q=None, recip=False, minmax=False):
    """One group (exact fp16 values as Fractions) -> (q list, scale, bias) as
    Fractions before the fp16 storage rounding."""
    mn, mx = min(w), max(w)
    s = max(_fl32(_fl32(mx - mn) / 255), _EPS32)
    if minmax:  # plain min/max affine: bias = min, positive scale
        bias = mn
    else:
        side = abs(mn) > abs(mx)
        s = s if side else -s
        edge = mn if side else mx
        q0 = rnd(_fl32(edge / s))
        bias = _Fr(0)
        if q0 != 0:
            s = _fl32(edge / q0)
            bias = edge
    sq = s if scale_for_q is None else scale_for_q(s)
    q = []
    for x in w:
        d = _fl32(x - bias)
        v = _fl32(d * _fl32(1 / sq)) if recip else _fl32(d / sq)
        q.append(min(max(rnd(v), 0), 255))
    return q, s, bias


def _alt_half_away(w):
    return _affine_exact(w, rnd=_round_half_away)


def _alt_fp16_scale(w):
    return _affine_exact(w, scale_for_q=_fl16)


def _alt_reciprocal(w):
    return _affine_exact(w, recip=True)


def _alt_minmax(w):
    return _affine_exact(w, minmax=True)


def _group(values, fill):
    """64 fp16 values: `values` then `fill` repeated (fp16 bits, exact Fractions)."""
    v = list(values) + [fill] * (64 - len(values))
    bits = np.array(v, np.float16).view(np.uint16)
    assert np.all(bits.view(np.float16).astype(np.float64) == np.array(v, np.float64)), "not fp16 values"
    return bits, [_Fr(float(x)) for x in bits.view(np.float16).astype(np.float64)]


def _f16_bits(x):
    return int(np.float16(float(_fl16(x))).view(np.uint16))


def _check_group(oracle, bits, w):
    q, s, b = oracle.quantize_mlx(bits.reshape(1, 64), 0, 64)
    eq, es, eb = _affine_exact(w)
    assert list(q[0]) == eq
    assert int(s[0, 0]) == _f16_bits(es) and int(b[0, 0]) == _f16_bits(eb)
    return list(q[0]), int(s[0, 0]), int(b[0, 0])


def test_affine_ties_round_half_to_even(oracle):
    # min 0, max 255: scale0 = 1, |0| > |255| is false so scale = -1, edge =
    # 255, q0 = -255, scale = 255 / -255 = -1, bias = 255; q = 255 - w.
    # w = 126.5 -> 128.5 exactly: rint gives 128, half-away 129.
    bits, w = _group([0.0, 255.0, 126.5, 125.5], 10.0)
    q, s, b = _check_group(oracle, bits, w)
    assert (q[0], q[1], q[2], q[3], q[4]) == (255, 0, 128, 130, 245)
    assert s == 0xBC00 and b == 0x5BF8  # fp16 -1 and 255
    assert _alt_half_away(w)[0][2] == 129


def test_affine_edge_sign_and_zero_point(oracle):
    # |max| >= |min| (max 8, min -4): scale = -(12/255) -> edge = 8, q0 =
    # rint(8 / -(12/255)) = -170, scale = 8 / -170 < 0, bias = 8:
    # q(8) = 0, q(-4) = 255, q(0) = 170 (zero sits on the grid).
    bits, w = _group([8.0, -4.0, 0.0, 2.0], 1.0)
    q, s, b = _check_group(oracle, bits, w)
    assert (q[0], q[1], q[2]) == (0, 255, 170)
    assert s & 0x8000 and b == 0x4800  # negative scale, bias fp16 8
    # plain min/max quantization maps the other way round
    mq = _alt_minmax(w)[0]
    assert (mq[0], mq[1]) == (255, 0)
    # |min| > |max| (min -8, max 4): positive scale, edge = -8 = bias
    bits, w = _group([-8.0, 4.0, 0.0], 1.0)
    q, s, b = _check_group(oracle, bits, w)
    assert (q[0], q[1], q[2]) == (0, 255, 170)
    assert not s & 0x8000 and b == 0xC800  # bias fp16 -8


def test_affine_constant_groups(oracle):
    # all zero: scale = max(0, 1e-7) negated (|0| > |0| is false), edge = 0,
    # q0 = 0 -> bias = 0; stored scale fp16(-1e-7) = -2 * 2^-24 (0x8002)
    bits, w = _group([], 0.0)
    q, s, b = _check_group(oracle, bits, w)
    assert q == [0] * 64 and s == 0x8002 and b == 0x0000
    # constant 3: q0 = rint(3 / -1e-7) = -3e7, scale = 3 / -3e7, bias = 3
    bits, w = _group([], 3.0)
    q, s, b = _check_group(oracle, bits, w)
    assert q == [0] * 64 and s == 0x8002 and b == 0x4200


def test_affine_quantizes_with_the_binary32_scale_and_divides(oracle):
    # min -7.62890625, max 4.33984375: edge = min, q0 = -255, scale =
    # -7.62890625 / -255 (binary32, not an fp16 value).  w = 0.023406982...
    # gives 164 with that scale and 163 with its fp16 rounding; w =
    # 3.814453125 gives 244 dividing and 245 multiplying by the reciprocal.
    bits, w = _group([-7.62890625, 4.33984375, 0.023406982421875, 3.814453125], 0.0)
    q, s, b = _check_group(oracle, bits, w)
    assert (q[0], q[1], q[2], q[3]) == (0, 255, 164, 244)
    assert _alt_fp16_scale(w)[0][2] == 163
    assert _alt_reciprocal(w)[0][3] == 245


def _affine_range16(w):
    """_affine_exact with the range max - min rounded to fp16 (the input
    dtype) before the / 255, as an op-by-op fp16 restatement computes it."""
    mn, mx = min(w), max(w)
    s = max(_fl32(_fl16(mx - mn) / 255), _EPS32)
    side = abs(mn) > abs(mx)
    s = s if side else -s
    edge = mn if side else mx
    q0 = _rint(_fl32(edge / s))
    bias = _Fr(0)
    if q0 != 0:
        s = _fl32(edge / q0)
        bias = edge
    return [min(max(_rint(_fl32(_fl32(x - bias) / s)), 0), 255) for x in w], s, bias


def test_affine_range_is_binary32_not_rounded_to_fp16(oracle):
    # min -3.38671875, max 1.591796875: max - min = 4.978515625 exactly in
    # binary32; in fp16 (spacing 2^-8 there) it is the tie 1274.5 ulps and
    # rounds to even, 4.9765625.  |min| > |max|, so edge = min and
    # q0 = rint(min / (range / 255)): -173.468.. -> -173 with the binary32
    # range, -173.536.. -> -174 with the fp16 one.  scale = min / q0 then
    # differs (0.0195764.. against 0.0194639..), and so do q(max) (254
    # against 255) and q(0) (173 against 174).
    bits, w = _group([-3.38671875, 1.591796875, 0.0], 0.0)
    q, s, b = _check_group(oracle, bits, w)
    assert (q[0], q[1], q[2]) == (0, 254, 173)
    assert b == 0xC2C6  # fp16 -3.38671875
    alt = _affine_range16(w)[0]
    assert (alt[0], alt[1], alt[2]) == (0, 255, 174)


def test_affine_matches_the_exact_restatement_on_random_groups(oracle):
    rng = np.random.default_rng(21)
    x = rng.standard_normal((240, 64)).astype(np.float32) * rng.choice([1e-4, 0.02, 1, 30], (240, 1)).astype(np.float32)
    x[:10, :] = np.abs(x[:10, :])     # one-signed groups
    x[10:20, :] = -np.abs(x[10:20, :])
    bits = oracle.f32_to_f16_bits(x)
    q, s, b = oracle.quantize_mlx(bits, 0, 64)
    wf = bits.view(np.float16).astype(np.float64)
    differs = {"half_away": 0, "fp16_scale": 0, "minmax": 0}
    for r in range(240):
        w = [_Fr(float(v)) for v in wf[r]]
        eq, es, eb = _affine_exact(w)
        assert list(q[r]) == eq, r
        assert int(s[r, 0]) == _f16_bits(es) and int(b[r, 0]) == _f16_bits(eb), r
        differs["fp16_scale"] += _alt_fp16_scale(w)[0] != eq
        differs["minmax"] += _alt_minmax(w)[0] != eq
        differs["half_away"] += _alt_half_away(w)[0] != eq
    # the scale-precision and sign choices show on ordinary data
    assert differs["fp16_scale"] > 0 and differs["minmax"] > 0, differs


def test_affine_bf16_input_is_cast_to_f16_first(oracle):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((10, 64)).astype(np.float32)
    b16 = oracle.f32_to_bf16_bits(x)
    f16 = oracle.bf16_bits_to_f32(b16).astype(np.float16).view(np.uint16)
    for a, c in zip(oracle.quantize_mlx(b16, 1), oracle.quantize_mlx(f16, 0)):
        np.testing.assert_array_equal(a, c)


# ------------------------------------------------------------- dequantizer

def test_dequant_ref_two_roundings_exhaustive_bytes(oracle):
    """f16(f16(f16(q)*s) + z) for every byte, against numpy float16 arithmetic."""
    rng = np.random.default_rng(7)
    q = np.tile(np.arange(256, dtype=np.uint8), (50, 1))
    s = (rng.uniform(1e-4, 1.0, (50, 1)).astype(np.float32)).astype(np.float16)
    z = (rng.standard_normal((50, 1)).astype(np.float32) * 10).astype(np.float16)
    got = oracle.dequant_ref_f16(q, s.view(np.uint16), z.view(np.uint16)).view(np.float16)
    want = (q.astype(np.float16) * s) + z   # two float16 roundings
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))
    # a fused multiply-add differs somewhere (the check has teeth)
    fused = (q.astype(np.float64) * s.astype(np.float64) + z.astype(np.float64)).astype(np.float16)
    assert np.any(fused.view(np.uint16) != want.view(np.uint16))


# -------------------------------------------------------------- attention

def _np_attention(q, k, v, limits, scale):
    out = np.zeros_like(q)
    for r in range(q.shape[0]):
        s = (k[: limits[r]] @ q[r]) * scale
        p = np.exp(s - s.max())
        out[r] = p @ v[: limits[r]] / p.sum()
    return out


def test_attention_closed_forms(oracle):
    rng = np.random.default_rng(8)
    D = 16
    v = rng.standard_normal((5, D))
    k = rng.standard_normal((5, D))
    q = rng.standard_normal((3, D))
    # one visible key -> that value row
    np.testing.assert_allclose(oracle.attention_f64(q, k, v, [1, 1, 1], 0.3), np.tile(v[0], (3, 1)), atol=1e-12)
    # identical keys -> mean of the values
    kk = np.tile(k[0], (5, 1))
    np.testing.assert_allclose(oracle.attention_f64(q, kk, v, [5, 5, 5], 0.3), np.tile(v.mean(0), (3, 1)),
                               atol=1e-12)
    # rows see different prefixes (causal limits); keys past the limit never matter
    lim = [2, 4, 5]
    k2 = k.copy()
    k2[4] = 1e6
    got = oracle.attention_f64(q, k2, v, [2, 4, 4], 0.3)
    np.testing.assert_allclose(got, _np_attention(q, k, v, [2, 4, 4], 0.3), atol=1e-12)
    np.testing.assert_allclose(oracle.attention_f64(q, k, v, lim, 0.3), _np_attention(q, k, v, lim, 0.3),
                               atol=1e-12)


def test_mlx_composed_attention_closed_forms(oracle):
    """One key: the output is that value row exactly (p = 1 in any dtype);
    equal keys: the mean of the values, within the output's rounding."""
    rng = np.random.default_rng(18)
    D = 64
    v16 = oracle.f32_to_f16_bits(rng.standard_normal((6, D)).astype(np.float32))
    k16 = oracle.f32_to_f16_bits(rng.standard_normal((6, D)).astype(np.float32))
    vf = oracle.f16_bits_to_f32(v16).astype(np.float64)
    for dt in (oracle.DT_F16, oracle.DT_BF16):
        qb = (oracle.f32_to_f16_bits if dt == oracle.DT_F16 else oracle.f32_to_bf16_bits)(
            rng.standard_normal((3, D)).astype(np.float32))
        one = oracle.attention_mlx_composed(qb, dt, k16, v16, [1, 1, 1], 0.125)
        np.testing.assert_array_equal(one, np.tile(vf[0], (3, 1)))
        same = np.tile(k16[0], (6, 1))
        mean = oracle.attention_mlx_composed(qb, dt, same, v16, [6, 6, 6], 0.125)
        tol = 2.0 ** -11 * np.abs(vf).max() * 2 if dt == oracle.DT_F16 else 1e-6
        np.testing.assert_allclose(mean, np.tile(vf.mean(0), (3, 1)), atol=tol)


def test_mlx_composed_attention_against_f64(oracle):
    """How far the reference's op-by-op SDPA sits from the exact result on
    N(0,1) data (T 2048, D 128, scale 1/sqrt(D)): with bf16 queries the
    query scaled and rounded to bf16 dominates (2^-9 relative per element),
    with fp16 queries the fp16 roundings of scores, weights and output add
    to it -- measurably off, but within the 2e-3 tolerance.  With the query
    scaling taken out (scale 1, queries pre-scaled exactly in float32 and
    exactly representable) the float32 form is within 1e-5."""
    rng = np.random.default_rng(19)
    T, D = 2048, 128
    k16 = oracle.f32_to_f16_bits(rng.standard_normal((T, D)).astype(np.float32))
    v16 = oracle.f32_to_f16_bits(rng.standard_normal((T, D)).astype(np.float32))
    qf = rng.standard_normal((8, D)).astype(np.float32)
    kd, vd = oracle.f16_bits_to_f32(k16), oracle.f16_bits_to_f32(v16)
    lim = [T, T - 1, 1000, 1, T, T, 64, 65]
    for dt, lo, hi in ((oracle.DT_BF16, 1e-5, 2e-3), (oracle.DT_F16, 1e-5, 2e-3)):
        qb = (oracle.f32_to_f16_bits if dt == oracle.DT_F16 else oracle.f32_to_bf16_bits)(qf)
        got = oracle.attention_mlx_composed(qb, dt, k16, v16, lim, 1 / np.sqrt(D))
        ref = oracle.attention_f64(oracle.bits_to_f32(qb, dt), kd, vd, lim, 1 / np.sqrt(D))
        err = np.abs(got - ref).max()
        assert lo <= err <= hi, (dt, err)
    # bf16 queries already scaled: scale 1 rounds nothing, the rest is float32
    qb = oracle.f32_to_bf16_bits(qf * np.float32(1 / np.sqrt(D)))
    got = oracle.attention_mlx_composed(qb, oracle.DT_BF16, k16, v16, lim, 1.0)
    ref = oracle.attention_f64(oracle.bits_to_f32(qb, oracle.DT_BF16), kd, vd, lim, 1.0)
    assert np.abs(got - ref).max() <= 1e-5


def test_masked_minus_10000_underflows_to_zero():
    """BatchedDecode.swift:22-28: exp(score - 10000) is 0 in f16, bf16, f32,
    so a length bound equals the reference's additive mask."""
    for dt in (np.float16, np.float32):
        assert np.exp(np.array(5.0 - 10000.0, dt)) == 0


# ------------------------------------------------------- stack and prefix

def test_stack_left_padded_closed_form(oracle):
    rows_q = [np.arange(2 * 1 * 3, dtype=np.uint8).reshape(2, 1, 3), (10 + np.arange(2 * 3 * 3)).astype(np.uint8).reshape(2, 3, 3)]
    rows_s = [np.full((2, 1, 1), 7, np.uint16), np.full((2, 3, 1), 9, np.uint16)]
    rows_z = [np.full((2, 1, 1), 1, np.uint16), np.full((2, 3, 1), 2, np.uint16)]
    q, s, z = oracle.stack_left_padded(rows_q, rows_s, rows_z, [1, 3])
    assert q.shape == (2, 2, 3, 3)
    assert q[0, 0].tolist() == [[0, 0, 0], [0, 0, 0], [0, 1, 2]]
    assert q[0, 1].tolist() == [[0, 0, 0], [0, 0, 0], [3, 4, 5]]
    assert q[1, 0].tolist() == [[10, 11, 12], [13, 14, 15], [16, 17, 18]]
    assert s[0, 0, :, 0].tolist() == [0, 0, 7] and z[0, 1, :, 0].tolist() == [0, 0, 1]


def test_fnv1a64_published_vectors(oracle):
    assert oracle.fnv1a64(b"") == 0xCBF29CE484222325
    assert oracle.fnv1a64(b"a") == 0xAF63DC4C8601EC8C
    assert oracle.fnv1a64(b"foobar") == 0x85944171F73967E8


def test_prefix_key_layout(oracle):
    """cacheKey bytes: 3, tag, model, FF, media, FF, tokens as 8-byte LE."""
    toks = [1, 258, -1]
    data = bytes([3, 2]) + b"m" + b"\xff" + b"img" + b"\xff" + b"".join(int(t).to_bytes(8, "little", signed=True) for t in toks)
    assert oracle.prefix_key("m", "img", 2, toks) == oracle.fnv1a64(data)
    assert oracle.prefix_key("m", None, 2, toks) == oracle.prefix_key("m", "", 2, toks)
    assert oracle.prefix_key("m", None, 1, toks) != oracle.prefix_key("m", None, 2, toks)


def test_common_prefix_length_reference_vectors(oracle):
    """PrefixCacheTests.swift:244-250."""
    cpl = oracle.common_prefix_length
    assert cpl([1, 2, 3, 4], [1, 2, 3, 4]) == 4
    assert cpl([1, 2, 3, 9], [1, 2, 3, 4]) == 3
    assert cpl([1, 2], [1, 2, 3, 4]) == 2
    assert cpl([9, 1], [1, 2]) == 0
    assert cpl([], [1]) == 0


# ---------------------------------------------------------------- RoPE rows
def _rope_table(max_pos, D, base=10000.0):
    from krill_amd.pool import rope_table

    return rope_table(max_pos, D, base)


def _bits(oracle, rng, shape, dt):
    x = rng.standard_normal(shape).astype(np.float32)
    return oracle.f32_to_bf16_bits(x) if dt == oracle.DT_BF16 else oracle.f32_to_f16_bits(x)


@pytest.mark.parametrize("bf16", [True, False])
def test_rope_position_zero_is_identity_and_quarter_turn_swaps(oracle, bf16):
    dt = oracle.DT_BF16 if bf16 else oracle.DT_F16
    rng = np.random.default_rng(3)
    D = 64
    x = _bits(oracle, rng, (5, D), dt)
    tab = _rope_table(4, D)
    assert np.array_equal(oracle.rope_rows(x, dt, np.zeros(5, np.int64), tab), x)
    quarter = np.concatenate([np.zeros((1, D // 2), np.float32), np.ones((1, D // 2), np.float32)], axis=1)
    y = oracle.rope_rows(x, dt, np.zeros(5, np.int64), quarter)
    xf, yf = oracle.bits_to_f32(x, dt), oracle.bits_to_f32(y, dt)
    np.testing.assert_array_equal(yf[:, : D // 2], -xf[:, D // 2:])
    np.testing.assert_array_equal(yf[:, D // 2:], xf[:, : D // 2])


@pytest.mark.parametrize("bf16", [True, False])
def test_rope_matches_float64_pair_rotation(oracle, bf16):
    dt = oracle.DT_BF16 if bf16 else oracle.DT_F16
    rng = np.random.default_rng(4)
    D, P = 128, 300
    x = _bits(oracle, rng, (P, D), dt)
    pos = rng.integers(0, 4096, P)
    tab = _rope_table(4096, D)
    got = oracle.bits_to_f32(oracle.rope_rows(x, dt, pos, tab), dt).astype(np.float64)
    xf = oracle.bits_to_f32(x, dt).astype(np.float64)
    h = D // 2
    ang = pos[:, None] * (10000.0 ** (-2.0 * np.arange(h) / D))[None, :]
    c, s = np.cos(ang), np.sin(ang)
    want = np.concatenate([xf[:, :h] * c - xf[:, h:] * s, xf[:, :h] * s + xf[:, h:] * c], axis=1)
    ulp = 2.0 ** -8 if bf16 else 2.0 ** -11
    # one rounding to the element dtype on top of the float32 steps and the table's rounding
    tol = ulp * np.abs(want) + 1e-6 * (np.abs(xf).max(axis=1, keepdims=True) + 1)
    assert np.all(np.abs(got - want) <= tol)
    n0 = np.hypot(xf[:, :h], xf[:, h:])
    n1 = np.hypot(got[:, :h], got[:, h:])
    assert np.all(np.abs(n1 - n0) <= 2 * ulp * n0 + 1e-6)


def test_rope_turns_compose(oracle):
    rng = np.random.default_rng(5)
    D, dt = 64, oracle.DT_F16
    x = _bits(oracle, rng, (50, D), dt)
    tab = _rope_table(64, D)
    twice = oracle.rope_rows(oracle.rope_rows(x, dt, np.full(50, 17), tab), dt, np.full(50, 23), tab)
    direct = oracle.rope_rows(x, dt, np.full(50, 40), tab)
    a, b = oracle.bits_to_f32(twice, dt), oracle.bits_to_f32(direct, dt)
    assert np.abs(a - b).max() <= 4 * 2.0 ** -11 * np.abs(b).max()


# ---- sliding-window layers: pins from the reference's own tests

def _visible(rows, k_total):
    return [[k for k in range(k_total) if lo <= k < hi] for lo, hi in rows]


def test_sliding_window_rows_reference_mask_vectors(oracle):
    # SlidingWindowMaskTests.swift:17-30: newLen 4, cacheLen 0, window 2
    assert _visible(oracle.sliding_window_rows(4, 0, 2), 4) == [[0], [0, 1], [1, 2], [2, 3]]
    # :32-43: total 3 <= window 10 -> the plain causal mask
    assert _visible(oracle.sliding_window_rows(3, 0, 10), 3) == [[0], [0, 1], [0, 1, 2]]
    # :45-53: newLen 1, cacheLen 600, window 512: keys 89..600, exactly 512 visible
    (row,) = _visible(oracle.sliding_window_rows(1, 600, 512), 601)
    assert row[0] == 89 and row[-1] == 600 and len(row) == 512 and 88 not in row


def test_attention_window_against_masked_softmax(oracle):
    rng = np.random.default_rng(3)
    T, D = 23, 8
    q, k, v = rng.standard_normal((5, D)), rng.standard_normal((T, D)), rng.standard_normal((T, D))
    lo, hi = [0, 4, 9, 17, 22], [3, 12, 20, 23, 23]
    got = oracle.attention_window_f64(q, k, v, lo, hi, 0.3)
    s = q @ k.T * 0.3
    mask = np.array([[lo[r] <= t < hi[r] for t in range(T)] for r in range(5)])
    s = np.where(mask, s, -np.inf)
    p = np.exp(s - s.max(axis=1, keepdims=True))
    want = (p / p.sum(axis=1, keepdims=True)) @ v
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    # a one-key window is that key's value row
    np.testing.assert_allclose(oracle.attention_window_f64(q[:1], k, v, [7], [8], 1.0)[0], v[7], rtol=0, atol=1e-15)


def test_rotating_retained_start_reference_vectors(oracle):
    # RotatingKVCacheTests.swift:115-131: window 4, ten single appends keep the
    # last min(t + 1, 4) tokens
    for t in range(10):
        total, start = oracle.rotating_retained_start([("append", 1)] * (t + 1), 4)
        assert total == t + 1 and total - start == min(t + 1, 4)
    # :133-161: truncate to 8 keeps 6, 7; one more append keeps 6, 7, 8
    ops = [("append", 1)] * 10
    assert oracle.rotating_retained_start(ops + [("truncate", 8)], 4) == (8, 6)
    assert oracle.rotating_retained_start(ops + [("truncate", 8), ("append", 1)], 4) == (9, 6)
    assert oracle.rotating_retained_start(ops + [("truncate", 6)], 4) == (6, 6)
    with pytest.raises(ValueError):
        oracle.rotating_retained_start(ops + [("truncate", 5)], 4)
    # chunked appends (RotatingKVCacheTests.swift:77-113): retained before each
    # append is min(retained, window - 1)
    total, start = oracle.rotating_retained_start([("append", L) for L in (5, 3, 12, 1, 9, 6)], 8)
    assert (total, total - start) == (36, 7 + 6)


# -------------------------------------------------------------- CPU baseline

@pytest.mark.parametrize("dtname", ["bf16", "f16"])
def test_cpu_baseline_step_is_the_composed_sdpa(oracle, dtname):
    """The timed CPU baseline (the reference's step restated in C: row
    quantize, concat, full fp16 dequant, SDPA as MLX's composed ops) against
    the row quantizer, the dequantizer and attention_mlx_composed, over two
    steps from an empty cache (one key, then two)."""
    B, Hkv, Hq, D = 2, 2, 4, 64
    R = Hq // Hkv
    dt = oracle.DT_BF16 if dtname == "bf16" else oracle.DT_F16
    rng = np.random.default_rng(40 + dt)
    base = oracle.Baseline(1, B, Hkv, Hq, D, np.zeros(B, np.int32), seed=1)
    mk = oracle.f32_to_bf16_bits if dt == oracle.DT_BF16 else oracle.f32_to_f16_bits
    ks, vs = [], []
    scale = 1.0 / np.sqrt(D)
    for step in range(2):
        q = mk(rng.standard_normal((1, B, Hq, D)).astype(np.float32))
        k = mk(rng.standard_normal((1, B, Hkv, D)).astype(np.float32))
        v = mk(rng.standard_normal((1, B, Hkv, D)).astype(np.float32))
        ks.append(k[0])
        vs.append(v[0])
        out = np.empty((1, B, Hq, D), np.float32)
        base.step(q, k, v, dt, scale, out)
        for b in range(B):
            for hk in range(Hkv):
                kr = np.stack([x[b, hk] for x in ks])  # [T, D] bits
                vr = np.stack([x[b, hk] for x in vs])
                kf16 = oracle.dequant_ref_f16(*oracle.quantize(kr, dt, 0))
                vf16 = oracle.dequant_ref_f16(*oracle.quantize(vr, dt, 0))
                qr = q[0, b, hk * R:(hk + 1) * R]
                want = oracle.attention_mlx_composed(qr, dt, kf16, vf16, [step + 1] * R, scale)
                got = out[0, b, hk * R:(hk + 1) * R].astype(np.float64)
                if step == 0:  # one key: the value row exactly
                    np.testing.assert_array_equal(got, want)
                np.testing.assert_allclose(got, want, rtol=2e-3 if dt == oracle.DT_F16 else 1e-5, atol=1e-6)
    base.close()
