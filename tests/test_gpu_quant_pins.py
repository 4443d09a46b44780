"""GPU: the quantizers' pinned cases through the append kernels.

The groups that pin the affine quantizer in the oracle's own tests (exact
ties, the sign of the scale and its edge, constant groups, the binary32
range and scale, and the division where a reciprocal multiply gives another
byte) and ladders
of exact half-integer quotients, as the K and V rows of a 64-row launch (the
block kernel, whose per-element division takes a reciprocal wherever that
cannot change the byte) and of one-row launches (the row kernel), in both
storage modes, head_dim 64 and 128.  The pool's bytes must equal the
oracle's quantization of the same rows."""
import numpy as np
import pytest

from kvutil import DT, MODE, Filled, check_snapshot, i32, to_dev

from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402


def _group(values, fill):
    v = list(values) + [fill] * (64 - len(values))
    return np.array(v, np.float32)


def _pinned_groups():
    g = [
        _group([0.0, 255.0, 126.5, 125.5], 10.0),  # ties round half to even
        _group([8.0, -4.0, 0.0, 2.0], 1.0),  # |max| >= |min|: negative scale, bias = max
        _group([-8.0, 4.0, 0.0], 1.0),  # |min| > |max|: positive scale, bias = min
        _group([], 0.0),  # constant 0
        _group([], 3.0),  # constant 3
        # binary32 scale; 3.814453125 gives 244 dividing, 245 by the reciprocal
        _group([-7.62890625, 4.33984375, 0.023406982421875, 3.814453125], 0.0),
        # (w - 255) / -1 = 254.5 - k: an exact tie in every element
        _group([0.0, 255.0] + [k + 0.5 for k in range(62)], 0.0),
        # (w - 127.5) / -0.5 = 254.5 - k: ties again, with another scale
        _group([0.0, 127.5] + [k / 2 + 0.25 for k in range(62)], 0.0),
        # the range max - min in binary32 (an fp16 rounding of it changes q0)
        _group([-3.38671875, 1.591796875, 0.0], 0.0),
    ]
    return np.stack(g)


def _rows(rng, n, D):
    """n rows of D values: pinned groups (a random one per 64-value group,
    sometimes negated or scaled by a power of two) and random rows."""
    pins = _pinned_groups()
    out = np.empty((n, D), np.float32)
    for r in range(n):
        if r % 4 == 3:
            x = rng.standard_normal(D).astype(np.float32) * np.float32(rng.choice([1e-3, 1.0, 30.0]))
            out[r] = x.astype(np.float16).astype(np.float32)
            continue
        for g in range(D // 64):
            grp = pins[rng.integers(len(pins))] * rng.choice([1.0, -1.0, 0.25, 4.0])
            out[r, 64 * g:64 * (g + 1)] = rng.permutation(grp)
    return out


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D", [64, 128])
def test_pinned_groups_through_block_and_row_kernels(mode, D):
    print(f"\ncase quant_pins mode={mode} D={D}", flush=True)
    rng = np.random.default_rng(31 + D)
    H, T, dt = 2, 128, "f16"
    pool = krill_amd.KVPool(1, H, D, 16, mode, dt, free_list_seed=5)
    kx = np.stack([_rows(rng, T, D) for _ in range(H)])
    vx = np.stack([_rows(rng, T, D) for _ in range(H)])
    kb, vb = O.f32_to_f16_bits(kx), O.f32_to_f16_bits(vx)
    assert np.array_equal(O.bits_to_f32(kb, DT[dt]), kx), "pinned values must be fp16-exact"
    # sequence 0: two 64-row launches (block kernel); sequence 1: one row per launch (row kernel)
    s0, s1 = pool.seq_create(), pool.seq_create()
    for c in range(T // 64):
        slots = pool.reserve_append(s0, 64)
        rows = slice(64 * c, 64 * c + 64)
        pool.quantize_append(0, to_dev(kb[None, :, rows], dt), to_dev(vb[None, :, rows], dt), i32(slots[None]))
    for t in range(T):
        slots = pool.reserve_append(s1, 1)
        pool.quantize_append(0, to_dev(kb[None, :, t:t + 1], dt), to_dev(vb[None, :, t:t + 1], dt),
                             i32(slots[None]))
    torch.cuda.synchronize()
    f = Filled.__new__(Filled)
    f.pool, f.lens, f.dt, f.layers, f.seqs = pool, [T, T], dt, (0,), [s0, s1]
    f.k = {0: [kb, kb]}
    f.v = {0: [vb, vb]}
    t_, n_ = pool.batch_tables(f.seqs, T // 64)
    snap = pool.gather(0, i32(t_), i32(n_), T)
    kq, ks, kz, vq, vs, vz = f.expected(0, 0)
    for b, kernel in enumerate(("block", "row")):
        for name, want in (("keys", kq), ("values", vq), ("key_scales", ks), ("value_scales", vs)):
            got = snap[name][b].cpu().numpy()
            got = got.view(np.uint16) if got.dtype != np.uint8 else got
            bad = np.argwhere(got != want)
            if len(bad):
                h, tk, c = bad[0]
                src = kx if name.startswith("key") else vx
                print(f"{kernel} kernel {name}: {len(bad)} differ, first head {h} token {tk} col {c}: got {got[h, tk, c]} "
                      f"want {want[h, tk, c]}; row min {src[h, tk].min()} max {src[h, tk].max()} value "
                      f"{src[h, tk, c] if name in ('keys', 'values') else ''}", flush=True)
            assert not len(bad), f"{kernel} kernel {name}"
    check_snapshot(snap, f, 0)
    # the ties really are ties for the oracle: its bytes follow half to even
    if mode == "affine_g64":
        q, _, _ = O.quantize(O.f32_to_f16_bits(_pinned_groups()[6:7]), DT[dt], MODE[mode])
        assert q[0, 2] == 254 and q[0, 3] == 254  # 254.5 -> 254, 253.5 -> 254
    pool.close()
