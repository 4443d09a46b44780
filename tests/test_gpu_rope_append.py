"""GPU: RoPE fused into the quantize-append (krill_quantize_append_rope)
against the oracle: K rows rotated by oracle.rope_rows (float32 steps, one
rounding to the element dtype) and quantized, V quantized as is; the pool
bytes must be identical, bit for bit, on the per-row kernel (short appends)
and the bulk kernel (>= 32 rows).  A row whose position lies outside the
table is not written."""
import numpy as np
import pytest

from kvutil import DT, MODE, i32, rand_bits, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd.pool import rope_table  # noqa: E402


def _case(mode, dt, D, L, seed, H=2, B=3, max_pos=5000, bad_row=None):
    rng = np.random.default_rng(seed)
    blocks = B * ((L + 63) // 64 + 1) + 4
    pool = krill_amd.KVPool(1, H, D, blocks, mode, dt, free_list_seed=seed)
    seqs = [pool.seq_create() for _ in range(B)]
    slots = np.stack([pool.reserve_append(s, L) for s in seqs]).astype(np.int32)
    k = rand_bits(rng, (B, H, L, D), dt, scale=3.0)
    v = rand_bits(rng, (B, H, L, D), dt)
    start = rng.integers(0, max_pos - L, B)
    pos = (start[:, None] + np.arange(L)[None, :]).astype(np.int32)
    if bad_row is not None:
        # first write other rows everywhere, then the RoPE append with one row out of the table
        k0 = rand_bits(rng, (B, H, L, D), dt)
        pool.quantize_append(0, to_dev(k0, dt), to_dev(k0, dt), i32(slots))
        pos[bad_row] = max_pos
    tab = rope_table(max_pos, D)
    pool.quantize_append_rope(0, to_dev(k, dt), to_dev(v, dt), i32(slots), i32(pos),
                              torch.from_numpy(tab).cuda())
    mb = (L + 63) // 64 + 1
    t, n = pool.batch_tables(seqs, mb)
    snap = {kk: vv.cpu().numpy() for kk, vv in pool.gather(0, i32(t), i32(n), L).items()}
    return pool, k, v, pos, tab, snap, (k0 if bad_row is not None else None)


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
@pytest.mark.parametrize("D", [64, 128, 256, 512])
@pytest.mark.parametrize("L", [1, 5, 70])
def test_rope_append_bit_exact(mode, D, L):
    dt = "bf16"
    print(f"\ncase rope_append mode={mode} D={D} L={L}", flush=True)
    pool, k, v, pos, tab, snap, _ = _case(mode, dt, D, L, seed=D + L)
    B, H = k.shape[:2]
    kr = O.rope_rows(k, DT[dt], np.broadcast_to(pos[:, None, :], (B, H, L)), tab)
    kq, ks, kz = O.quantize(kr, DT[dt], MODE[mode])
    vq, vs, vz = O.quantize(v, DT[dt], MODE[mode])
    np.testing.assert_array_equal(snap["keys"], kq)
    np.testing.assert_array_equal(snap["key_scales"].view(np.uint16), ks)
    np.testing.assert_array_equal(snap["key_zeros"].view(np.uint16), kz)
    np.testing.assert_array_equal(snap["values"], vq)
    np.testing.assert_array_equal(snap["value_scales"].view(np.uint16), vs)
    np.testing.assert_array_equal(snap["value_zeros"].view(np.uint16), vz)
    pool.close()


@pytest.mark.parametrize("L", [4, 40])
def test_rope_append_f16_and_position_outside_table(L):
    dt, mode, D = "f16", "affine_g64", 128
    print(f"\ncase rope_append_bad_pos L={L}", flush=True)
    pool, k, v, pos, tab, snap, k0 = _case(mode, dt, D, L, seed=7 + L, bad_row=1)
    B, H = k.shape[:2]
    pos_ok = np.minimum(pos, tab.shape[0] - 1)
    kr = O.rope_rows(k, DT[dt], np.broadcast_to(pos_ok[:, None, :], (B, H, L)), tab)
    kq, _, _ = O.quantize(kr, DT[dt], MODE[mode])
    vq, _, _ = O.quantize(v, DT[dt], MODE[mode])
    k0q, _, _ = O.quantize(k0, DT[dt], MODE[mode])
    for b in range(B):
        want_k, want_v = (k0q[b], k0q[b]) if b == 1 else (kq[b], vq[b])
        np.testing.assert_array_equal(snap["keys"][b], want_k)
        np.testing.assert_array_equal(snap["values"][b], want_v)
    pool.close()
