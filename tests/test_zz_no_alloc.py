"""GPU: krill_decode_append_attention_noalloc, the decode step whose split-K
partials go to the library's static device scratch instead of a caller
workspace, against krill_decode_append_attention on a twin pool: the
attention output and the pool bytes must be identical, bit for bit, on two
steps in a row, the second over fewer and shorter sequences (the scratch
keeps the first step's partials).  A step whose workspace exceeds the
scratch is refused before any launch."""
import ctypes

import numpy as np
import pytest

from kvutil import Filled, i32, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd import _lib as L  # noqa: E402

SCRATCH_BYTES = 32 << 20  # KRILL_NOALLOC_SCRATCH_BYTES


def _noalloc(pool, layer, q, kn, vn, tables, lens, max_len, scale, out):
    B, Hq, _, D = q.shape
    H = pool.num_kv_heads
    return L.lib().krill_decode_append_attention_noalloc(
        pool.handle, layer, q.data_ptr(), kn.data_ptr(), vn.data_ptr(), H * D, D, tables.data_ptr(),
        lens.data_ptr(), B, tables.shape[1], max_len, Hq, float(scale), out.data_ptr(), L.DTYPE_F32,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))


def _step(pools, fills, idx, rng, dt, R, layer=0):
    """One decode step of sequences `idx` on both pools: the workspace entry
    point on pools[0], the static-scratch one on pools[1]; returns both
    outputs and the tables/lengths after the step."""
    H, D = pools[0].num_kv_heads, pools[0].head_dim
    B = len(idx)
    kn = rand_bits(rng, (B, H, 1, D), dt)
    vn = rand_bits(rng, (B, H, 1, D), dt)
    q = rand_bits(rng, (B, H * R, 1, D), dt)
    for p, f in zip(pools, fills):
        for b in idx:
            p.reserve_append(f.seqs[b], 1)
            f.lens[b] += 1
    seqs = [[f.seqs[b] for b in idx] for f in fills]
    full = [fills[0].lens[b] for b in idx]
    mb = max((T + 63) // 64 for T in full)
    tabs = [p.batch_tables(s, mb)[0] for p, s in zip(pools, seqs)]
    np.testing.assert_array_equal(tabs[0], tabs[1])
    tables, tl = i32(tabs[0]), i32(np.array(full, np.int32))
    qd, kd, vd = to_dev(q, dt), to_dev(kn, dt), to_dev(vn, dt)
    scale = 1.0 / np.sqrt(D)
    out_ws = pools[0].decode_append_attention(layer, qd, kd, vd, tables, tl, max(full), scale)
    out_na = torch.full((B, H * R, 1, D), float("nan"), dtype=torch.float32, device="cuda")
    L.check(_noalloc(pools[1], layer, qd, kd, vd, tables, tl, max(full), scale, out_na))
    torch.cuda.synchronize()
    return out_ws, out_na, tables, full


def _same_pool_bytes(pools, tables, full, layer=0):
    S = max(full)
    snaps = [p.gather(layer, tables, i32(np.array(full, np.int32)), S) for p in pools]
    for name in snaps[0]:
        a, b = snaps[0][name].cpu().numpy(), snaps[1][name].cpu().numpy()
        assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), f"pool {name} differs"


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_noalloc_step_matches_the_workspace_entry_point(mode):
    """Qwen3-14B heads (40 query / 8 KV, D 128): a first step over five
    sequences of 512 to 8192 tokens (many split partials), then a second
    step over two of them only."""
    print(f"\ncase noalloc mode={mode}", flush=True)
    dt, H, R, D = "bf16", 8, 5, 128
    prefill = [511, 1999, 4095, 64, 8191]
    blocks = sum((T + 130) // 64 for T in prefill) + 8
    pools, fills = [], []
    for _ in range(2):
        p = krill_amd.KVPool(1, H, D, blocks, mode, dt, free_list_seed=7)
        fills.append(Filled(p, prefill, np.random.default_rng(77), dt))
        pools.append(p)
    for b in range(len(prefill)):
        assert fills[0].seqs[b] == fills[1].seqs[b]
    need = pools[1].workspace_size(len(prefill), H * R, 1, max(prefill) + 1)
    assert 0 < need <= SCRATCH_BYTES
    rng = np.random.default_rng(78)
    # first call: all five sequences
    out_ws, out_na, tables, full = _step(pools, fills, [0, 1, 2, 3, 4], rng, dt, R)
    assert torch.equal(out_ws, out_na), "first step: output differs from the workspace entry point"
    _same_pool_bytes(pools, tables, full)
    # second call, smaller: two sequences, fewer partials than the first left in the scratch
    out_ws, out_na, tables, full = _step(pools, fills, [3, 1], rng, dt, R)
    assert out_na.shape[0] == 2
    assert torch.equal(out_ws, out_na), "second step: output differs from the workspace entry point"
    _same_pool_bytes(pools, tables, full)
    for p in pools:
        p.close()


def test_noalloc_refuses_a_step_beyond_the_scratch():
    """Short sequences in a batch large enough that the step's workspace
    exceeds the scratch: KRILL_E_RANGE before any launch, the output left as
    it was."""
    print("\ncase noalloc refuse", flush=True)
    dt, H, R, D = "bf16", 8, 5, 128
    pool = krill_amd.KVPool(1, H, D, 64, "affine_g64", dt, free_list_seed=3)
    B = 1024
    while pool.workspace_size(B, H * R, 1, 1) <= SCRATCH_BYTES:
        B += 256
    pool.close()
    pool = krill_amd.KVPool(1, H, D, B + 8, "affine_g64", dt, free_list_seed=3)
    seqs = [pool.seq_create() for _ in range(B)]
    for s in seqs:
        pool.reserve_append(s, 1)
    t, n = pool.batch_tables(seqs, 1)
    tables, tl = i32(t), i32(n)
    rng = np.random.default_rng(5)
    q = to_dev(rand_bits(rng, (B, H * R, 1, D), dt), dt)
    kn = to_dev(rand_bits(rng, (B, H, 1, D), dt), dt)
    vn = to_dev(rand_bits(rng, (B, H, 1, D), dt), dt)
    out = torch.zeros((B, H * R, 1, D), dtype=torch.float32, device="cuda")
    rc = _noalloc(pool, 0, q, kn, vn, tables, tl, 1, 1.0 / np.sqrt(D), out)
    torch.cuda.synchronize()
    assert rc == L.KRILL_E_RANGE, rc
    assert "static scratch" in L.last_error()
    assert not out.any()
    pool.close()
