"""GPU: the reference-shaped cache API (krill_amd.cache) and the KrillKernels
registry (krill_amd.kernels), driven through the sequences of the
reference's cache tests (Tests/KrillCoreTests/KVCacheTests.swift:54-331)
with int8 caches, against the oracle.

The reference's tests feed tiny ramps to the fp16 KVCache; here the same
call sequences run on PagedQuantizedKVCache with head_dim 64 rows, and every
dequantized snapshot must equal the oracle's quantize + dequantize of the
rows the sequence should hold (bit-exact fp16), every quantized snapshot
the oracle's bytes."""
import numpy as np
import pytest

from kvutil import DT, MODE, i32, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd import KrillKernels, make_quantized_kv_caches  # noqa: E402
from oracle import oracle as O  # noqa: E402

H, D = 2, 64
CASES = [("ref_row", "f16"), ("affine_g64", "bf16")]


def _pool(mode, dt, layers=1, blocks=64, heads=H):
    return krill_amd.KVPool(layers, heads, D, blocks, mode, dt, free_list_seed=9)


def _deq(rows, mode, dt):
    """Oracle fp16 bits of rows [H, T, D] after quantize + dequantize."""
    q, s, z = O.quantize(rows, DT[dt], MODE[mode])
    if mode == "ref_row":
        return O.dequant_ref_f16(q, s, z)
    return O.f32_to_f16_bits(O.dequant_f64(q, s, z, 1))


def _bits(t):
    return t.cpu().numpy().view(np.uint16)


def _check(result, krows, vrows, mode, dt):
    """(keys, values) fp16 [1, H, T, D] equal the oracle of rows [H, T, D]."""
    k, v = result
    assert tuple(k.shape) == (1, krows.shape[0], krows.shape[1], D)
    np.testing.assert_array_equal(_bits(k)[0], _deq(krows, mode, dt))
    np.testing.assert_array_equal(_bits(v)[0], _deq(vrows, mode, dt))


class _Rows:
    """Seeded K/V rows and the device tensors update() takes."""

    def __init__(self, seed, dt, heads=H):
        self.rng, self.dt, self.heads = np.random.default_rng(seed), dt, heads

    def take(self, L):
        k = rand_bits(self.rng, (1, self.heads, L, D), self.dt)
        v = rand_bits(self.rng, (1, self.heads, L, D), self.dt)
        return k, v, to_dev(k, self.dt), to_dev(v, self.dt)


@pytest.mark.parametrize("mode,dt", CASES)
def test_update_concatenates_along_sequence_axis(mode, dt):
    print(f"\ncase cache_api concat {mode}", flush=True)
    pool = _pool(mode, dt)
    cache = make_quantized_kv_caches(pool)[0]
    r = _Rows(1, dt)
    k1, v1, dk, dv = r.take(1)
    first = cache.update(dk, dv)
    _check(first, k1[0], v1[0], mode, dt)
    k2, v2, dk, dv = r.take(2)
    res = cache.update(dk, dv)
    assert cache.sequence_length == 3
    _check(res, np.concatenate([k1[0], k2[0]], 1), np.concatenate([v1[0], v2[0]], 1), mode, dt)
    snap = cache.snapshot()
    _check(snap, np.concatenate([k1[0], k2[0]], 1), np.concatenate([v1[0], v2[0]], 1), mode, dt)
    assert cache.memory_size_bytes == 2 * 3 * H * D + 4 * 3 * H * pool.groups * 2
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_restore_overwrites_state_and_sets_sequence_length(mode, dt):
    print(f"\ncase cache_api restore {mode}", flush=True)
    pool = _pool(mode, dt, layers=2)
    src = make_quantized_kv_caches(pool)
    r = _Rows(2, dt)
    ks, vs, dk, dv = r.take(2)
    for c in src:
        c.update(dk, dv)
    snap = src[0].quantized_snapshot()
    assert snap.sequence_length == 2
    dst = make_quantized_kv_caches(pool)
    k4, v4, dk4, dv4 = r.take(4)
    k4b, v4b, dk4b, dv4b = r.take(4)
    dst[0].update(dk4, dv4)
    dst[1].update(dk4b, dv4b)
    dst[0].restore_quantized(snap)
    assert dst[0].sequence_length == 2
    _check(dst[0].snapshot(), ks[0], vs[0], mode, dt)
    # the other layer keeps its four tokens (restore replaces one layer's arrays)
    assert dst[1].sequence_length == 4
    _check(dst[1].snapshot(), k4b[0], v4b[0], mode, dt)
    # both layers restored: the sequence releases the positions beyond them
    dst[1].restore_quantized(src[1].quantized_snapshot())
    assert dst[0].s.length == 2 and dst[1].sequence_length == 2
    _check(dst[1].snapshot(), ks[0], vs[0], mode, dt)
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_truncate_slices_sequence_axis_and_beyond_length_is_noop(mode, dt):
    print(f"\ncase cache_api truncate {mode}", flush=True)
    pool = _pool(mode, dt)
    cache = make_quantized_kv_caches(pool)[0]
    k, v, dk, dv = _Rows(3, dt).take(4)
    cache.update(dk, dv)
    cache.truncate(3)
    assert cache.sequence_length == 3
    _check(cache.snapshot(), k[0, :, :3], v[0, :, :3], mode, dt)
    before = [_bits(t) for t in cache.snapshot()]
    cache.truncate(6)
    cache.truncate(-1)
    assert cache.sequence_length == 3
    after = [_bits(t) for t in cache.snapshot()]
    for a, b in zip(before, after):
        np.testing.assert_array_equal(a, b)
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_reset_after_update_clears_state(mode, dt):
    print(f"\ncase cache_api reset {mode}", flush=True)
    pool = _pool(mode, dt)
    cache = make_quantized_kv_caches(pool)[0]
    _, _, dk, dv = _Rows(4, dt).take(2)
    cache.update(dk, dv)
    used = pool.stats()["blocks_used"]
    cache.reset()
    assert cache.sequence_length == 0
    assert cache.snapshot() is None and cache.quantized_snapshot() is None
    assert pool.stats()["blocks_used"] == used - 1
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_update_after_restore_concatenates(mode, dt):
    print(f"\ncase cache_api restore_then_update {mode}", flush=True)
    pool = _pool(mode, dt)
    r = _Rows(5, dt)
    src = make_quantized_kv_caches(pool)[0]
    k2, v2, dk, dv = r.take(2)
    src.update(dk, dv)
    cache = make_quantized_kv_caches(pool)[0]
    cache.restore_quantized(src.quantized_snapshot())
    k1, v1, dk, dv = r.take(1)
    res = cache.update(dk, dv)
    assert cache.sequence_length == 3
    _check(res, np.concatenate([k2[0], k1[0]], 1), np.concatenate([v2[0], v1[0]], 1), mode, dt)
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_truncate_then_update_overwrites_stale_rows(mode, dt):
    """The speculative rollback: 10 rows, truncate to 6, 2 new rows; equals a
    fresh cache fed the 6 kept rows and the 2 new ones."""
    print(f"\ncase cache_api truncate_then_update {mode}", flush=True)
    pool = _pool(mode, dt)
    r = _Rows(6, dt)
    k10, v10, dk10, dv10 = r.take(10)
    k2, v2, dk2, dv2 = r.take(2)
    cache = make_quantized_kv_caches(pool)[0]
    cache.update(dk10, dv10)
    cache.truncate(6)
    assert cache.sequence_length == 6
    res = cache.update(dk2, dv2)
    assert cache.sequence_length == 8
    kk, vv = np.concatenate([k10[0, :, :6], k2[0]], 1), np.concatenate([v10[0, :, :6], v2[0]], 1)
    _check(res, kk, vv, mode, dt)
    ref = make_quantized_kv_caches(pool)[0]
    ref.update(dk10[:, :, :6].contiguous(), dv10[:, :, :6].contiguous())
    ref_res = ref.update(dk2, dv2)
    for a, b in zip(res, ref_res):
        np.testing.assert_array_equal(_bits(a), _bits(b))
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_restore_does_not_alias_source(mode, dt):
    print(f"\ncase cache_api no_alias {mode}", flush=True)
    pool = _pool(mode, dt)
    r = _Rows(7, dt)
    src = make_quantized_kv_caches(pool)[0]
    k4, v4, dk, dv = r.take(4)
    src.update(dk, dv)
    snap = src.quantized_snapshot()
    saved = {n: t.clone() for n, t in snap.as_dict().items()}
    cache = make_quantized_kv_caches(pool)[0]
    cache.restore_quantized(snap)
    cache.truncate(2)
    _, _, dk, dv = r.take(2)
    cache.update(dk, dv)
    torch.cuda.synchronize()
    for n, t in snap.as_dict().items():
        assert torch.equal(t, saved[n]), f"restore aliased the snapshot's {n}"
    _check(src.snapshot(), k4[0], v4[0], mode, dt)  # the source cache is untouched too
    pool.close()


def test_restore_into_shared_blocks_is_refused():
    print("\ncase cache_api restore_shared", flush=True)
    pool = _pool("affine_g64", "bf16")
    r = _Rows(8, "bf16")
    a = make_quantized_kv_caches(pool)[0]
    _, _, dk, dv = r.take(70)
    a.update(dk, dv)
    fork = make_quantized_kv_caches(pool, pool.seq_fork(a.s.seq, 70))[0]
    with pytest.raises(RuntimeError, match="shared"):
        fork.restore_quantized(a.quantized_snapshot())
    pool.close()


@pytest.mark.parametrize("mode,dt", CASES)
def test_growth_across_capacity_boundary_preserves_contents(mode, dt):
    """300 updates of 2 rows (one head): 600 rows over 10 blocks."""
    print(f"\ncase cache_api growth {mode}", flush=True)
    pool = _pool(mode, dt, heads=1)
    cache = make_quantized_kv_caches(pool)[0]
    r = _Rows(9, dt, heads=1)
    ks, vs = [], []
    for _ in range(300):
        k, v, dk, dv = r.take(2)
        cache.append(dk, dv)
        ks.append(k[0])
        vs.append(v[0])
    assert cache.sequence_length == 600
    _check(cache.snapshot(), np.concatenate(ks, 1), np.concatenate(vs, 1), mode, dt)
    q = cache.quantized_snapshot()
    kq, kscale, kzero = O.quantize(np.concatenate(ks, 1), DT[dt], MODE[mode])
    np.testing.assert_array_equal(q.keys.cpu().numpy()[0], kq)
    np.testing.assert_array_equal(q.key_scales.cpu().numpy()[0].view(np.uint16), kscale)
    np.testing.assert_array_equal(q.key_zeros.cpu().numpy()[0].view(np.uint16), kzero)
    pool.close()


def test_krill_kernels_decode_and_verify_over_caches():
    """KrillKernels over the caches of one layer: a batched append, the
    decode step with the new token fused, the verify window, and the
    stacked snapshot, each against the oracle or the pool-level call."""
    from kvutil import Filled, oracle_attention

    print("\ncase krill_kernels", flush=True)
    assert KrillKernels.is_available()
    assert "ABI" in KrillKernels.status()
    dt, Hk, R = "bf16", 2, 4
    lens = [5, 64, 300]
    pool = krill_amd.KVPool(2, Hk, D, 32, "affine_g64", dt, free_list_seed=4)
    rng = np.random.default_rng(10)
    B = len(lens)
    layer_caches = [make_quantized_kv_caches(pool) for _ in range(B)]
    f = Filled.__new__(Filled)  # the oracle's view: rows per sequence of layer 1
    f.pool, f.dt, f.layers, f.seqs, f.lens = pool, dt, (1,), [c[0].s.seq for c in layer_caches], []
    f.k, f.v = {1: []}, {1: []}
    # prefill: both layers of every sequence, layer by layer in one batched launch each
    for layer in (0, 1):
        for b, T in enumerate(lens):
            k = rand_bits(rng, (1, Hk, T, D), dt)
            v = rand_bits(rng, (1, Hk, T, D), dt)
            KrillKernels.quantize_append([layer_caches[b][layer]], to_dev(k, dt), to_dev(v, dt))
            if layer == 1:
                f.k[1].append(k[0])
                f.v[1].append(v[0])
    caches = [c[1] for c in layer_caches]
    # one batched append of 3 rows to every sequence (layer 1 runs ahead of layer 0)
    k3 = rand_bits(rng, (B, Hk, 3, D), dt)
    v3 = rand_bits(rng, (B, Hk, 3, D), dt)
    KrillKernels.quantize_append(caches, to_dev(k3, dt), to_dev(v3, dt))
    for b in range(B):
        f.k[1][b] = np.concatenate([f.k[1][b], k3[b]], 1)
        f.v[1][b] = np.concatenate([f.v[1][b], v3[b]], 1)
    f.lens = [T + 3 for T in lens]
    assert [c.sequence_length for c in caches] == f.lens
    assert [c[0].sequence_length for c in layer_caches] == lens
    # verify over the last 3 positions
    scale = 1.0 / np.sqrt(D)
    qv = rand_bits(rng, (B, Hk * R, 3, D), dt)
    out = KrillKernels.paged_verify_attention(to_dev(qv, dt), caches, scale)
    torch.cuda.synchronize()
    assert np.abs(out.float().cpu().numpy() - oracle_attention(pool, f, 1, qv, dt, scale)).max() <= 2e-3
    # decode step with the new token fused
    kn = rand_bits(rng, (B, Hk, 1, D), dt)
    vn = rand_bits(rng, (B, Hk, 1, D), dt)
    q = rand_bits(rng, (B, Hk * R, 1, D), dt)
    out = KrillKernels.paged_decode_attention(to_dev(q, dt), caches, scale, to_dev(kn, dt), to_dev(vn, dt))
    torch.cuda.synchronize()
    for b in range(B):
        f.k[1][b] = np.concatenate([f.k[1][b], kn[b]], 1)
        f.v[1][b] = np.concatenate([f.v[1][b], vn[b]], 1)
    f.lens = [T + 1 for T in f.lens]
    assert [c.sequence_length for c in caches] == f.lens
    assert np.abs(out.float().cpu().numpy() - oracle_attention(pool, f, 1, q, dt, scale)).max() <= 2e-3
    # without new tokens: the same call as the pool's attention over the tables
    again = KrillKernels.paged_decode_attention(to_dev(q, dt), caches, scale)
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    direct = pool.attention(1, to_dev(q, dt), i32(t), i32(n), max(f.lens), scale)
    torch.cuda.synchronize()
    assert torch.equal(again, direct)
    # the stacked, left-padded snapshot (stackCachesLeftPaddedQuantized)
    from kvutil import check_snapshot

    check_snapshot(KrillKernels.stacked_quantized(caches), f, 1, left_pad=True)
    with pytest.raises(ValueError):
        KrillKernels.paged_decode_attention(to_dev(q, dt), [caches[0], layer_caches[1][0], caches[2]], scale)
    pool.close()
