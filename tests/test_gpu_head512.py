"""GPU: head_dim 512, the full-attention layers of Gemma 4.

Int8 KV is enabled for Gemma 4 only in the reference
(Sources/KrillRegistry/ModelAdapter.swift:151-172), and its full-attention
layers use globalHeadDim = 512 (Sources/KrillCore/Gemma4Model.swift:124,
:212, :332) with SDPA scale 1.0 (:516-517); 26B-A4B runs them with 2 KV
heads for 16 query heads (num_global_key_value_heads, :283-286), so 8
query rows per KV head at decode.  Here decode runs on the VALU kernel with
each 64-token block split over four 128-dim waves of one workgroup, and
more than 8 rows per KV head (verify windows, prefill chunks, the shared
prefix's pass) run in row groups of at most 8.

Cases, each against the float64 oracle at 2e-3 max-abs (cache bytes
bit-exact where they are written):
- the Gemma-4 full-attention decode step with the append fused, both storage
  modes, bf16 and f16, random queries at scale 1.0 (scores of spread
  about 22: a sharp softmax) and at 1/sqrt(D);
- peaked softmax: queries solved from chosen keys' dequantized rows so that
  one or three keys hold over 99 % of the weight, with x20 outlier channels;
- causal verify windows over row groups: 4 positions x 8 rows (4 groups of
  8) and 5 positions x 3 rows (3 groups of 5);
- a 64-position prefill chunk (64 row groups);
- the shared-prefix cascade against the single pass;
- KV-shared layers (Gemma4Model.swift:478-482, ModelLoader.swift:1069-1070):
  a shared layer attends the donor layer's cache through KrillKernels and
  appends nothing.
"""
import numpy as np
import pytest

from kvutil import DT, MODE, Filled, check_snapshot, i32, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd import KrillKernels  # noqa: E402
from krill_amd.cache import make_quantized_kv_caches  # noqa: E402
from oracle import oracle as O  # noqa: E402

ATOL = 2e-3
D = 512
H, R = 2, 8  # Gemma 4 26B-A4B full-attention layers: 2 KV heads, 16 query heads


def _pool(mode, dt, lens, seed, layers=1, extra=2):
    nb = sum((T + extra + 63) // 64 for T in lens) + 8
    return krill_amd.KVPool(layers, H, D, nb, mode, dt, free_list_seed=seed)


def _decode_step(pool, f, q, scale, rng, dt, layer=0):
    """One fused decode step (a new token per sequence) on `layer`; extends
    f and returns (output, tables, lens)."""
    B = len(f.lens)
    kn = rand_bits(rng, (B, H, 1, D), dt)
    vn = rand_bits(rng, (B, H, 1, D), dt)
    for s in f.seqs:
        pool.reserve_append(s, 1)
    f.lens = [T + 1 for T in f.lens]
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    out = pool.decode_append_attention(layer, to_dev(q, dt), to_dev(kn, dt), to_dev(vn, dt), i32(t), i32(n),
                                       max(f.lens), scale)
    torch.cuda.synchronize()
    for b in range(B):
        f.k[layer][b] = np.concatenate([f.k[layer][b], kn[b]], axis=1)
        f.v[layer][b] = np.concatenate([f.v[layer][b], vn[b]], axis=1)
    return out, i32(t), i32(n)


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("scale", [1.0, 1.0 / np.sqrt(D)])
def test_gemma4_full_attention_decode_step(mode, dt, scale):
    print(f"\ncase head512 decode mode={mode} dt={dt} scale={scale:.4f}", flush=True)
    rng = np.random.default_rng(512 + int(scale * 100) + (dt == "f16"))
    lens = [0, 1, 63, 64, 65, 700, 2049, 4000]
    pool = _pool(mode, dt, lens, seed=5)
    f = Filled(pool, lens, rng, dt, max_chunk=300, outlier_frac=0.01)
    q = rand_bits(rng, (len(lens), H * R, 1, D), dt)
    out, t, n = _decode_step(pool, f, q, scale, rng, dt)
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    check_snapshot(pool.gather(0, t, n, max(f.lens)), f, 0)
    pool.close()


def _peaked(f, pool, dt, n_hot, scale, rng):
    """q [B, Hq, 1, D] putting the weight on n_hot chosen keys (scores 24,
    23.3, 22.6 after the scale), off the outlier channels."""
    B = len(f.lens)
    mode = MODE[pool.quant_mode]
    q = np.zeros((B, H * R, 1, D), np.float32)
    targets = np.array([24.0, 23.3, 22.6])[:n_hot] / scale
    for b, T in enumerate(f.lens):
        kq, ks, kz, _, _, _ = f.expected(0, b)
        kd = O.dequant_f64(kq, ks, kz, mode)
        for hk in range(H):
            keep = (kd[hk].std(axis=0) < 5.0).astype(np.float64)
            for r in range(R):
                hot = rng.choice(T, size=n_hot, replace=False)
                Kh = kd[hk, hot] * keep
                q[b, hk * R + r, 0] = np.linalg.solve(Kh @ Kh.T, targets) @ Kh
    return O.f32_to_bf16_bits(q) if dt == "bf16" else O.f32_to_f16_bits(q)


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("n_hot,outliers", [(1, 0.0), (3, 0.01)])
def test_peaked_softmax_with_outliers(mode, n_hot, outliers):
    print(f"\ncase head512 peaked mode={mode} hot={n_hot} outliers={outliers}", flush=True)
    dt, scale = "bf16", 1.0
    rng = np.random.default_rng(77 + n_hot)
    lens = [900, 2500]
    pool = _pool(mode, dt, lens, seed=9)
    f = Filled(pool, lens, rng, dt, max_chunk=400, outlier_frac=outliers)
    q = _peaked(f, pool, dt, n_hot, scale, rng)
    t, n, _ = f.tables()
    out = pool.attention(0, to_dev(q, dt), t, n, max(lens), scale)
    torch.cuda.synchronize()
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    # the weight really sits on the chosen keys
    qf = O.bits_to_f32(q, DT[dt]).astype(np.float64)
    kq, ks, kz, _, _, _ = f.expected(0, 0)
    s = O.dequant_f64(kq, ks, kz, MODE[mode])[0] @ qf[0, 0, 0] * scale
    p = np.exp(s - s.max())
    assert np.sort(p / p.sum())[-3:].sum() > 0.99
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    pool.close()


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("Hq,Lq", [(16, 4), (6, 5), (16, 64)])
def test_causal_windows_in_row_groups(mode, Hq, Lq):
    """Verify windows and a prefill chunk: Hq/2 rows per position, Lq
    positions causal inside the window; 32 rows run as 4 groups of 8, 15 as 3
    groups of 5, 512 as 64 groups of 8."""
    print(f"\ncase head512 causal mode={mode} Hq={Hq} Lq={Lq}", flush=True)
    dt, scale = "bf16", 1.0
    rng = np.random.default_rng(Hq * 100 + Lq)
    lens = [Lq, 300, 1100] if Lq < 64 else [64, 200]
    pool = _pool(mode, dt, lens, seed=3)
    f = Filled(pool, lens, rng, dt, max_chunk=256)
    t, n, _ = f.tables()
    q = rand_bits(rng, (len(lens), Hq, Lq, D), dt)
    out = pool.attention(0, to_dev(q, dt), t, n, max(lens), scale)
    torch.cuda.synchronize()
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    pool.close()


def test_shared_prefix_cascade_matches_single_pass():
    print("\ncase head512 cascade", flush=True)
    dt, mode, scale = "bf16", "affine_g64", 1.0
    rng = np.random.default_rng(4242)
    PT, B = 300, 5
    extra = [0, 1, 64, 130, 7]
    nb = (PT + 63) // 64 + sum((PT % 64 + T + 1 + 63) // 64 for T in extra) + 8
    pool = krill_amd.KVPool(1, H, D, nb, mode, dt, free_list_seed=21)
    pre = Filled(pool, [PT], rng, dt, max_chunk=200)
    forks = [pool.seq_fork(pre.seqs[0], PT) for _ in range(B)]
    suf = Filled(pool, extra, rng, dt, seqs=forks, max_chunk=200)
    P = PT // 64
    lens = [PT + T for T in extra]
    t, n = pool.batch_tables(forks, max((T + 63) // 64 for T in lens))
    q = rand_bits(rng, (B, H * R, 1, D), dt)
    single = pool.attention(0, to_dev(q, dt), i32(t), i32(n), max(lens), scale)
    casc = pool.attention_shared_prefix(0, to_dev(q, dt), i32(t[0, :P]), i32(np.ascontiguousarray(t[:, P:])),
                                        i32(n - 64 * P), int(n.max()) - 64 * P, scale)
    torch.cuda.synchronize()
    # the oracle's view: prefix rows then each fork's own rows
    f = Filled.__new__(Filled)
    f.pool, f.dt, f.layers, f.seqs, f.lens = pool, dt, (0,), forks, lens
    f.k = {0: [np.concatenate([pre.k[0][0], k], axis=1) for k in suf.k[0]]}
    f.v = {0: [np.concatenate([pre.v[0][0], v], axis=1) for v in suf.v[0]]}
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    e1 = float(np.abs(single.float().cpu().numpy() - ref).max())
    e2 = float(np.abs(casc.float().cpu().numpy() - ref).max())
    print(f"single {e1:.3e} cascade {e2:.3e}", flush=True)
    assert e1 <= ATOL and e2 <= ATOL, (e1, e2)
    assert float((single - casc).abs().max()) <= 1e-4
    pool.close()


def test_kv_shared_layer_attends_the_donor_cache():
    """Gemma 4's KV-shared layers (i >= firstKVSharedLayer) reuse the donor
    layer's K/V and compute none of their own (Gemma4Model.swift:478-482,
    donors from ModelLoader.swift:1069-1070); the reference re-dequantizes
    the donor's cache for them (snapshot(), QuantizedKVCache.swift:82-89).
    Paged: the shared layer's attention is a call on the donor layer's caches
    with no new token -- after the donor's own decode step, so it sees the
    step's token -- and the shared layer's cache stays empty.  Layers: 0
    donor, 1 an ordinary layer, 2 shared (donor 0)."""
    print("\ncase head512 kv_shared", flush=True)
    dt, mode, scale = "bf16", "affine_g64", 1.0
    rng = np.random.default_rng(1069)
    lens = [40, 300, 129]
    B = len(lens)
    pool = krill_amd.KVPool(3, H, D, 3 * sum((T + 64) // 64 for T in lens) + 8, mode, dt, free_list_seed=8)
    caches = [make_quantized_kv_caches(pool) for _ in range(B)]
    f = Filled.__new__(Filled)  # the oracle's view of layer 0
    f.pool, f.dt, f.layers, f.seqs, f.lens = pool, dt, (0,), [c[0].s.seq for c in caches], list(lens)
    f.k, f.v = {0: []}, {0: []}
    for layer in (0, 1):  # prefill of the layers that own a cache
        for b, T in enumerate(lens):
            k = rand_bits(rng, (1, H, T, D), dt)
            v = rand_bits(rng, (1, H, T, D), dt)
            KrillKernels.quantize_append([caches[b][layer]], to_dev(k, dt), to_dev(v, dt))
            if layer == 0:
                f.k[0].append(k[0])
                f.v[0].append(v[0])
    donor = [c[0] for c in caches]
    # the decode step: the donor layer appends its token and attends
    kn = rand_bits(rng, (B, H, 1, D), dt)
    vn = rand_bits(rng, (B, H, 1, D), dt)
    q0 = rand_bits(rng, (B, H * R, 1, D), dt)
    KrillKernels.paged_decode_attention(to_dev(q0, dt), donor, scale, to_dev(kn, dt), to_dev(vn, dt))
    for b in range(B):
        f.k[0][b] = np.concatenate([f.k[0][b], kn[b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], vn[b]], axis=1)
    f.lens = [T + 1 for T in lens]
    # ... then the shared layer: its own queries over the donor's cache
    q2 = rand_bits(rng, (B, H * R, 1, D), dt)
    out = KrillKernels.paged_decode_attention(to_dev(q2, dt), donor, scale)
    torch.cuda.synchronize()
    ref = oracle_attention(pool, f, 0, q2, dt, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    assert [c[0].sequence_length for c in caches] == f.lens
    assert [c[1].sequence_length for c in caches] == lens  # layer 1 has not run its step yet
    assert [c[2].sequence_length for c in caches] == [0] * B  # the shared layer owns nothing
    assert [c[2].memory_size_bytes for c in caches] == [0] * B
    pool.close()
