"""GPU parity at the benchmark workloads' own sizes, against the oracle.

Each case runs one workload's shape, batch and context lengths (one or two
layers of it) through the C ABI and checks the attention output against the
float64 oracle (2e-3 max-abs) and the cache bytes against the oracle's
quantization (bit-exact):
- Llama-3.2-1B, one sequence of 2048 tokens, a decode step with the append
  fused on the first and the last of 16 layers;
- Qwen3-14B, 32 sequences of U[512, 8192] tokens, the fused decode step, in
  affine group-64 and in the reference's row mode;
- Llama-3-8B, 64 sequences forked from one 4120-token prefix, each with
  U[0, 1024] tokens of its own (copy-on-write of the shared partial block),
  the shared-prefix decode step with the append fused; the prefix sequence
  is unchanged;
- Llama-3-8B speculative verify: 16 sequences of U[1024, 8192] tokens, 8
  draft rows appended and attended causally, then the rollback of
  SpeculativeDecoder.swift:309-318 (keep the accepted rows, truncate the
  rest), then one more fused decode step: the rows truncated away are
  neither attended nor left in the cache;
- Llama-3-8B shared prefix with the pool crossing its 90 % watermark: an
  unreferenced prefix entry is evicted while the forks append, its blocks
  are reissued to them (stale bytes beyond each fork's length), then the
  cascade step, against the oracle;
- Qwen3-30B-A3B long context: 2 of the 8 sequences at 131072 tokens with
  x20 outlier channels, the fused decode step; and all 8 sequences at
  131072 tokens (the benchmark's grid) with keys equal inside each 64-token
  block, where the output has a closed form over per-block sums.
Inputs are seeded N(0,1) bf16, affine int8 in groups of 64 unless a case
names the row mode."""
import numpy as np
import pytest

from kvutil import Filled, check_snapshot, i32, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402

ATOL = 2e-3
DT = "bf16"


def _blocks(lens, extra=1):
    return sum((T + extra + 63) // 64 for T in lens) + 8


def _fused_steps(pool, f, rng, R, outlier_frac=0.0):
    """One decode step for every sequence of `f` on each of its layers: one
    slot reserved per sequence, then per layer the fused append + attention.
    Extends `f` by the new token; returns the largest error against the
    oracle over the layers."""
    B, H, D = len(f.lens), pool.num_kv_heads, pool.head_dim
    for s in f.seqs:
        pool.reserve_append(s, 1)
    f.lens = [T + 1 for T in f.lens]
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    assert list(n) == f.lens
    tables, lens = i32(t), i32(n)
    scale = 1.0 / np.sqrt(D)
    worst = 0.0
    for layer in f.layers:
        kn = rand_bits(rng, (B, H, 1, D), DT, outlier_frac=outlier_frac)
        vn = rand_bits(rng, (B, H, 1, D), DT, outlier_frac=outlier_frac)
        q = rand_bits(rng, (B, H * R, 1, D), DT)
        out = pool.decode_append_attention(layer, to_dev(q, DT), to_dev(kn, DT), to_dev(vn, DT), tables, lens,
                                           max(f.lens), scale)
        torch.cuda.synchronize()
        for b in range(B):
            f.k[layer][b] = np.concatenate([f.k[layer][b], kn[b]], axis=1)
            f.v[layer][b] = np.concatenate([f.v[layer][b], vn[b]], axis=1)
        ref = oracle_attention(pool, f, layer, q, DT, scale)
        worst = max(worst, float(np.abs(out.float().cpu().numpy() - ref).max()))
    return worst, tables, lens


def test_llama32_1b_b1_decode_step():
    print("\ncase config llama-3.2-1b b1 T2048", flush=True)
    rng = np.random.default_rng(20261201)
    H, R, D = 8, 4, 64
    pool = krill_amd.KVPool(16, H, D, _blocks([2048]), "affine_g64", DT, free_list_seed=1)
    f = Filled(pool, [2048], rng, DT, layers=(0, 15), max_chunk=512)
    err, tables, lens = _fused_steps(pool, f, rng, R)
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    for layer in (0, 15):
        check_snapshot(pool.gather(layer, tables, lens, 2049), f, layer)
    pool.close()


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_qwen3_14b_b32_decode_step(mode):
    print(f"\ncase config qwen3-14b b32 U[512,8192] {mode}", flush=True)
    rng = np.random.default_rng(20261202)
    H, R, D = 8, 5, 128
    ctx = [int(x) for x in rng.integers(512, 8193, 32)]
    pool = krill_amd.KVPool(1, H, D, _blocks(ctx), mode, DT, free_list_seed=2)
    f = Filled(pool, ctx, rng, DT, max_chunk=512)
    err, tables, lens = _fused_steps(pool, f, rng, R)
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    check_snapshot(pool.gather(0, tables, lens, max(f.lens)), f, 0)
    pool.close()


class _Joined(Filled):
    """The prefix rows followed by each fork's own rows, as the oracle sees them."""

    def __init__(self, pre, suf):
        self.pool, self.dt, self.layers = pre.pool, pre.dt, pre.layers
        self.seqs = list(suf.seqs)
        self.lens = [pre.lens[0] + T for T in suf.lens]
        self.k = {l: [np.concatenate([pre.k[l][0], k], axis=1) for k in suf.k[l]] for l in self.layers}
        self.v = {l: [np.concatenate([pre.v[l][0], v], axis=1) for v in suf.v[l]] for l in self.layers}


def test_llama3_8b_shared_prefix_b64_step():
    print("\ncase config llama-3-8b shared prefix 4120 b64", flush=True)
    rng = np.random.default_rng(20261203)
    H, R, D, B, PT = 8, 4, 128, 64, 4120
    extra = [int(x) for x in rng.integers(0, 1025, B)]
    nb = (PT + 63) // 64 + sum((PT % 64 + T + 1 + 63) // 64 for T in extra) + 8
    pool = krill_amd.KVPool(1, H, D, nb, "affine_g64", DT, free_list_seed=3)
    pre = Filled(pool, [PT], rng, DT, max_chunk=512)
    forks = [pool.seq_fork(pre.seqs[0], PT) for _ in range(B)]
    cow0 = pool.stats()["cow_copies"]
    suf = Filled(pool, extra, rng, DT, seqs=forks, max_chunk=512)
    # every fork that appended wrote into the shared partial block first: one copy each
    assert pool.stats()["cow_copies"] - cow0 == sum(1 for T in extra if T > 0)
    f = _Joined(pre, suf)
    P = PT // 64
    for s in f.seqs:
        pool.reserve_append(s, 1)  # the forks without tokens of their own copy the block now
    assert pool.stats()["cow_copies"] - cow0 == B
    f.lens = [T + 1 for T in f.lens]
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    assert (t[:, :P] == t[0, :P]).all()  # the 64 full prefix blocks stay shared
    assert len(set(t[:, P].tolist())) == B  # each fork has its own copy of the partial block
    kn = rand_bits(rng, (B, H, 1, D), DT)
    vn = rand_bits(rng, (B, H, 1, D), DT)
    q = rand_bits(rng, (B, H * R, 1, D), DT)
    scale = 1.0 / np.sqrt(D)
    out = pool.attention_shared_prefix(0, to_dev(q, DT), i32(t[0, :P]), i32(np.ascontiguousarray(t[:, P:])),
                                       i32(n - 64 * P), int(n.max()) - 64 * P, scale, k_new=to_dev(kn, DT),
                                       v_new=to_dev(vn, DT))
    torch.cuda.synchronize()
    for b in range(B):
        f.k[0][b] = np.concatenate([f.k[0][b], kn[b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], vn[b]], axis=1)
    ref = oracle_attention(pool, f, 0, q, DT, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    # the forks' caches, and the prefix sequence untouched by their appends
    check_snapshot(pool.gather(0, i32(t), i32(n), max(f.lens)), f, 0)
    tp, np_ = pool.batch_tables(pre.seqs, (PT + 63) // 64)
    check_snapshot(pool.gather(0, i32(tp), i32(np_), PT), pre, 0)
    pool.close()


def test_llama3_8b_verify_rollback_then_decode():
    print("\ncase config llama-3-8b verify b16 k8 + rollback", flush=True)
    rng = np.random.default_rng(20261204)
    H, R, D, B, k = 8, 4, 128, 16, 8
    ctx = [int(x) for x in rng.integers(1024, 8193, B)]
    pool = krill_amd.KVPool(1, H, D, _blocks(ctx, k + 1), "affine_g64", DT, free_list_seed=4)
    f = Filled(pool, ctx, rng, DT, max_chunk=512)
    # verify: the k rows of the window appended, then attended causally
    kd = rand_bits(rng, (B, H, k, D), DT)
    vd = rand_bits(rng, (B, H, k, D), DT)
    slots = np.stack([pool.reserve_append(s, k) for s in f.seqs])
    pool.quantize_append(0, to_dev(kd, DT), to_dev(vd, DT), i32(slots))
    for b in range(B):
        f.k[0][b] = np.concatenate([f.k[0][b], kd[b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], vd[b]], axis=1)
    f.lens = [T + k for T in ctx]
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    q = rand_bits(rng, (B, H * R, k, D), DT)
    scale = 1.0 / np.sqrt(D)
    out = pool.attention(0, to_dev(q, DT), i32(t), i32(n), max(f.lens), scale)
    torch.cuda.synchronize()
    ref = oracle_attention(pool, f, 0, q, DT, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"verify max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"verify max abs error {err:.3e}"
    # accepted drafts a in [0, k]: the window's first row and the a accepted
    # drafts stay (all k rows on full acceptance), the rest is truncated
    acc = rng.integers(0, k + 1, B)
    acc[:2] = (0, k)  # both ends
    keep = np.minimum(acc + 1, k)
    free0 = pool.stats()["blocks_free"]
    for b in range(B):
        L = ctx[b] + int(keep[b])
        pool.seq_truncate(f.seqs[b], L)
        assert pool.seq_length(f.seqs[b]) == L
        f.k[0][b] = f.k[0][b][:, :L]
        f.v[0][b] = f.v[0][b][:, :L]
    freed = sum((ctx[b] + k + 63) // 64 - (ctx[b] + int(keep[b]) + 63) // 64 for b in range(B))
    assert pool.stats()["blocks_free"] - free0 == freed
    f.lens = [ctx[b] + int(keep[b]) for b in range(B)]
    # the next decode step writes over the first truncated row
    err, tables, lens = _fused_steps(pool, f, rng, R)
    print(f"after rollback max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"after rollback max abs error {err:.3e}"
    check_snapshot(pool.gather(0, tables, lens, max(f.lens)), f, 0)
    pool.close()


def test_qwen3_30b_a3b_128k_decode_step():
    print("\ncase config qwen3-30b-a3b 128k outliers (2 of 8 sequences)", flush=True)
    rng = np.random.default_rng(20261205)
    H, R, D, T = 4, 8, 128, 131072
    pool = krill_amd.KVPool(1, H, D, _blocks([T, T]), "affine_g64", DT, free_list_seed=5)
    f = Filled(pool, [T, T], rng, DT, max_chunk=4096, outlier_frac=0.01)
    err, tables, lens = _fused_steps(pool, f, rng, R, outlier_frac=0.01)
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    pool.close()


def test_llama3_8b_shared_prefix_after_watermark_eviction():
    """Config 3 with LRU eviction on the GPU: a 1000-token prefix entry that
    no sequence holds any more is the pool's oldest; while 64 forks of a
    4120-token prefix append their own tokens the pool crosses 90 % of its
    blocks, the entry is evicted (PrefixCache.swift:535-551 at block level)
    and its blocks are handed to the forks.  The cascade step with the
    append fused must then match the oracle, and the forks' bytes too."""
    print("\ncase config llama-3-8b shared prefix b64 + watermark eviction", flush=True)
    rng = np.random.default_rng(20261213)
    H, R, D, B, PT, VT = 8, 4, 128, 64, 4120, 1000
    extra = [int(x) for x in rng.integers(0, 1025, B)]
    P = PT // 64
    used_final = (PT + 63) // 64 + sum((PT % 64 + T + 1 + 63) // 64 for T in extra)
    nb = used_final + 12  # 90 % of it is below used_final + the entry's 16 blocks
    pool = krill_amd.KVPool(1, H, D, nb, "affine_g64", DT, free_list_seed=13, max_prefix_entries=8,
                            min_prefix_len=8)
    victim = Filled(pool, [VT], rng, DT, max_chunk=512)
    vblocks = set(pool.block_table(victim.seqs[0]).tolist())
    assert pool.prefix_store(victim.seqs[0], np.arange(VT), "m")
    pool.seq_free(victim.seqs[0])  # only the entry holds its 16 blocks now
    pre = Filled(pool, [PT], rng, DT, max_chunk=512)
    forks = [pool.seq_fork(pre.seqs[0], PT) for _ in range(B)]
    suf = Filled(pool, extra, rng, DT, seqs=forks, max_chunk=512)
    f = _Joined(pre, suf)
    for s in f.seqs:
        pool.reserve_append(s, 1)
    st = pool.stats()
    assert st["evicted_entries"] == 1 and st["evicted_blocks"] == len(vblocks), st
    assert pool.prefix_lookup(np.arange(VT), "m") == (0, None)
    f.lens = [T + 1 for T in f.lens]
    t, n = pool.batch_tables(f.seqs, max((T + 63) // 64 for T in f.lens))
    held = set(t[:, P:][t[:, P:] >= 0].tolist())
    assert len(held & vblocks) > 0, "the evicted entry's blocks were not reissued"
    kn = rand_bits(rng, (B, H, 1, D), DT)
    vn = rand_bits(rng, (B, H, 1, D), DT)
    q = rand_bits(rng, (B, H * R, 1, D), DT)
    scale = 1.0 / np.sqrt(D)
    out = pool.attention_shared_prefix(0, to_dev(q, DT), i32(t[0, :P]), i32(np.ascontiguousarray(t[:, P:])),
                                       i32(n - 64 * P), int(n.max()) - 64 * P, scale, k_new=to_dev(kn, DT),
                                       v_new=to_dev(vn, DT))
    torch.cuda.synchronize()
    for b in range(B):
        f.k[0][b] = np.concatenate([f.k[0][b], kn[b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], vn[b]], axis=1)
    ref = oracle_attention(pool, f, 0, q, DT, scale)
    err = float(np.abs(out.float().cpu().numpy() - ref).max())
    print(f"max abs error {err:.3e} ({len(held & vblocks)} reissued blocks)", flush=True)
    assert err <= ATOL, f"max abs error {err:.3e}"
    check_snapshot(pool.gather(0, i32(t), i32(n), max(f.lens)), f, 0)
    pool.close()


def test_qwen3_30b_a3b_b8_128k_blockwise_equal_keys():
    """Config 5 at its own batch: 8 sequences of 131072 tokens (the grid and
    split the benchmark times), x20 outlier channels in V.  Every token of a
    64-token block has the same K row (its own per (sequence, head, block)),
    so each block's keys score alike and the output of query row r is
        sum_j exp(s_rj) Vsum_j / sum_j n_j exp(s_rj)
    over blocks j (n_j tokens, Vsum_j the sum of its dequantized V rows,
    s_rj = scale q_r . k_j on the dequantized key), computed in float64 from
    the oracle's quantization, block sums accumulated while the pool fills.
    Then one fused decode step (the new token in a block of its own)."""
    from kvutil import DT as ODT, MODE
    from oracle import oracle as O

    print("\ncase config qwen3-30b-a3b b8 128k blockwise-equal keys", flush=True)
    rng = np.random.default_rng(20261215)
    H, R, D, B, T, C = 4, 8, 128, 8, 131072, 8192
    NBK = T // 64
    mode = MODE["affine_g64"]
    pool = krill_amd.KVPool(1, H, D, B * (NBK + 1) + 8, "affine_g64", DT, free_list_seed=15)
    seqs = [pool.seq_create() for _ in range(B)]
    kblk = rand_bits(rng, (B, H, NBK + 1, D), DT)  # the last: the new token's row
    ch = rng.choice(D, size=max(1, int(round(0.01 * D))), replace=False)  # outlier channels of V
    vsum = np.zeros((B, H, NBK + 1, D), np.float64)
    for c0 in range(0, T, C):
        slots = np.stack([pool.reserve_append(s, C) for s in seqs])
        kb = np.repeat(kblk[:, :, c0 // 64:(c0 + C) // 64], 64, axis=2)
        x = rng.standard_normal((B, H, C, D)).astype(np.float32)
        x[..., ch] *= 20.0
        vb = O.f32_to_bf16_bits(x)
        pool.quantize_append(0, to_dev(kb, DT), to_dev(vb, DT), i32(slots))
        for b in range(B):
            vq, vs, vz = O.quantize(vb[b], ODT[DT], mode)
            vd = O.dequant_f64(vq, vs, vz, mode)  # [H, C, D]
            vsum[b, :, c0 // 64:(c0 + C) // 64] = vd.reshape(H, C // 64, 64, D).sum(axis=2)
    torch.cuda.synchronize()
    # the decode step: one more token per sequence, in block NBK
    for s in seqs:
        pool.reserve_append(s, 1)
    kn = np.ascontiguousarray(kblk[:, :, NBK:NBK + 1])
    x = rng.standard_normal((B, H, 1, D)).astype(np.float32)
    x[..., ch] *= 20.0
    vn = O.f32_to_bf16_bits(x)
    for b in range(B):
        vq, vs, vz = O.quantize(vn[b], ODT[DT], mode)
        vsum[b, :, NBK] = O.dequant_f64(vq, vs, vz, mode)[:, 0]
    q = rand_bits(rng, (B, H * R, 1, D), DT)
    t, n = pool.batch_tables(seqs, NBK + 1)
    assert (n == T + 1).all()
    scale = 1.0 / np.sqrt(D)
    out = pool.decode_append_attention(0, to_dev(q, DT), to_dev(kn, DT), to_dev(vn, DT), i32(t), i32(n), T + 1,
                                       scale).float().cpu().numpy()
    torch.cuda.synchronize()
    cnt = np.full(NBK + 1, 64.0)
    cnt[NBK] = 1.0
    qf = O.bits_to_f32(q, ODT[DT]).astype(np.float64)
    worst = 0.0
    for b in range(B):
        kq, ks, kz = O.quantize(kblk[b], ODT[DT], mode)
        kd = O.dequant_f64(kq, ks, kz, mode)  # [H, NBK + 1, D]
        for hk in range(H):
            for r in range(R):
                hq = hk * R + r
                sc = scale * (kd[hk] @ qf[b, hq, 0])
                w = np.exp(sc - sc.max())
                ref = (w[:, None] * vsum[b, hk]).sum(axis=0) / (w * cnt).sum()
                worst = max(worst, float(np.abs(out[b, hq, 0] - ref).max()))
    print(f"max abs error {worst:.3e}", flush=True)
    assert worst <= ATOL, f"max abs error {worst:.3e}"
    pool.close()
