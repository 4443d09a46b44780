"""GPU: sliding-window layers in paged form (pool option KRILL_OPT_WINDOW +
krill_attention_windowed).  The reference's gate (RotatingKVCacheTests.swift
:40-113): the retained window attended without a mask must equal the full
cache with the sliding mask, at decode (L = 1) and chunked-prefill shapes.
Here both sides are built: a windowed pool whose blocks below the window go
back to the pool, and a pool that keeps every block attended with the same
window rule; both must match the oracle (attention over each row's visible
keys [max(first retained, p - window + 1), p]) within 2e-3 and each other to
float32 reassociation.  The first retained token follows RotatingKVCache's
retention (oracle.rotating_retained_start)."""
import numpy as np
import pytest

from kvutil import DT, MODE, i32, rand_bits, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402

ATOL = 2e-3
DTS = "bf16"


class Seqs:
    """B sequences appended through the product path in one pool; the
    oracle's copy of every token and the ops applied to each sequence."""

    def __init__(self, pool, B, total, rng, dt=DTS):
        H, D = pool.num_kv_heads, pool.head_dim
        self.pool, self.B, self.dt = pool, B, dt
        self.seqs = [pool.seq_create() for _ in range(B)]
        self.k = [rand_bits(rng, (H, total, D), dt) for _ in range(B)]
        self.v = [rand_bits(rng, (H, total, D), dt) for _ in range(B)]
        self.ops = [[] for _ in range(B)]
        self.len = [0] * B

    def append(self, b, L):
        s, p = self.seqs[b], self.len[b]
        slots = self.pool.reserve_append(s, L)
        self.pool.quantize_append(0, to_dev(self.k[b][None, :, p:p + L], self.dt),
                                  to_dev(self.v[b][None, :, p:p + L], self.dt), i32(slots[None]))
        self.len[b] += L
        self.ops[b].append(("append", L))

    def truncate(self, b, n):
        self.pool.seq_truncate(self.seqs[b], n)
        self.len[b] = n
        self.ops[b].append(("truncate", n))

    def tables(self):
        mb = max((n + 63) // 64 for n in self.len)
        t, n = self.pool.batch_tables(self.seqs, mb)
        return i32(t), i32(n), mb


def _oracle_rows(seqs, b, q_bits, window, start, mode):
    """Expected outputs [Hq, Lq, D] of sequence b's last Lq query rows."""
    H = seqs.pool.num_kv_heads
    Hq, Lq, D = q_bits.shape
    R = Hq // H
    n = seqs.len[b]
    kq, ks, kz = O.quantize(seqs.k[b][:, :n], DT[seqs.dt], MODE[mode])
    vq, vs, vz = O.quantize(seqs.v[b][:, :n], DT[seqs.dt], MODE[mode])
    kd, vd = O.dequant_f64(kq, ks, kz, MODE[mode]), O.dequant_f64(vq, vs, vz, MODE[mode])
    qf = O.bits_to_f32(q_bits, DT[seqs.dt]).astype(np.float64)
    rows = O.sliding_window_rows(Lq, n - Lq, window)
    lo = [max(start, a) for a, _ in rows]
    hi = [h for _, h in rows]
    out = np.zeros((Hq, Lq, D))
    for hq in range(Hq):
        out[hq] = O.attention_window_f64(qf[hq], kd[hq // R], vd[hq // R], lo, hi, 1.0 / np.sqrt(D))
    return out


def _check(pools, seqs_list, window, Lq, mode, rng, R, tol_pair=1e-5):
    """Windowed attention of the last Lq rows of every sequence in each pool
    (first pool: window option set, blocks below the window dropped; second:
    every block kept, attended with the first pool's first retained tokens,
    or with none (None) while no sequence has dropped any)."""
    B = seqs_list[0].B
    H, D = pools[0].num_kv_heads, pools[0].head_dim
    dt = seqs_list[0].dt
    q = rand_bits(rng, (B, H * R, Lq, D), dt)
    st = pools[0].batch_starts(seqs_list[0].seqs)
    outs = []
    for pool, seqs in zip(pools, seqs_list):
        t, n, mb = seqs.tables()
        starts = None if pool is pools[1] and not st.any() else i32(st)
        out = pool.attention_windowed(0, to_dev(q, dt), t, n, starts, window, int(max(seqs.len)), 1.0 / np.sqrt(D))
        torch.cuda.synchronize()
        outs.append(out.cpu().numpy())
    seqs = seqs_list[0]
    for b in range(B):
        total, start = O.rotating_retained_start(seqs.ops[b], window)
        assert total == seqs.len[b] and int(pools[0].batch_starts([seqs.seqs[b]])[0]) == start
        want = _oracle_rows(seqs, b, q[b], window, start, mode)
        for o in outs:
            err = np.abs(o[b] - want).max()
            assert err <= ATOL, (b, err)
    dev = np.abs(outs[0] - outs[1]).max()
    assert dev <= tol_pair, dev


def _pools(mode, H, D, blocks, window, seed, dt=DTS):
    a = krill_amd.KVPool(1, H, D, blocks, mode, dt, free_list_seed=seed)
    a.set_option(krill_amd._lib.OPT_WINDOW, window)
    b = krill_amd.KVPool(1, H, D, blocks, mode, dt, free_list_seed=seed + 1)
    return a, b


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R", [(128, 4), (64, 2), (256, 2), (512, 8)])
def test_window_decode_parity(mode, D, R):
    print(f"\ncase window_decode mode={mode} D={D} R={R}", flush=True)
    W, H, steps = 100, 2, 24
    rng = np.random.default_rng(D + R)
    pools = _pools(mode, H, D, 64, W, seed=D)
    fills = [[70, 64, 30], [5], [200, 3]]
    sl = []
    for pool in pools:
        ss = Seqs(pool, 3, 420, np.random.default_rng(7))
        for b, chunks in enumerate(fills):
            for L in chunks:
                ss.append(b, L)
        sl.append(ss)
    for step in range(steps):
        for ss in sl:
            for b in range(3):
                ss.append(b, 1)
        if step % 6 == 5 or step == 0:
            _check(pools, sl, W, 1, mode, rng, R)
    # the windowed pool holds only the blocks of each window (+ the partly filled last one)
    used = pools[0].stats()["blocks_used"]
    assert used <= 3 * ((W + 62) // 64 + 1), used
    for p in pools:
        p.close()


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_window_chunk_parity(mode):
    """Chunks straddling the window (RotatingKVCacheTests.swift:77-113 with
    64-token blocks): the chunk's rows on MFMA when R * L > 8."""
    print(f"\ncase window_chunks mode={mode}", flush=True)
    W, H, D, R = 100, 2, 64, 4
    rng = np.random.default_rng(11)
    pools = _pools(mode, H, D, 64, W, seed=3)
    sl = [Seqs(p, 1, 600, np.random.default_rng(9)) for p in pools]
    for L in [50, 30, 120, 1, 10, 90, 60, 200, 2]:
        for ss in sl:
            ss.append(0, L)
        _check(pools, sl, W, L, mode, rng, R, tol_pair=1e-3)
    for p in pools:
        p.close()


def test_window_truncate_then_decode():
    """After a rollback inside the retained tail the first retained token
    binds (fewer than window keys visible), as in RotatingKVCacheTests
    .swift:133-161."""
    print("\ncase window_truncate", flush=True)
    W, H, D, R = 100, 2, 128, 4
    rng = np.random.default_rng(13)
    pools = _pools("affine_g64", H, D, 32, W, seed=5)
    sl = [Seqs(p, 2, 400, np.random.default_rng(17)) for p in pools]
    for ss in sl:
        ss.append(0, 250)
        ss.append(0, 50)   # trims to the last 99 of 250 first
        ss.append(1, 120)
        ss.append(1, 1)
        ss.truncate(0, 230)
        ss.append(0, 1)
        ss.append(1, 1)
    _, start = O.rotating_retained_start(sl[0].ops[0], W)
    assert start == 151 and sl[0].len[0] - start < W  # the start binds
    _check(pools, sl, W, 1, "affine_g64", rng, R)
    for p in pools:
        p.close()


@pytest.mark.parametrize("Lq", [1, 40])
def test_window_f16_inputs(Lq):
    """fp16 K/V/queries (the other input dtype), decode and a chunk on MFMA."""
    print(f"\ncase window_f16 Lq={Lq}", flush=True)
    W, H, D, R = 130, 2, 128, 4
    rng = np.random.default_rng(41 + Lq)
    pools = _pools("affine_g64", H, D, 48, W, seed=9, dt="f16")
    sl = [Seqs(p, 2, 700, np.random.default_rng(43), dt="f16") for p in pools]
    for ss in sl:
        ss.append(0, 300)
        ss.append(1, 90)
        ss.append(0, Lq)
        ss.append(1, Lq)
    _check(pools, sl, W, Lq, "affine_g64", rng, R, tol_pair=1e-3)
    for p in pools:
        p.close()


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_window_prefill_chunk_32_row_waves(mode):
    """A 32-position chunk x 5 query heads per KV head (160 rows) over four
    long sequences with an 8192-token window (windowed calls are planned on
    min(max_seq_len, window + Lq + 62) tokens: here long enough for 32-row
    waves in groups of four), each chunk appended after its prefix; the
    longest sequence's first retained token (9) and its rows' window starts
    fall inside its first block."""
    print(f"\ncase window_prefill_rows32 mode={mode}", flush=True)
    W, H, D, R, Lq = 8192, 8, 128, 5, 32
    rng = np.random.default_rng(71)
    lens = [8200, 3000, 6100, 900]
    pools = _pools(mode, H, D, sum((n + Lq + 63) // 64 for n in lens) + 8, W, seed=21)
    sl = [Seqs(p, len(lens), max(lens) + Lq, np.random.default_rng(73)) for p in pools]
    for ss in sl:
        for b, n in enumerate(lens):
            ss.append(b, n)
            ss.append(b, Lq)
    _check(pools, sl, W, Lq, mode, rng, R, tol_pair=1e-3)
    for p in pools:
        p.close()


@pytest.mark.parametrize("rope", [False, True])
@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R", [(128, 4), (256, 2)])
def test_window_fused_decode_step(mode, D, R, rope):
    """krill_decode_append_attention_windowed: the newest token written at
    lens - 1 and windowed attention in one launch (with RoPE of the queries
    and the new K row when rope) equals the two calls -- quantize-append
    (_rope) at the reserved slot, then krill_attention_windowed on the
    (oracle-rotated) queries -- in output and pool bytes, bit for bit, over
    several steps with window trims; without RoPE also the oracle."""
    from krill_amd.pool import rope_table

    print(f"\ncase window_fused mode={mode} D={D} R={R} rope={rope}", flush=True)
    W, H, B, steps = 100, 2, 3, 5
    rng = np.random.default_rng(D + R + 7 * rope)
    # two pools with the window option and the same block order
    pools = []
    for _ in range(2):
        p = krill_amd.KVPool(1, H, D, 64, mode, DTS, free_list_seed=D)
        p.set_option(krill_amd._lib.OPT_WINDOW, W)
        pools.append(p)
    fills = [[70, 64, 30], [5], [200, 3]]
    sl = []
    for pool in pools:
        ss = Seqs(pool, B, 420, np.random.default_rng(7))
        for b, chunks in enumerate(fills):
            for L in chunks:
                ss.append(b, L)
        sl.append(ss)
    cs = rope_table(512, D, 1.0e4)
    csd = torch.from_numpy(cs).cuda()
    scale = 1.0 / np.sqrt(D)
    for step in range(steps):
        q = rand_bits(rng, (B, H * R, 1, D), DTS)
        pos = np.array([sl[0].len[b] for b in range(B)], np.int32)  # the new tokens' positions
        # pool 0: two calls
        p0, s0 = pools[0], sl[0]
        slots = np.stack([p0.reserve_append(s0.seqs[b], 1) for b in range(B)]).astype(np.int32)
        kn = np.stack([s0.k[b][:, pos[b]:pos[b] + 1] for b in range(B)])
        vn = np.stack([s0.v[b][:, pos[b]:pos[b] + 1] for b in range(B)])
        if rope:
            p0.quantize_append_rope(0, to_dev(kn, DTS), to_dev(vn, DTS), i32(slots), i32(pos.reshape(B, 1)), csd)
            qq = O.rope_rows(q, DT[DTS], np.broadcast_to(pos[:, None, None], (B, H * R, 1)), cs)
        else:
            p0.quantize_append(0, to_dev(kn, DTS), to_dev(vn, DTS), i32(slots))
            qq = q
        for b in range(B):
            s0.len[b] += 1
            s0.ops[b].append(("append", 1))
        t0, n0, _ = s0.tables()
        st0 = i32(p0.batch_starts(s0.seqs))
        out_two = p0.attention_windowed(0, to_dev(qq, DTS), t0, n0, st0, W, int(max(s0.len)), scale)
        # pool 1: the fused step
        p1, s1 = pools[1], sl[1]
        for b in range(B):
            p1.reserve_append(s1.seqs[b], 1)
            s1.len[b] += 1
            s1.ops[b].append(("append", 1))
        t1, n1, _ = s1.tables()
        st1 = i32(p1.batch_starts(s1.seqs))
        out_fused = p1.decode_append_attention_windowed(0, to_dev(q, DTS), to_dev(kn, DTS), to_dev(vn, DTS), t1, n1,
                                                        st1, W, int(max(s1.len)), scale,
                                                        cos_sin=csd if rope else None)
        torch.cuda.synchronize()
        assert torch.equal(out_two, out_fused), step
        g0 = {k: v.cpu().numpy() for k, v in p0.gather(0, t0, n0, int(max(s0.len))).items()}
        g1 = {k: v.cpu().numpy() for k, v in p1.gather(0, t1, n1, int(max(s1.len))).items()}
        for k in g0:
            np.testing.assert_array_equal(g0[k], g1[k])
        if not rope:
            got = out_fused.cpu().numpy()
            for b in range(B):
                total, start = O.rotating_retained_start(s1.ops[b], W)
                want = _oracle_rows(s1, b, q[b], W, start, mode)
                err = np.abs(got[b] - want).max()
                assert err <= ATOL, (step, b, err)
    for p in pools:
        p.close()


def test_window_view_limit():
    """Up to 8 rows per KV head at head_dim <= 256 the windowed call runs one
    workgroup per (sequence, KV head), each wave reading at most 64 blocks:
    at head_dim 256 with 8 rows, two waves, so a view (window + Lq + 62
    tokens, capped at max_seq_len) of 8192 tokens is attended and one past it
    is refused with KRILL_E_UNSUPPORTED; the MFMA path takes that call."""
    from krill_amd._lib import KrillError, KRILL_E_UNSUPPORTED, OPT_ATTN_PATH
    print("\ncase window_view_limit D=256 R=8", flush=True)
    D, H, R, W = 256, 1, 8, 8200
    pool = krill_amd.KVPool(1, H, D, 300, "affine_g64", DTS, free_list_seed=3)
    pool.set_option(krill_amd._lib.OPT_WINDOW, W)
    ss = Seqs(pool, 2, 8192, np.random.default_rng(11))
    for b, L in enumerate([8192, 3000]):
        for p in range(0, L, 1024):
            ss.append(b, min(1024, L - p))
    rng = np.random.default_rng(12)
    q = rand_bits(rng, (2, H * R, 1, D), DTS)
    qd = to_dev(q, DTS)
    st = i32(pool.batch_starts(ss.seqs))
    want = [_oracle_rows(ss, b, q[b], W, int(pool.batch_starts([ss.seqs[b]])[0]), "affine_g64") for b in range(2)]

    def run(mb, msl):
        t, n = pool.batch_tables(ss.seqs, mb)
        out = pool.attention_windowed(0, qd, i32(t), i32(n), st, W, msl, 1.0 / np.sqrt(D))
        torch.cuda.synchronize()
        return out.cpu().numpy()

    out = run(128, 8192)  # view 8192: the decode kernel's limit for this shape
    for b in range(2):
        assert np.abs(out[b] - want[b]).max() <= ATOL, b
    with pytest.raises(KrillError) as e:
        run(130, 8200)  # view min(8200, 8200 + 1 + 62) = 8200 > 8192
    assert e.value.code == KRILL_E_UNSUPPORTED
    pool.set_option(OPT_ATTN_PATH, 2)
    out2 = run(130, 8200)
    for b in range(2):
        assert np.abs(out2[b] - want[b]).max() <= ATOL, b
    pool.close()
