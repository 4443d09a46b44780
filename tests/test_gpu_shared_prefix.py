"""GPU: decode attention over a shared prefix (krill_decode_attention_shared_prefix).

B sequences are forked from one prefix sequence (the reference's prefix-cache
hit: every request of a batch starts from the same cached system prompt,
PrefixCache.swift:161-170) and then each appends its own tokens.  The cascade
attends the P full prefix blocks once for all B sequences and each suffix on
its own; its output must match the oracle (2e-3 max-abs, as every attention
test) and the ordinary decode attention over the whole tables: to float32
reassociation when both run on the VALU kernel (at most 8 query rows per KV
head in the prefix pass), to 1e-3 when the prefix pass runs on MFMA (bf16
operands, the softmax weights rounded per block) and the single pass on VALU."""
import numpy as np
import pytest

from kvutil import Filled, i32, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402

ATOL = 2e-3


def _single_tol(B, R):
    return 1e-5 if B * R <= 8 else 1e-3


class _Joined(Filled):
    """Prefix rows followed by each fork's own rows, as the oracle sees them."""

    def __init__(self, pre: Filled, suf: Filled):
        self.pool, self.dt, self.layers = pre.pool, pre.dt, pre.layers
        self.seqs = suf.seqs
        self.lens = [pre.lens[0] + T for T in suf.lens]
        self.k = {l: [np.concatenate([pre.k[l][0], k], axis=1) for k in suf.k[l]] for l in self.layers}
        self.v = {l: [np.concatenate([pre.v[l][0], v], axis=1) for v in suf.v[l]] for l in self.layers}


def _forked(mode, D, H, prefix_tokens, extra, dt, seed, split_blocks=0, path=0):
    """A pool holding one prefix sequence and len(extra) forks of it, fork b
    with extra[b] tokens of its own."""
    rng = np.random.default_rng(seed)
    nb = (prefix_tokens + 63) // 64 + sum((prefix_tokens % 64 + T + 64) // 64 for T in extra) + 8
    pool = krill_amd.KVPool(1, H, D, nb, mode, dt, free_list_seed=seed)
    pool.set_option(krill_amd._lib.OPT_SPLIT_BLOCKS, split_blocks)
    pool.set_option(krill_amd._lib.OPT_ATTN_PATH, path)
    pre = Filled(pool, [prefix_tokens], rng, dt)
    forks = [pool.seq_fork(pre.seqs[0], prefix_tokens) for _ in extra]
    suf = Filled(pool, extra, rng, dt, seqs=forks)
    return pool, rng, _Joined(pre, suf)


def _split_tables(pool, seqs, P, mb):
    t, n = pool.batch_tables(seqs, mb)
    assert (t[:, :P] == t[0, :P]).all()  # the forks share the prefix blocks
    return i32(t[0, :P]), i32(np.ascontiguousarray(t[:, P:])), i32(n - 64 * P), int(n.max()) - 64 * P


def _case(mode, D, H, R, prefix_tokens, extra, dt="bf16", seed=0, split_blocks=0, out_dtype=None, path=0):
    pool, rng, joined = _forked(mode, D, H, prefix_tokens, extra, dt, seed, split_blocks, path)
    tables, lens, mb = joined.tables()
    P = prefix_tokens // 64
    t = tables.cpu().numpy()
    assert (t[:, :P] == t[0, :P]).all()  # the forks share the prefix blocks
    prefix_table = i32(t[0, :P])
    suffix_tables = i32(np.ascontiguousarray(t[:, P:]) if mb > P else np.zeros((len(extra), 1), np.int32))
    suffix_lens = lens - 64 * P
    max_suffix = int(suffix_lens.max().item())
    B = len(extra)
    q = rand_bits(rng, (B, H * R, 1, D), dt)
    scale = 1.0 / np.sqrt(D)
    qd = to_dev(q, dt)
    out = pool.attention_shared_prefix(0, qd, prefix_table, suffix_tables, suffix_lens, max_suffix, scale,
                                       out_dtype)
    whole = pool.attention(0, qd, tables, lens, max(joined.lens), scale, out_dtype)
    torch.cuda.synchronize()
    got, single = out.float().cpu().numpy(), whole.float().cpu().numpy()
    ref = oracle_attention(pool, joined, 0, q, dt, scale)
    pool.close()
    return got, single, ref


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R,extra", [
    (128, 5, [0, 1, 70, 300]),       # 20 prefix rows per KV head: MFMA prefix pass
    (128, 2, [0, 5]),                # 4 rows: VALU prefix pass
    (64, 4, [3, 64, 65, 0, 130]),    # 20 rows, D 64
    (256, 2, [1, 2, 3, 4, 5, 6, 7, 8, 9, 10]),  # 20 rows in two 16-row groups (D 256)
])
def test_shared_prefix_matches_oracle_and_single_pass(mode, D, R, extra):
    print(f"\ncase shared_prefix mode={mode} D={D} R={R} B={len(extra)}", flush=True)
    for prefix_tokens in (200, 128):  # a shared partial block in every suffix, or none
        got, single, ref = _case(mode, D, 2, R, prefix_tokens, extra, seed=D + R + prefix_tokens)
        err = np.abs(got - ref).max()
        assert err <= ATOL, f"prefix {prefix_tokens}: max abs error {err:.3e}"
        dev = np.abs(got - single).max()
        assert dev <= _single_tol(len(extra), R), f"prefix {prefix_tokens}: cascade vs single pass {dev:.3e}"


@pytest.mark.parametrize("split_blocks", [1, 3])
def test_shared_prefix_split_partials(split_blocks):
    # one block per wave: the 1500-token prefix's 23 blocks over 23 waves
    print(f"\ncase shared_prefix_split sb={split_blocks}", flush=True)
    got, single, ref = _case("affine_g64", 128, 2, 5, 1500, [10, 0, 900], seed=7, split_blocks=split_blocks)
    assert np.abs(got - ref).max() <= ATOL
    assert np.abs(got - single).max() <= _single_tol(3, 5)


def test_shared_prefix_qwen3_14b_shape():
    """Hq 40, Hkv 8, D 128, affine g64: 8 sequences behind a 4096-token prefix."""
    print("\ncase shared_prefix_qwen3_14b", flush=True)
    rng = np.random.default_rng(11)
    extra = [int(x) for x in rng.integers(1, 200, 8)]
    got, single, ref = _case("affine_g64", 128, 8, 5, 4096, extra, seed=12)
    assert np.abs(got - ref).max() <= ATOL
    assert np.abs(got - single).max() <= _single_tol(8, 5)


@pytest.mark.parametrize("out_dtype", ["bf16", "f16"])
def test_shared_prefix_low_precision_output(out_dtype):
    print(f"\ncase shared_prefix_out {out_dtype}", flush=True)
    td = torch.bfloat16 if out_dtype == "bf16" else torch.float16
    got, _, ref = _case("affine_g64", 128, 2, 5, 300, [7, 100], seed=9, out_dtype=td)
    ulp = 2.0 ** -8 if out_dtype == "bf16" else 2.0 ** -11
    err = np.abs(got - ref) - ulp * np.maximum(np.abs(ref), 1e-30)
    assert err.max() <= ATOL


def test_shared_prefix_rejects_empty_prefix_and_small_workspace():
    print("\ncase shared_prefix_errors", flush=True)
    pool = krill_amd.KVPool(1, 2, 128, 16, "affine_g64", "bf16", free_list_seed=1)
    q = torch.zeros((2, 4, 1, 128), dtype=torch.bfloat16, device="cuda")
    tabs = i32(np.zeros((2, 2), np.int32))
    lens = i32([1, 1])
    with pytest.raises(krill_amd._lib.KrillError, match="prefix_blocks"):
        pool.attention_shared_prefix(0, q, i32(np.zeros(0, np.int32)), tabs, lens, 1, 0.1)
    ws = torch.empty(16, dtype=torch.uint8, device="cuda")
    out = torch.empty((2, 4, 1, 128), dtype=torch.float32, device="cuda")
    L = krill_amd._lib
    rc = L.lib().krill_decode_attention_shared_prefix(
        pool._h, 0, q.data_ptr(), tabs.data_ptr(), 1, tabs.data_ptr(), lens.data_ptr(), 2, 2, 1, 4, 0.1,
        out.data_ptr(), L.DTYPE_F32, ws.data_ptr(), ws.numel(), None)
    assert rc == L.KRILL_E_INVAL and "workspace" in L.last_error()
    pool.close()


@pytest.mark.parametrize("path", [0, 2])
def test_shared_prefix_fused_append_bit_identical(path):
    """The append fused into the cascade (VALU suffix pass, or the MFMA one
    after its own append launch) leaves the same cache bytes and output as
    quantize-append followed by the cascade."""
    print(f"\ncase shared_prefix_fused_append path={path}", flush=True)
    D, H, R, prefix_tokens, extra = 128, 2, 5, 200, [0, 3, 64, 130]
    P, B = prefix_tokens // 64, len(extra)
    mb = (prefix_tokens + max(extra) + 1 + 63) // 64
    outs, snaps = [], []
    for fused in (False, True):
        pool, _, joined = _forked("affine_g64", D, H, prefix_tokens, extra, "bf16", seed=31, path=path)
        rng = np.random.default_rng(99)
        kn, vn = (to_dev(rand_bits(rng, (B, H, 1, D), "bf16"), "bf16") for _ in range(2))
        q = to_dev(rand_bits(rng, (B, H * R, 1, D), "bf16"), "bf16")
        slots = np.stack([pool.reserve_append(s, 1) for s in joined.seqs]).astype(np.int32)
        ptab, stab, slen, smax = _split_tables(pool, joined.seqs, P, mb)
        if fused:
            out = pool.attention_shared_prefix(0, q, ptab, stab, slen, smax, 0.1, k_new=kn, v_new=vn)
        else:
            pool.quantize_append(0, kn, vn, i32(slots))
            out = pool.attention_shared_prefix(0, q, ptab, stab, slen, smax, 0.1)
        t, n = pool.batch_tables(joined.seqs, mb)
        snap = pool.gather(0, i32(t), i32(n), int(n.max()))
        torch.cuda.synchronize()
        outs.append(out.cpu())
        snaps.append({k: v.cpu().numpy() for k, v in snap.items()})
        pool.close()
    assert torch.equal(outs[0], outs[1])
    for k in snaps[0]:
        assert np.array_equal(snaps[0][k].view(np.uint8), snaps[1][k].view(np.uint8)), k


def test_shared_prefix_f16_inputs():
    print("\ncase shared_prefix_f16", flush=True)
    got, single, ref = _case("affine_g64", 128, 2, 5, 200, [0, 9, 130], dt="f16", seed=17)
    assert np.abs(got - ref).max() <= ATOL
    assert np.abs(got - single).max() <= _single_tol(3, 5)


@pytest.mark.parametrize("prefix_split", [0, 4, 8])
def test_shared_prefix_prefix_split(prefix_split):
    """KRILL_OPT_PREFIX_SPLIT (shared-prefix blocks per workgroup of the
    prefix pass): the 65-block prefix of a Llama-3-8B-shaped batch over fewer,
    longer workgroups gives the same output call after call and stays within
    the oracle tolerance."""
    print(f"\ncase shared_prefix_split prefix_split={prefix_split}", flush=True)
    D, H, R, prefix_tokens, extra = 128, 8, 4, 4120, [0, 3, 64, 130, 900, 17, 1000, 2]
    pool, rng, joined = _forked("affine_g64", D, H, prefix_tokens, extra, "bf16", seed=61)
    P, B = prefix_tokens // 64, len(extra)
    mb = (prefix_tokens + max(extra) + 63) // 64
    ptab, stab, slen, smax = _split_tables(pool, joined.seqs, P, mb)
    q = rand_bits(rng, (B, H * R, 1, D), "bf16")
    qd = to_dev(q, "bf16")
    L = krill_amd._lib
    pool.set_option(L.OPT_PREFIX_SPLIT, prefix_split)
    outs = []
    for _ in range(2):
        outs.append(pool.attention_shared_prefix(0, qd, ptab, stab, slen, smax, 0.1))
        torch.cuda.synchronize()
    ref = oracle_attention(pool, joined, 0, q, "bf16", 0.1)
    pool.close()
    assert torch.equal(outs[0], outs[1])
    err = np.abs(outs[1].cpu().numpy() - ref).max()
    print(f"max abs error {err:.3e}", flush=True)
    assert err <= ATOL


def test_shared_prefix_graph_replays_match_eager():
    """A cascade call (prefix pass, suffix pass, merge) captured in a HIP
    graph on a side stream and replayed three times, with eager work and
    synchronizations between the replays: every replay equals the eager call
    bit for bit."""
    print("\ncase shared_prefix_graph", flush=True)
    D, H, R, prefix_tokens, extra = 128, 4, 4, 1000, [5, 300, 0, 77]
    pool, rng, joined = _forked("affine_g64", D, H, prefix_tokens, extra, "bf16", seed=67)
    P, B = prefix_tokens // 64, len(extra)
    mb = (prefix_tokens + max(extra) + 63) // 64
    ptab, stab, slen, smax = _split_tables(pool, joined.seqs, P, mb)
    qd = to_dev(rand_bits(rng, (B, H * R, 1, D), "bf16"), "bf16")
    ws = torch.empty(max(pool.shared_prefix_workspace_size(B, H * R, P, smax), 1), dtype=torch.uint8, device="cuda")
    out_e = pool.attention_shared_prefix(0, qd, ptab, stab, slen, smax, 0.1, ws=ws)
    torch.cuda.synchronize()
    out_g = torch.empty_like(out_e)
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=cap):
        pool.attention_shared_prefix(0, qd, ptab, stab, slen, smax, 0.1, ws=ws, out=out_g)
    torch.cuda.synchronize()
    for rep in range(3):
        torch.randn(1 << 20, device="cuda").sum().item()
        out_g.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out_g, out_e), rep
    pool.close()
