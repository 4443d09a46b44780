"""GPU: the decode step with the append fused (krill_decode_append_attention)
against the same step as two calls, quantize-append at the reserved slots
and then decode attention, whose parity with the oracle the other GPU tests
pin.  The pool bytes (every token, scale and zero) and the attention output
must be identical, bit for bit; one case also checks the new token's bytes
and the output against the oracle directly."""
import numpy as np
import pytest

from kvutil import DT, MODE, Filled, i32, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd import _lib  # noqa: E402

ATOL = 2e-3


def _pool(H, D, mode, dt, blocks, layers, seed, split_blocks, path):
    p = krill_amd.KVPool(layers, H, D, blocks, mode, dt, free_list_seed=seed)
    p.set_option(_lib.OPT_SPLIT_BLOCKS, split_blocks)
    p.set_option(_lib.OPT_ATTN_PATH, path)
    return p


def _step_both_ways(mode, dt, D, H, R, prefill, seed, split_blocks=0, path=0, layer=0, layers=1, skip=()):
    """Two pools with the same history; one decode step each way.  `skip`:
    sequences that take no token this step (passed with length 0)."""
    B = len(prefill)
    blocks = sum((T + 64) // 64 for T in prefill) + 8
    pools, fills = [], []
    for _ in range(2):
        p = _pool(H, D, mode, dt, blocks, layers, seed, split_blocks, path)
        fills.append(Filled(p, prefill, np.random.default_rng(seed), dt, layers=(layer,)))
        pools.append(p)
    rng = np.random.default_rng(seed + 1)
    kn = rand_bits(rng, (B, H, 1, D), dt)
    vn = rand_bits(rng, (B, H, 1, D), dt)
    q = rand_bits(rng, (B, H * R, 1, D), dt)
    lens = np.array([0 if b in skip else T + 1 for b, T in enumerate(prefill)], np.int32)
    slots = []
    for p, f in zip(pools, fills):
        sl = np.full((B, 1), -1, np.int32)
        for b in range(B):
            if b not in skip:
                sl[b, 0] = p.reserve_append(f.seqs[b], 1)[0]
        slots.append(sl)
    np.testing.assert_array_equal(slots[0], slots[1])
    full = [T + (0 if b in skip else 1) for b, T in enumerate(prefill)]  # cached tokens after the step
    mb = max(1, max((T + 63) // 64 for T in full))
    tabs = [p.batch_tables(f.seqs, mb)[0] for p, f in zip(pools, fills)]
    np.testing.assert_array_equal(tabs[0], tabs[1])
    tables, tl = i32(tabs[0]), i32(lens)
    max_len = max(1, int(lens.max()))
    scale = 1.0 / np.sqrt(D)
    qd, kd, vd = to_dev(q, dt), to_dev(kn, dt), to_dev(vn, dt)

    pools[0].quantize_append(layer, kd, vd, i32(slots[0]))
    out_two = pools[0].attention(layer, qd, tables, tl, max_len, scale)
    out_fused = pools[1].decode_append_attention(layer, qd, kd, vd, tables, tl, max_len, scale)
    torch.cuda.synchronize()
    assert torch.equal(out_two, out_fused), "fused output differs from append + attention"

    # the whole cache, both pools: every sequence's tokens up to its new length
    S = max(1, max(full))
    snaps = [p.gather(layer, tables, i32(full), S) for p in pools]
    for name in snaps[0]:
        a, b_ = snaps[0][name].cpu().numpy(), snaps[1][name].cpu().numpy()
        assert np.array_equal(a.view(np.uint8), b_.view(np.uint8)), f"pool {name} differs"
    ctx = dict(pools=pools, fills=fills, q=q, kn=kn, vn=vn, lens=lens, out=out_fused, snap=snaps[1],
               tables=tables, scale=scale)
    return ctx


def _close(ctx):
    for p in ctx["pools"]:
        p.close()


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D,R", [(128, 5), (64, 4), (256, 2), (512, 8)])
def test_fused_step_matches_two_calls(mode, dt, D, R):
    # new tokens at the last slot of a block (63, 127), the first slot of a
    # new block (64, 200 -> 201 stays inside), a sequence's first token (0)
    print(f"\ncase fused mode={mode} dt={dt} D={D} R={R}", flush=True)
    ctx = _step_both_ways(mode, dt, D, 2, R, [63, 64, 0, 200, 127, 130, 1], seed=D + R)
    _close(ctx)


@pytest.mark.parametrize("split_blocks", [1, 64])
def test_fused_step_many_sequences_per_wave(split_blocks):
    # 150 short sequences: with 64 blocks per wave one wave writes the new
    # tokens of up to 64 sequences; with 1 block per wave every wave writes
    # at most one; sequences 3 and 77 take no token this step
    print(f"\ncase fused_many sb={split_blocks}", flush=True)
    rng = np.random.default_rng(31)
    prefill = [int(x) for x in rng.integers(0, 140, size=150)]
    ctx = _step_both_ways("affine_g64", "bf16", 128, 2, 5, prefill, seed=31, split_blocks=split_blocks,
                          skip=(3, 77))
    _close(ctx)


def test_fused_step_mfma_path_and_second_layer():
    # the MFMA path writes the tokens with their own launch first
    print("\ncase fused_mfma_layer1", flush=True)
    ctx = _step_both_ways("affine_g64", "bf16", 128, 2, 5, [65, 400, 0], seed=12, path=2, layer=1, layers=2)
    _close(ctx)


def test_fused_step_qwen3_14b_shape_against_oracle():
    """Hq 40, Hkv 8, D 128, affine g64: the fused step against the oracle:
    the new token's bytes and the attention output over the extended cache."""
    print("\ncase fused_qwen3_14b_oracle", flush=True)
    dt = "bf16"
    prefill = [511, 1999, 4095, 64, 8192]
    ctx = _step_both_ways("affine_g64", dt, 128, 8, 5, prefill, seed=20261203)
    f = ctx["fills"][1]
    # extend the oracle's rows with the step's token and check its bytes
    for b, T in enumerate(prefill):
        f.k[0][b] = np.concatenate([f.k[0][b], ctx["kn"][b]], axis=1)
        f.v[0][b] = np.concatenate([f.v[0][b], ctx["vn"][b]], axis=1)
    f.lens = [T + 1 for T in prefill]
    snap = {k: v.cpu().numpy() for k, v in ctx["snap"].items()}
    for b, T in enumerate(prefill):
        kq, ks, kz, vq, vs, vz = f.expected(0, b)
        np.testing.assert_array_equal(snap["keys"][b, :, T], kq[:, T])
        np.testing.assert_array_equal(snap["values"][b, :, T], vq[:, T])
        np.testing.assert_array_equal(snap["key_scales"][b, :, T].view(np.uint16), ks[:, T])
        np.testing.assert_array_equal(snap["value_zeros"][b, :, T].view(np.uint16), vz[:, T])
    ref = oracle_attention(ctx["pools"][1], f, 0, ctx["q"], dt, ctx["scale"])
    err = np.abs(ctx["out"].float().cpu().numpy() - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"
    _close(ctx)


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R,dt", [(128, 5, "bf16"), (64, 4, "f16"), (256, 2, "bf16"), (128, 16, "bf16"),
                                    (512, 8, "bf16"), (512, 16, "f16")])
def test_fused_rope_step_matches_rope_append_and_rotated_queries(mode, D, R, dt):
    """krill_decode_append_attention_rope against krill_quantize_append_rope at
    the reserved slots + decode attention on queries rotated by the oracle
    (R = 16: more than 8 rows per KV head, the MFMA path; at D = 512 two
    row groups of 8 on the d-sliced kernel, the first writing the token)."""
    from krill_amd.pool import rope_table
    from oracle import oracle as O

    print(f"\ncase fused_rope mode={mode} D={D} R={R} dt={dt}", flush=True)
    H, seed = 2, 40 + D + R
    prefill = [70, 1, 200, 64, 517]
    B = len(prefill)
    blocks = sum((T + 64) // 64 for T in prefill) + 8
    pools, fills = [], []
    for _ in range(2):
        p = _pool(H, D, mode, dt, blocks, 1, seed, 0, 0)
        fills.append(Filled(p, prefill, np.random.default_rng(seed), dt))
        pools.append(p)
    rng = np.random.default_rng(seed + 1)
    kn = rand_bits(rng, (B, H, 1, D), dt)
    vn = rand_bits(rng, (B, H, 1, D), dt)
    q = rand_bits(rng, (B, H * R, 1, D), dt)
    lens = np.array([T + 1 for T in prefill], np.int32)
    slots = [np.stack([p.reserve_append(f.seqs[b], 1) for b in range(B)]).astype(np.int32)
             for p, f in zip(pools, fills)]
    np.testing.assert_array_equal(slots[0], slots[1])
    mb = max((T + 63) // 64 for T in lens)
    tabs = [p.batch_tables(f.seqs, mb)[0] for p, f in zip(pools, fills)]
    tables, tl = i32(tabs[0]), i32(lens)
    max_len = int(lens.max())
    cs = rope_table(max_len + 3, D, 1.0e6)
    csd = torch.from_numpy(cs).cuda()
    pos = (lens - 1).astype(np.int32)
    scale = 1.0 / np.sqrt(D)
    # two calls: RoPE append of the new rows, attention on oracle-rotated queries
    pools[0].quantize_append_rope(0, to_dev(kn, dt), to_dev(vn, dt), i32(slots[0]), i32(pos.reshape(B, 1)), csd)
    q_rot = O.rope_rows(q, DT[dt], np.broadcast_to(pos[:, None, None], (B, H * R, 1)), cs)
    out_two = pools[0].attention(0, to_dev(q_rot, dt), tables, tl, max_len, scale)
    out_fused = pools[1].decode_append_attention_rope(0, to_dev(q, dt), to_dev(kn, dt), to_dev(vn, dt), tables, tl,
                                                      max_len, scale, csd)
    torch.cuda.synchronize()
    assert torch.equal(out_two, out_fused), "fused RoPE step differs from RoPE append + attention"
    snaps = [p.gather(0, tables, tl, max_len) for p in pools]
    for name in snaps[0]:
        a, b_ = snaps[0][name].cpu().numpy(), snaps[1][name].cpu().numpy()
        assert np.array_equal(a.view(np.uint8), b_.view(np.uint8)), f"pool {name} differs"
    # and the new K bytes are the oracle's quantization of the rotated row
    kr = O.rope_rows(kn, DT[dt], np.broadcast_to(pos[:, None, None], (B, H, 1)), cs)
    kq, _, _ = O.quantize(kr, DT[dt], MODE[mode])
    got = snaps[1]["keys"].cpu().numpy()
    for b in range(B):
        np.testing.assert_array_equal(got[b, :, lens[b] - 1], kq[b, :, 0])
    for p in pools:
        p.close()
