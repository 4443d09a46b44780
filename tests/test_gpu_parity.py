"""GPU parity: every kernel through the C ABI against the CPU oracle.

Bit-exact for quantize-append / gather / scatter / COW (integer and byte
work); attention within 2e-3 max-abs of the float64 oracle (fp32 output)."""
import numpy as np
import pytest

from kvutil import DT, MODE, Filled, check_snapshot, i32, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from oracle import oracle as O  # noqa: E402

ATOL = 2e-3


def make_pool(H, D, mode, dt, blocks=64, layers=1, seed=11, **kw):
    return krill_amd.KVPool(layers, H, D, blocks, mode, dt, free_list_seed=seed, **kw)


def gpu(t):
    return t.cpu().numpy()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D", [64, 128, 256, 512])
def test_quantize_append_bit_exact(mode, dt, D):
    print(f"\ncase quantize_append mode={mode} dt={dt} D={D}", flush=True)
    rng = np.random.default_rng(100 + D)
    pool = make_pool(3, D, mode, dt, blocks=40)
    f = Filled(pool, [1, 64, 137, 5], rng, dt, outlier_frac=0.05)
    tables, lens, _ = f.tables()
    torch.cuda.synchronize()
    check_snapshot(pool.gather(0, tables, lens, max(f.lens)), f, 0)
    pool.close()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
@pytest.mark.parametrize("D", [64, 128, 256, 512])
def test_bulk_append_block_staging_bit_exact(mode, D):
    # appends of up to 200 rows (the 64-row chunks staged per block in LDS):
    # sequences starting at block edges and inside blocks, chunks straddling
    # two blocks, short sequences padded with slot -1 (the per-row path)
    print(f"\ncase bulk_append mode={mode} D={D}", flush=True)
    rng = np.random.default_rng(300 + D)
    pool = make_pool(2, D, mode, "bf16", blocks=64)
    f = Filled(pool, [1, 63, 64, 65, 127, 300, 517], rng, "bf16", max_chunk=200, outlier_frac=0.02)
    tables, lens, _ = f.tables()
    torch.cuda.synchronize()
    check_snapshot(pool.gather(0, tables, lens, max(f.lens)), f, 0)
    pool.close()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
def test_gather_left_padded_matches_reference_stack(mode):
    print(f"\ncase gather_left_pad mode={mode}", flush=True)
    rng = np.random.default_rng(5)
    H, D = 2, 128
    pool = make_pool(H, D, mode, "bf16", blocks=24)
    f = Filled(pool, [70, 3, 128, 65], rng, "bf16")
    tables, lens, _ = f.tables()
    sMax = max(f.lens)
    snap = pool.gather(0, tables, lens, sMax, left_pad=True)
    torch.cuda.synchronize()
    check_snapshot(snap, f, 0, left_pad=True)
    # the reference's own stacker on the oracle rows (BatchedDecode.swift:96-151)
    exp = [f.expected(0, b) for b in range(len(f.lens))]
    oq, os_, oz = O.stack_left_padded([e[0] for e in exp], [e[1] for e in exp], [e[2] for e in exp], f.lens, sMax)
    np.testing.assert_array_equal(gpu(snap["keys"]), oq)
    np.testing.assert_array_equal(gpu(snap["key_scales"]).view(np.uint16), os_)
    np.testing.assert_array_equal(gpu(snap["key_zeros"]).view(np.uint16), oz)
    pool.close()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
def test_scatter_restores_snapshot_bit_exact(mode):
    print(f"\ncase scatter mode={mode}", flush=True)
    rng = np.random.default_rng(8)
    H, D = 2, 64
    pool = make_pool(H, D, mode, "f16", blocks=32)
    f = Filled(pool, [90, 17], rng, "f16")
    tables, lens, _ = f.tables()
    S = max(f.lens)
    snap = pool.gather(0, tables, lens, S, left_pad=True)
    # restore each row's own slice (scatterBack, ContinuousBatcher.swift:743-801) into fresh sequences
    new = [pool.seq_create() for _ in f.lens]
    Lmax = S
    slots = np.full((len(f.lens), Lmax), -1, np.int32)
    for b, T in enumerate(f.lens):
        slots[b, :T] = pool.reserve_append(new[b], T)
    starts = np.array([S - T for T in f.lens], np.int32)
    pool.scatter(0, snap, i32(starts), i32(slots))
    t2, n2 = pool.batch_tables(new, (S + 63) // 64)
    snap2 = pool.gather(0, i32(t2), i32(n2), S)
    torch.cuda.synchronize()
    check_snapshot(snap2, f, 0)
    pool.close()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
def test_scatter_at_unaligned_offset_and_whole_blocks(mode):
    """Rows restored behind 10 existing tokens (chunks straddle blocks: the
    row path) and into a fresh sequence (whole blocks: the block path) leave
    the same bytes as the source."""
    print(f"\ncase scatter_offset mode={mode}", flush=True)
    rng = np.random.default_rng(21)
    H, D = 2, 128
    pool = make_pool(H, D, mode, "bf16", blocks=40)
    f = Filled(pool, [300], rng, "bf16")
    tables, lens, _ = f.tables()
    snap = pool.gather(0, tables, lens, 300)
    head = Filled(pool, [10], rng, "bf16")
    dst = head.seqs[0]
    fresh = pool.seq_create()
    slots = np.stack([pool.reserve_append(dst, 300), pool.reserve_append(fresh, 300)])
    snap2 = {k: torch.cat([v, v]) for k, v in snap.items()}
    pool.scatter(0, snap2, i32([0, 0]), i32(slots))
    t2, n2 = pool.batch_tables([dst, fresh], (310 + 63) // 64)
    got = pool.gather(0, i32(t2), i32(n2), 310)
    torch.cuda.synchronize()
    for k in snap:
        a = snap[k].cpu().numpy()[0].view(np.uint8)
        assert np.array_equal(got[k].cpu().numpy()[0, :, 10:310].view(np.uint8), a), k
        assert np.array_equal(got[k].cpu().numpy()[1, :, :300].view(np.uint8), a), k
    pool.close()


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
def test_gather_dequant_matches_oracle(mode):
    print(f"\ncase gather_dequant mode={mode}", flush=True)
    rng = np.random.default_rng(9)
    H, D = 2, 128
    pool = make_pool(H, D, mode, "bf16", blocks=16)
    f = Filled(pool, [33, 100], rng, "bf16")
    tables, lens, _ = f.tables()
    k, v = pool.gather_dequant(0, tables, lens, 100)
    k, v = gpu(k).view(np.uint16), gpu(v).view(np.uint16)
    for b, T in enumerate(f.lens):
        kq, ks, kz, vq, vs, vz = f.expected(0, b)
        if mode == "ref_row":
            ek, ev = O.dequant_ref_f16(kq, ks, kz), O.dequant_ref_f16(vq, vs, vz)
        else:
            ek = O.f32_to_f16_bits(O.dequant_f64(kq, ks, kz, 1))
            ev = O.f32_to_f16_bits(O.dequant_f64(vq, vs, vz, 1))
        np.testing.assert_array_equal(k[b, :, :T], ek)
        np.testing.assert_array_equal(v[b, :, :T], ev)
    pool.close()


def _attn_case(mode, D, H, R, lens, Lq=1, dt="bf16", split_blocks=0, path=0, out_dtype=None, seed=0,
               outlier_frac=0.0, scale=None):
    rng = np.random.default_rng(seed)
    nb = sum((T + 63) // 64 for T in lens) + 8
    pool = make_pool(H, D, mode, dt, blocks=nb)
    pool.set_option(krill_amd._lib.OPT_SPLIT_BLOCKS, split_blocks)
    pool.set_option(krill_amd._lib.OPT_ATTN_PATH, path)
    f = Filled(pool, lens, rng, dt, outlier_frac=outlier_frac)
    tables, tl, _ = f.tables()
    q = rand_bits(rng, (len(lens), H * R, Lq, D), dt)
    scale = 1.0 / np.sqrt(D) if scale is None else scale
    out = pool.attention(0, to_dev(q, dt), tables, tl, max(lens), scale, out_dtype)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = oracle_attention(pool, f, 0, q, dt, scale)
    pool.close()
    return got, ref


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R", [(128, 5), (64, 4), (128, 8), (256, 2), (128, 1), (512, 8), (512, 1)])
def test_decode_attention_valu(mode, D, R):
    print(f"\ncase decode_valu mode={mode} D={D} R={R}", flush=True)
    got, ref = _attn_case(mode, D, 2, R, [1, 63, 64, 65, 300, 700], seed=D + R)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R,Lq,dt", [(128, 3, 1, "bf16"), (128, 6, 1, "f16"), (128, 7, 1, "bf16"),
                                       (128, 2, 2, "f16"), (128, 1, 3, "bf16"), (128, 2, 3, "bf16"),
                                       (512, 3, 1, "bf16"), (512, 6, 1, "f16")])
def test_decode_attention_matrix_core_scores_rows(mode, D, R, Lq, dt):
    """Every row count of the decode kernel's matrix-core scores (3-8 rows
    per KV head at head_dim 128, 1-8 per row group at 512): the S^T tiles
    carry 16 rows, the rows past R * Lq are zero operands, and the sums go
    back to one token per lane through LDS; short query chunks (Lq > 1) mix
    causal limits into the rows."""
    print(f"\ncase decode_msc mode={mode} D={D} R={R} Lq={Lq} dt={dt}", flush=True)
    got, ref = _attn_case(mode, D, 2, R, [Lq, 63, 64, 65, 300, 700], Lq=Lq, dt=dt, path=1, seed=D + 7 * R + Lq)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("split_blocks", [1, 2, 3])
def test_decode_attention_split_merge(split_blocks):
    print(f"\ncase decode_split sb={split_blocks}", flush=True)
    got, ref = _attn_case("affine_g64", 128, 2, 5, [1, 200, 513, 1000], split_blocks=split_blocks, seed=3)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
def test_decode_attention_many_partials(mode):
    # one block per wave: the 5000-token sequence spreads over 79 waves, so
    # the merge walks more than 64 partial slots; the empty sequence and the
    # sequences around it cross wave boundaries at different offsets
    print(f"\ncase decode_many_partials mode={mode}", flush=True)
    got, ref = _attn_case(mode, 128, 2, 5, [70, 0, 5000, 130, 64], split_blocks=1, seed=5)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("R", [5, 1])
def test_decode_attention_any_workspace_contents(R):
    """Callers reuse one workspace across calls without clearing it: whatever
    it holds before the call (zeros, all ones, 0x7F bytes, random bytes, the
    previous call's partials) the output is the same, bit for bit, and within
    the bound of the float64 oracle.  The automatic split over many ragged
    and empty sequences puts wave and sequence boundaries at many offsets."""
    print(f"\ncase decode_any_workspace R={R}", flush=True)
    rng = np.random.default_rng(77 + R)
    H, D, dt = 2, 128, "bf16"
    lens = [int(x) for x in rng.integers(1, 1500, size=40)] + [0, 64, 65, 1]
    pool = make_pool(H, D, "affine_g64", dt, blocks=sum((T + 63) // 64 for T in lens) + 8)
    f = Filled(pool, lens, rng, dt)
    tables, tl, _ = f.tables()
    qb = rand_bits(rng, (len(lens), H * R, 1, D), dt)
    q = to_dev(qb, dt)
    need = pool.workspace_size(len(lens), H * R, 1, max(lens))
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    outs = []
    for fill in ("zeros", "ones", "0x7f", "random", "previous"):
        if fill == "zeros":
            ws.zero_()
        elif fill == "ones":
            ws.fill_(0xFF)
        elif fill == "0x7f":
            ws.fill_(0x7F)
        elif fill == "random":
            ws.copy_(torch.from_numpy(rng.integers(0, 256, size=need, dtype=np.uint8)).cuda())
        out = pool.attention(0, q, tables, tl, max(lens), 1.0 / np.sqrt(D), ws=ws)
        torch.cuda.synchronize()
        outs.append(out.float().cpu().numpy())
        print(f"workspace {fill}: done", flush=True)
    for o in outs[1:]:
        assert np.array_equal(o, outs[0])
    ref = oracle_attention(pool, f, 0, qb, dt, 1.0 / np.sqrt(D))
    err = np.abs(outs[0] - ref).max()
    pool.close()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("out_dtype", ["bf16", "f16"])
def test_decode_attention_low_precision_output(out_dtype):
    print(f"\ncase decode_out {out_dtype}", flush=True)
    td = torch.bfloat16 if out_dtype == "bf16" else torch.float16
    got, ref = _attn_case("affine_g64", 128, 2, 5, [77, 300], out_dtype=td, seed=4)
    # output rounding (half an ulp of the output dtype) on top of the 2e-3 bound
    ulp = 2.0 ** -8 if out_dtype == "bf16" else 2.0 ** -11
    err = np.abs(got - ref) - 0.5 * ulp * np.maximum(np.abs(ref), 1e-30) * 2
    assert err.max() <= ATOL


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D", [128, 64])
def test_verify_attention_mfma_causal(mode, D):
    print(f"\ncase verify_mfma mode={mode} D={D}", flush=True)
    got, ref = _attn_case(mode, D, 2, 4, [9, 64, 200, 1030], Lq=8, seed=21 + D)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D,R,Lq", [(128, 5, 5), (64, 3, 6), (128, 2, 16), (64, 17, 1)])
def test_verify_attention_token_split_partial_rows(mode, D, R, Lq):
    # 17-32 rows per KV head: one 32-row group whose two waves split the
    # tokens; here with 18-32 valid rows, edge and split blocks, ragged lengths
    print(f"\ncase verify_token_split mode={mode} D={D} R={R} Lq={Lq}", flush=True)
    got, ref = _attn_case(mode, D, 2, R, [Lq, 40, 64, 65, 129, 700], Lq=Lq, split_blocks=2 if R == 2 else 0,
                          seed=3 * R + Lq)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_verify_attention_mfma_splits_and_row_groups():
    print("\ncase verify_mfma_rowgroups", flush=True)
    # 16 draft rows x 5 heads = 80 rows -> several row groups; small splits
    got, ref = _attn_case("affine_g64", 128, 2, 5, [40, 300, 777], Lq=16, split_blocks=2, seed=5)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("mode", ["affine_g64", "ref_row"])
@pytest.mark.parametrize("D", [128, 64])
def test_prefill_chunk_32_row_waves(mode, D):
    """A prefill chunk of 32 positions x 5 query heads per KV head (160 rows)
    over a batch long enough (8 x 129 blocks of max_seq_len) that every
    workgroup of the 32-row grid streams at least 16 blocks: 32-row waves
    (two MFMA row tiles per converted byte) in groups of four, five row
    groups, so the second group holds one row group and three spare waves;
    causal rows, ragged lengths, edge blocks."""
    print(f"\ncase prefill_rows32 mode={mode} D={D}", flush=True)
    got, ref = _attn_case(mode, D, 8, 5, [8200, 2500, 900, 65, 4000, 7000, 130, 3000], Lq=32, seed=61 + D)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_verify_attention_valu_small_rows():
    print("\ncase verify_valu", flush=True)
    got, ref = _attn_case("affine_g64", 128, 2, 2, [10, 130], Lq=3, seed=6)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_decode_via_mfma_path_matches_valu():
    print("\ncase decode_mfma_forced", flush=True)
    got, ref = _attn_case("affine_g64", 128, 2, 5, [65, 400], path=2, seed=12)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_copy_on_write_preserves_the_sharer():
    print("\ncase cow", flush=True)
    rng = np.random.default_rng(13)
    H, D, dt = 2, 128, "bf16"
    pool = make_pool(H, D, "affine_g64", dt, blocks=16, layers=2)
    f = Filled(pool, [100], rng, dt, layers=(0, 1))
    a = f.seqs[0]
    fork = pool.seq_fork(a, 70)  # shares blocks 0 (full) and 1 (tokens 64..69 of 36 filled)
    extra_k = rand_bits(rng, (1, H, 5, D), dt)
    extra_v = rand_bits(rng, (1, H, 5, D), dt)
    slots = pool.reserve_append(fork, 5)  # tail block shared -> copy-on-write
    assert pool.stats()["cow_copies"] == 1
    for layer in (0, 1):
        pool.quantize_append(layer, to_dev(extra_k, dt), to_dev(extra_v, dt), i32(slots.reshape(1, 5)))
    for layer in (0, 1):
        # the sharer is unchanged
        t, n = pool.batch_tables([a], 2)
        check_snapshot(pool.gather(layer, i32(t), i32(n), 100), f, layer)
        # the fork = first 70 tokens of a + the 5 new ones
        t2, n2 = pool.batch_tables([fork], 2)
        snap = pool.gather(layer, i32(t2), i32(n2), 75)
        kq, ks, kz, vq, vs, vz = f.expected(layer, 0)
        mode = MODE["affine_g64"]
        nk = O.quantize(extra_k[0], DT[dt], mode)
        np.testing.assert_array_equal(gpu(snap["keys"])[0, :, :70], kq[:, :70])
        np.testing.assert_array_equal(gpu(snap["keys"])[0, :, 70:], nk[0])
        np.testing.assert_array_equal(gpu(snap["key_scales"])[0, :, 70:].view(np.uint16), nk[1])
    pool.close()


def test_qwen3_14b_shape_decode_step():
    """Config 2 shapes (Hq 40, Hkv 8, D 128, affine g64) on 4 ragged sequences."""
    print("\ncase qwen3_14b_shape", flush=True)
    got, ref = _attn_case("affine_g64", 128, 8, 5, [512, 1999, 4096, 8193], seed=20261203)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_outlier_channels_long_context_shape():
    """Config 5 flavour: Hkv 4, R 8, 1% channels x20, long context."""
    print("\ncase outliers_long", flush=True)
    got, ref = _attn_case("affine_g64", 128, 4, 8, [9000, 20000], seed=20261205, outlier_frac=0.01)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


def test_long_context_uniform_keys_give_mean_of_values():
    """Full long-context size (131072 tokens, the 128k MoE shape: Hkv 4, 8
    query rows per KV head): with every key row equal all scores are equal,
    so the output is the mean of the dequantized value rows -- a closed form
    that checks the split over hundreds of waves and the merge at full size."""
    print("\ncase long_context_uniform_keys", flush=True)
    H, R, D = 4, 8, 128
    lens = [131072, 65537]
    rng = np.random.default_rng(20261205)
    pool = make_pool(H, D, "affine_g64", "bf16", blocks=sum((T + 63) // 64 for T in lens) + 4)
    seqs = [pool.seq_create() for _ in lens]
    krow = rand_bits(rng, (H, 1, D), "bf16")
    vals = []
    C = 4096
    for s, T in zip(seqs, lens):
        v = rand_bits(rng, (H, T, D), "bf16", outlier_frac=0.01)
        vals.append(v)
        for t0 in range(0, T, C):
            n = min(C, T - t0)
            slots = pool.reserve_append(s, n)
            k = np.ascontiguousarray(np.broadcast_to(krow, (H, n, D)))
            pool.quantize_append(0, to_dev(k[None], "bf16"), to_dev(v[None, :, t0:t0 + n], "bf16"), i32(slots[None]))
    t, n = pool.batch_tables(seqs, (max(lens) + 63) // 64)
    q = rand_bits(rng, (len(lens), H * R, 1, D), "bf16")
    out = pool.attention(0, to_dev(q, "bf16"), i32(t), i32(n), max(lens), 1.0 / np.sqrt(D))
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    mode = MODE["affine_g64"]
    for b, v in enumerate(vals):
        vq, vs, vz = O.quantize(v, DT["bf16"], mode)
        mean = O.dequant_f64(vq, vs, vz, mode).mean(axis=1)  # [H, D]
        want = np.repeat(mean, R, axis=0)                     # query head hq reads KV head hq // R
        err = np.abs(got[b, :, 0] - want).max()
        assert err <= ATOL, (b, err)
    pool.close()


def test_chunked_prefill_512_rows():
    """A 512-token prefill chunk on top of a cache (5 query heads per KV
    head: 2560 rows per KV head in 80 row groups of 32 on the MFMA path),
    causal inside the chunk."""
    print("\ncase chunked_prefill_512", flush=True)
    got, ref = _attn_case("affine_g64", 128, 2, 5, [600, 1100], Lq=512, seed=31)
    err = np.abs(got - ref).max()
    assert err <= ATOL, f"max abs error {err:.3e}"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_decode_attention_against_the_reference_op_by_op_sdpa(dt):
    """The reference's own cache (row mode) and its SDPA arithmetic: the
    kernel against MLX's op-by-op SDPA over the dequantized fp16 cache
    (oracle.attention_mlx_composed: fp16 products for fp16 queries, float32
    for bf16), Qwen3-14B heads, within 2e-3; prints how far each sits from
    the float64 result."""
    print(f"\ncase decode_vs_mlx_composed dt={dt}", flush=True)
    H, R, D = 8, 5, 128
    lens = [511, 2049, 64, 3000]
    rng = np.random.default_rng(77)
    pool = make_pool(H, D, "ref_row", dt, blocks=sum((T + 63) // 64 for T in lens) + 8)
    f = Filled(pool, lens, rng, dt, max_chunk=512)
    tables, tl, _ = f.tables()
    q = rand_bits(rng, (len(lens), H * R, 1, D), dt)
    scale = 1.0 / np.sqrt(D)
    out = pool.attention(0, to_dev(q, dt), tables, tl, max(lens), scale)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref64 = oracle_attention(pool, f, 0, q, dt, scale)
    mlx = np.zeros_like(ref64)
    for b, T in enumerate(lens):
        kq, ks, kz, vq, vs, vz = f.expected(0, b)
        k16, v16 = O.dequant_ref_f16(kq, ks, kz), O.dequant_ref_f16(vq, vs, vz)
        for hk in range(H):
            rows = q[b, hk * R:(hk + 1) * R, 0]
            mlx[b, hk * R:(hk + 1) * R, 0] = O.attention_mlx_composed(rows, DT[dt], k16[hk], v16[hk], [T] * R,
                                                                      scale)
    e_kernel, e_mlx, e_between = (np.abs(got - ref64).max(), np.abs(mlx - ref64).max(), np.abs(got - mlx).max())
    print(f"kernel-f64 {e_kernel:.3e}  mlx_composed-f64 {e_mlx:.3e}  kernel-mlx_composed {e_between:.3e}",
          flush=True)
    assert e_kernel <= ATOL and e_between <= ATOL
    pool.close()
