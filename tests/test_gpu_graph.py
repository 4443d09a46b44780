"""GPU: a decode step captured in a HIP graph and replayed.

A serving loop captures its per-step launches once and replays them (the
bench's decode steps do): the copy of the step's block tables and lengths
from pinned host memory, then the fused append + decode attention of every
layer, with max_seq_len an upper bound for all steps.  Each replay is checked
against the same calls issued eagerly, bit for bit, over three steps of new
tables (the sequences grow by one token per step), with eager work of the
program and synchronizations between the replays; the last step's output is
also checked against the float64 oracle (2e-3)."""
import numpy as np
import pytest

from kvutil import Filled, oracle_attention, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402

DT = "bf16"


@pytest.mark.parametrize("R", [5, 1])
def test_decode_step_graph_replays_match_eager(R):
    print(f"\ncase graph_replay R={R}", flush=True)
    rng = np.random.default_rng(41 + R)
    H, D, layers, steps = 8, 128, 2, 3
    ctx = [300, 1000, 65, 2000, 7]
    B = len(ctx)
    mb = (max(ctx) + steps + 63) // 64
    pool = krill_amd.KVPool(layers, H, D, sum((T + steps + 63) // 64 for T in ctx) + 8, "affine_g64", DT,
                            free_list_seed=11)
    f = Filled(pool, ctx, rng, DT, layers=tuple(range(layers)), max_chunk=512)
    max_len = max(ctx) + steps
    scale = 1.0 / np.sqrt(D)
    # per step and layer: the new token's K/V rows and the queries
    kn = [[rand_bits(rng, (B, H, 1, D), DT) for _ in range(layers)] for _ in range(steps)]
    vn = [[rand_bits(rng, (B, H, 1, D), DT) for _ in range(layers)] for _ in range(steps)]
    qs = [[rand_bits(rng, (B, H * R, 1, D), DT) for _ in range(layers)] for _ in range(steps)]
    # the graph's fixed buffers
    tab_h = torch.zeros((B, mb), dtype=torch.int32).pin_memory()
    len_h = torch.zeros((B,), dtype=torch.int32).pin_memory()
    tab_d = torch.zeros((B, mb), dtype=torch.int32, device="cuda")
    len_d = torch.zeros((B,), dtype=torch.int32, device="cuda")
    q_d = [torch.empty((B, H * R, 1, D), dtype=torch.bfloat16, device="cuda") for _ in range(layers)]
    k_d = [torch.empty((B, H, 1, D), dtype=torch.bfloat16, device="cuda") for _ in range(layers)]
    v_d = [torch.empty((B, H, 1, D), dtype=torch.bfloat16, device="cuda") for _ in range(layers)]
    out_g = [torch.empty((B, H * R, 1, D), dtype=torch.float32, device="cuda") for _ in range(layers)]
    ws = torch.empty(max(pool.workspace_size(B, H * R, 1, max_len), 1), dtype=torch.uint8, device="cuda")

    def step_calls(out):
        tab_d.copy_(tab_h, non_blocking=True)
        len_d.copy_(len_h, non_blocking=True)
        for layer in range(layers):
            pool.decode_append_attention(layer, q_d[layer], k_d[layer], v_d[layer], tab_d, len_d, max_len, scale,
                                         ws=ws, out=out[layer])

    def host_step(s):
        for seq in f.seqs:
            pool.reserve_append(seq, 1)
        t, n = pool.batch_tables(f.seqs, mb)
        tab_h.numpy()[:] = t
        len_h.numpy()[:] = n
        for layer in range(layers):
            q_d[layer].copy_(to_dev(qs[s][layer], DT))
            k_d[layer].copy_(to_dev(kn[s][layer], DT))
            v_d[layer].copy_(to_dev(vn[s][layer], DT))
        torch.cuda.synchronize()
        return n

    # the eager reference of step 0, then the capture (which runs nothing)
    host_step(0)
    out_e = [torch.empty_like(o) for o in out_g]
    step_calls(out_e)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream()
    with torch.cuda.graph(g, stream=cap):
        step_calls(out_g)
    torch.cuda.synchronize()

    for s in range(steps):
        if s > 0:
            host_step(s)
            step_calls(out_e)  # eager: writes the same newest tokens the replay writes again
            torch.cuda.synchronize()
        # eager work of the program between replays
        torch.randn(1 << 20, device="cuda").sum().item()
        for o in out_g:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(out_g[layer], out_e[layer]), (s, layer)
        print(f"step {s}: replay == eager", flush=True)

    # the cache after the replays: the oracle's attention over every token appended
    for s in range(steps):
        for b in range(B):
            for layer in range(layers):
                f.k[layer][b] = np.concatenate([f.k[layer][b], kn[s][layer][b]], axis=1)
                f.v[layer][b] = np.concatenate([f.v[layer][b], vn[s][layer][b]], axis=1)
    f.lens = [T + steps for T in ctx]
    for layer in range(layers):
        ref = oracle_attention(pool, f, layer, qs[steps - 1][layer], DT, scale)
        err = float(np.abs(out_g[layer].cpu().numpy() - ref).max())
        print(f"layer {layer} max abs error {err:.3e}", flush=True)
        assert err <= 2e-3
    pool.close()


def test_capture_refuses_queued_copy_on_write_and_replays_after_an_eager_flush():
    """A sequence forked from another inside a partly filled block: its first
    append queues a copy-on-write copy of that block.  Capturing a decode step
    while the copy is queued is refused (the graph would repeat the copy on
    every replay) and leaves the copy queued; after an eager flush the
    captured step replays bit for bit like the eager one, the sharer keeps its
    bytes and the fork holds the sharer's first 70 tokens plus its own."""
    from krill_amd import _lib as L
    from kvutil import MODE, check_snapshot, i32
    from oracle import oracle as O

    print("\ncase graph_cow_refused_then_flushed", flush=True)
    rng = np.random.default_rng(77)
    H, D, R, layers = 2, 128, 4, 2
    pool = krill_amd.KVPool(layers, H, D, 16, "affine_g64", DT, free_list_seed=5)
    f = Filled(pool, [100], rng, DT, layers=tuple(range(layers)))
    a = f.seqs[0]
    fork = pool.seq_fork(a, 70)  # block 1 (tokens 64..99 of a) shared, partly filled for the fork
    pool.reserve_append(fork, 1)  # position 70: copy-on-write of block 1 queued
    assert pool.stats()["cow_copies"] == 1 and pool.stats()["pending_copies"] == 1
    t, n = pool.batch_tables([fork], 2)
    tab, lens = i32(t), i32(n)
    q = [to_dev(rand_bits(rng, (1, H * R, 1, D), DT), DT) for _ in range(layers)]
    kn = [rand_bits(rng, (1, H, 1, D), DT) for _ in range(layers)]
    vn = [rand_bits(rng, (1, H, 1, D), DT) for _ in range(layers)]
    k_d = [to_dev(x, DT) for x in kn]
    v_d = [to_dev(x, DT) for x in vn]
    scale = 1.0 / np.sqrt(D)
    ws = torch.empty(max(pool.workspace_size(1, H * R, 1, 71), 1), dtype=torch.uint8, device="cuda")
    out_g = [torch.empty((1, H * R, 1, D), dtype=torch.float32, device="cuda") for _ in range(layers)]
    marker = torch.zeros(1, device="cuda")
    torch.cuda.synchronize()

    cap = torch.cuda.Stream()
    g0 = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g0, stream=cap):
        marker.add_(1.0)  # the refused capture still records a node
        with pytest.raises(L.KrillError) as ei:
            pool.decode_append_attention(0, q[0], k_d[0], v_d[0], tab, lens, 71, scale, ws=ws, out=out_g[0])
    assert ei.value.code == L.KRILL_E_STATE, str(ei.value)
    assert pool.stats()["pending_copies"] == 1  # still queued, nothing captured
    del g0

    pool.flush()  # eager: the copy runs now, outside any graph
    assert pool.stats()["pending_copies"] == 0

    def step(out):
        for layer in range(layers):
            pool.decode_append_attention(layer, q[layer], k_d[layer], v_d[layer], tab, lens, 71, scale, ws=ws,
                                         out=out[layer])

    out_e = [torch.empty_like(o) for o in out_g]
    step(out_e)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=cap):
        step(out_g)
    torch.cuda.synchronize()
    for rep in range(3):
        torch.randn(1 << 16, device="cuda").sum().item()  # eager work between replays
        for o in out_g:
            o.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(out_g[layer], out_e[layer]), (rep, layer)

    mode = MODE["affine_g64"]
    for layer in range(layers):
        ta, na = pool.batch_tables([a], 2)
        check_snapshot(pool.gather(layer, i32(ta), i32(na), 100), f, layer)  # the sharer is unchanged
        snap = pool.gather(layer, tab, lens, 71)
        kq, ks, kz, vq, vs, vz = f.expected(layer, 0)
        nk = O.quantize(kn[layer][0], O.DT_BF16, mode)
        nv = O.quantize(vn[layer][0], O.DT_BF16, mode)
        keys = snap["keys"].cpu().numpy()
        vals = snap["values"].cpu().numpy()
        np.testing.assert_array_equal(keys[0, :, :70], kq[:, :70])
        np.testing.assert_array_equal(vals[0, :, :70], vq[:, :70])
        np.testing.assert_array_equal(keys[0, :, 70:], nk[0])
        np.testing.assert_array_equal(vals[0, :, 70:], nv[0])
    pool.close()
