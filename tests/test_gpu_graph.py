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
