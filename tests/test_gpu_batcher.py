"""GPU: the epoch-free continuous batcher end to end.  Requests arrive at
different steps, prefill in chunks, decode in a batch whose membership
changes at every admission and retirement; every attention output (prefill
rows and decode rows, every layer) must match the oracle's attention over
that request's own tokens, run in a batch or alone, and every block must be
back in the pool at the end."""
import numpy as np
import pytest

from kvutil import DT, MODE, rand_bits, to_dev
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd.batcher import ContinuousBatcher, Request  # noqa: E402

ATOL = 2e-3
H, R, D, LAYERS, DTS = 2, 2, 128, 2, "bf16"


class SynthModel:
    """Projections of request rid at position p, layer l: fixed seeded rows
    (independent of batching), attention outputs recorded per (rid, l, p)."""

    def __init__(self, reqs, seed=0):
        self.q, self.k, self.v, self.out = {}, {}, {}, {}
        for r in reqs:
            T = r.prompt_len + r.max_new_tokens
            rng = np.random.default_rng(seed * 1000 + r.rid)
            for l in range(LAYERS):
                self.q[r.rid, l] = rand_bits(rng, (H * R, T, D), DTS)
                self.k[r.rid, l] = rand_bits(rng, (H, T, D), DTS)
                self.v[r.rid, l] = rand_bits(rng, (H, T, D), DTS)

    def prefill(self, req, start, n, layer):
        sl = slice(start, start + n)
        return tuple(to_dev(a[req.rid, layer][None, :, sl], DTS) for a in (self.q, self.k, self.v))

    def decode(self, reqs, positions, layer):
        return tuple(to_dev(np.stack([a[r.rid, layer][:, p: p + 1] for r, p in zip(reqs, positions)]), DTS)
                     for a in (self.q, self.k, self.v))

    def consume(self, reqs, layer, positions, out):
        o = out.float().cpu().numpy()
        if len(reqs) == 1 and o.shape[2] == len(positions):  # prefill chunk: [1, Hq, n, D]
            for j, p in enumerate(positions):
                self.out[reqs[0].rid, layer, int(p)] = o[0, :, j]
        else:  # decode: [B, Hq, 1, D]
            for b, (r, p) in enumerate(zip(reqs, positions)):
                self.out[r.rid, layer, int(p)] = o[b, :, 0]


def _oracle(model, req, layer, scale):
    T = req.prompt_len + req.max_new_tokens
    mode = MODE["affine_g64"]
    kd = O.dequant_f64(*O.quantize(model.k[req.rid, layer], DT[DTS], mode), mode)
    vd = O.dequant_f64(*O.quantize(model.v[req.rid, layer], DT[DTS], mode), mode)
    qf = O.bits_to_f32(model.q[req.rid, layer], DT[DTS]).astype(np.float64)
    out = np.zeros((H * R, T, D))
    for hk in range(H):
        rows = np.concatenate([qf[hk * R + h] for h in range(R)])  # [R*T, D], head-major
        lim = [t + 1 for h in range(R) for t in range(T)]
        o = O.attention_f64(rows, kd[hk], vd[hk], lim, scale)
        for h in range(R):
            out[hk * R + h] = o[h * T:(h + 1) * T]
    return out


def _run(reqs, arrivals, max_rows, prefill_chunk, seed=0, stream=None):
    model = SynthModel(reqs, seed)
    blocks = sum((r.prompt_len + r.max_new_tokens + 63) // 64 for r in reqs) + 4
    pool = krill_amd.KVPool(LAYERS, H, D, blocks, "affine_g64", DTS, free_list_seed=seed + 1)
    scale = 1.0 / np.sqrt(D)
    cb = ContinuousBatcher(pool, model, max_rows, H * R, scale, prefill_chunk=prefill_chunk,
                           out_dtype=torch.float32, stream=stream)
    step = 0
    while step < 1000:
        for r in arrivals.get(step, []):
            cb.submit(r)
        if cb.idle and step > max(arrivals):
            break
        cb.step()
        step += 1
    torch.cuda.synchronize()
    stats = pool.stats()
    pool.close()
    return model, stats, cb


def _requests():
    spec = [(0, 70, 5), (1, 5, 9), (2, 130, 3), (3, 64, 6), (4, 1, 4), (5, 200, 2)]
    return [Request(rid, T, g) for rid, T, g in spec]


def test_batcher_staggered_arrivals_match_oracle():
    print("\ncase batcher_staggered", flush=True)
    reqs = _requests()
    arrivals = {0: reqs[:3], 2: reqs[3:4], 4: reqs[4:5], 5: reqs[5:]}
    model, stats, cb = _run(reqs, arrivals, max_rows=3, prefill_chunk=48)
    assert stats["blocks_used"] == 0 and stats["live_seqs"] == 0
    assert cb.admitted == len(reqs) and cb.retired == len(reqs)
    scale = 1.0 / np.sqrt(D)
    for r in reqs:
        T = r.prompt_len + r.max_new_tokens
        for l in range(LAYERS):
            want = _oracle(model, r, l, scale)
            # positions 0 .. prompt-1 from the prefill chunks, the rest from decode steps
            got = np.stack([model.out[r.rid, l, p] for p in range(T)], axis=1)
            err = np.abs(got - want).max()
            assert err <= ATOL, (r.rid, l, err)


def test_batched_equals_alone():
    print("\ncase batcher_alone", flush=True)
    reqs = _requests()
    batched, _, _ = _run(reqs, {0: reqs[:4], 3: reqs[4:]}, max_rows=4, prefill_chunk=64)
    reqs2 = _requests()
    alone, _, _ = _run(reqs2, {0: reqs2}, max_rows=1, prefill_chunk=64)
    assert batched.out.keys() == alone.out.keys()
    dev = max(np.abs(batched.out[k] - alone.out[k]).max() for k in batched.out)
    assert dev <= 1e-5, dev


def test_batcher_on_its_own_stream_matches_the_current_stream():
    # the whole step (inputs, table uploads, workspace, kernels) on a side
    # stream (default priority): the same outputs as on torch's current stream
    print("\ncase batcher_stream", flush=True)
    arrivals = lambda rq: {0: rq[:3], 2: rq[3:]}  # noqa: E731
    reqs = _requests()
    cur, _, _ = _run(reqs, arrivals(reqs), max_rows=3, prefill_chunk=48)
    reqs2 = _requests()
    side, stats, _ = _run(reqs2, arrivals(reqs2), max_rows=3, prefill_chunk=48, stream=torch.cuda.Stream())
    assert stats["blocks_used"] == 0
    assert cur.out.keys() == side.out.keys()
    for k in cur.out:
        assert np.array_equal(cur.out[k], side.out[k]), k


def test_cancel_frees_blocks():
    print("\ncase batcher_cancel", flush=True)
    reqs = [Request(0, 100, 50), Request(1, 30, 50), Request(2, 10, 2)]
    model = SynthModel(reqs)
    pool = krill_amd.KVPool(LAYERS, H, D, 16, "affine_g64", DTS, free_list_seed=2)
    cb = ContinuousBatcher(pool, model, 2, H * R, 0.1, out_dtype=torch.float32)
    for r in reqs:
        cb.submit(r)
    cb.step()
    used = pool.stats()["blocks_used"]
    assert used == (100 + 1 + 63) // 64 + (30 + 1 + 63) // 64
    cb.cancel(0)
    cb.step()  # row 0 leaves, request 2 joins
    assert [r.req.rid for r in cb.rows] == [1, 2]
    cb.cancel(1)
    cb.run()
    torch.cuda.synchronize()
    assert pool.stats()["blocks_used"] == 0 and cb.idle
    pool.close()
