"""Benchmark of the int8 paged KV hot path on one MI355X.

A step is one pass of the hot path over one batch, for every layer, plus the
host block-manager work of the step (slot reservation, block tables, rollback)
and its small host->device copies:
- decode workloads: quantize-append one new token per sequence into the
  paged pool and paged int8 decode attention over each sequence's whole
  cache (one fused call per layer; --unfused: the two calls);
- verify: quantize-append k draft tokens per sequence, causal verify
  attention of the k rows over the cache (MFMA path), then the host rolls
  each sequence back to its accepted length;
- shared prefix: decode steps of sequences forked from one refcounted
  prefix (copy-on-write of the shared partial block, LRU eviction of
  unreferenced prefix entries at 90 % occupancy); attention as the
  shared-prefix cascade (--single-pass: one decode attention over the
  whole tables).

Default workload: Qwen3-14B-shaped KV (40 layers, 40 query / 8 KV heads,
head_dim 128), affine int8 in groups of 64 with fp16 scale/bias, batch 32,
context lengths uniform in [512, 8192], 64-token blocks whose ids are a
seeded random permutation of the pool, bf16 N(0,1) inputs resident in HBM.

Synthetic inputs: Philox4x32-10 (Salmon et al., SC'11), key (seed, stream),
counters 0, 1, 2, ...; N(0,1) by Box-Muller in float64, rounded to float32
and then (RNE) to bf16; context lengths and other integer draws from the
same generator.  Seed = 20261201 + the workload's configuration index.

Prints one JSON line.
"""
from __future__ import annotations

import argparse
import ctypes
import gc
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

# ---------------------------------------------------------------- inputs
_M32 = 0xFFFFFFFF


def philox4x32_10(c0, c1, c2, c3, k0: int, k1: int):
    """Philox4x32-10 on int64 tensors holding uint32 words (the 64-bit
    products wrap in int64 with their bits intact): ten rounds of
    (c0, c1, c2, c3) <- (hi(M1 c2) ^ c1 ^ k0, lo(M1 c2), hi(M0 c0) ^ c3 ^ k1,
    lo(M0 c0)), the key bumped by the Weyl constants between rounds."""
    for _ in range(10):
        p0 = c0 * 0xD2511F53
        p1 = c2 * 0xCD9E8D57
        c0, c1, c2, c3 = ((p1 >> 32) & _M32) ^ c1 ^ k0, p1 & _M32, ((p0 >> 32) & _M32) ^ c3 ^ k1, p0 & _M32
        k0 = (k0 + 0x9E3779B9) & _M32
        k1 = (k1 + 0xBB67AE85) & _M32
    return c0, c1, c2, c3


class Philox:
    """One input stream: key (seed, stream), 64-bit counters from 0; each
    counter gives four uint32 words.  Uniforms are word / 2^32; normals come
    four per counter from Box-Muller on (w0, w1) and (w2, w3):
    sqrt(-2 ln((w0 + 1) / 2^32)) * (cos, sin)(2 pi w1 / 2^32), in float64,
    rounded to float32."""

    def __init__(self, seed: int, stream: int, device="cpu"):
        self.k0, self.k1, self.pos, self.device = seed & _M32, stream & _M32, 0, device

    def _words(self, n_ctr: int):
        import torch

        c = torch.arange(self.pos, self.pos + n_ctr, dtype=torch.int64, device=self.device)
        self.pos += n_ctr
        z = torch.zeros_like(c)
        return torch.stack(philox4x32_10(c & _M32, (c >> 32) & _M32, z, z, self.k0, self.k1), dim=-1)

    def uniform(self, n: int):
        return self._words((n + 3) // 4).reshape(-1)[:n].double() * 2.0 ** -32

    def integers(self, low: int, high: int, size=None):
        """size integers in [low, high) (high exclusive, as numpy's); one int
        without a size."""
        import torch

        u = self.uniform(1 if size is None else int(size)).cpu()
        r = (low + torch.floor(u * (high - low)).long()).numpy().astype(np.int64)
        return int(r[0]) if size is None else r

    def normal(self, shape):
        """float32 N(0, 1) tensor of `shape` on the stream's device."""
        import torch

        n = int(np.prod(shape))
        w = self._words((n + 3) // 4).double()
        r1 = torch.sqrt(-2.0 * torch.log((w[:, 0] + 1.0) * 2.0 ** -32))
        r2 = torch.sqrt(-2.0 * torch.log((w[:, 2] + 1.0) * 2.0 ** -32))
        a1, a2 = (2.0 * math.pi * 2.0 ** -32) * w[:, 1], (2.0 * math.pi * 2.0 ** -32) * w[:, 3]
        z = torch.stack([r1 * torch.cos(a1), r1 * torch.sin(a1), r2 * torch.cos(a2), r2 * torch.sin(a2)], dim=-1)
        return z.reshape(-1)[:n].float().reshape(shape)

    def choice(self, n: int, k: int) -> np.ndarray:
        """k distinct integers of [0, n): the first k of a Fisher-Yates shuffle."""
        perm = np.arange(n)
        u = self.uniform(k).cpu().numpy()
        for i in range(k):
            j = i + int(u[i] * (n - i))
            perm[i], perm[j] = perm[j], perm[i]
        return perm[:k]


# configuration index of each workload (seed = 20261201 + index); the first
# five are the reference's benchmark configurations in their order
CONFIG_INDEX = {"llama-3.2-1b-b1": 0, "qwen3-14b-b32": 1, "llama-3-8b-shared-prefix-b64": 2,
                "llama-3-8b-verify-b16": 3, "qwen3-30b-a3b-b8-128k": 4, "qwen3-14b-prefill-b8-c512": 5,
                "qwen3-14b-b32-continuous": 6, "gemma3-12b-sliding-b32": 7, "gemma4-26b-full-b32": 8}
# streams of one run
S_LENGTHS, S_FILL, S_STEP, S_ACCEPT, S_OUTLIERS, S_CPU = range(6)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0  # dense fp16/bf16
METRIC = "int8-KV paged decode-attn GB/s (% HBM peak) + tokens/s, B=32 Qwen3-14B shape"

WORKLOADS = {
    "qwen3-14b-b32": dict(kind="decode", layers=40, Hq=40, Hkv=8, D=128, B=32, lo=512, hi=8192),
    "llama-3.2-1b-b1": dict(kind="decode", layers=16, Hq=32, Hkv=8, D=64, B=1, lo=2048, hi=2048),
    "qwen3-30b-a3b-b8-128k": dict(kind="decode", layers=48, Hq=32, Hkv=4, D=128, B=8, lo=131072, hi=131072,
                                  outlier_frac=0.01),
    # 64 sequences forked from one prefix of 4096 + 24 tokens (the last block shared while partly
    # filled, so each fork's first append copies it), unique suffixes U[0, 1024]
    "llama-3-8b-shared-prefix-b64": dict(kind="shared_prefix", layers=32, Hq=32, Hkv=8, D=128, B=64, lo=0,
                                         hi=1024, prefix=4096 + 24),
    "llama-3-8b-verify-b16": dict(kind="verify", layers=32, Hq=32, Hkv=8, D=128, B=16, lo=1024, hi=8192,
                                  draft=8),
    # chunked prefill: 512 new rows per sequence on top of its cache, every row kept
    "qwen3-14b-prefill-b8-c512": dict(kind="verify", layers=40, Hq=40, Hkv=8, D=128, B=8, lo=2048, hi=6144,
                                      draft=512, rollback=False),
    # the default decode workload with one request leaving and one joining (prompt U[512, 8192],
    # its K/V appended into a fresh sequence) at every step, no epoch restack
    "qwen3-14b-b32-continuous": dict(kind="continuous", layers=40, Hq=40, Hkv=8, D=128, B=32, lo=512, hi=8192,
                                     churn=1),
    # the sliding-window layers of a Gemma-3-12B-shaped model (window 1024), contexts as the headline
    "gemma3-12b-sliding-b32": dict(kind="window", layers=40, Hq=16, Hkv=8, D=256, B=32, lo=512, hi=8192,
                                   window=1024),
    # the full-attention layers of a Gemma-4-26B-A4B-shaped model (head_dim 512, 2 KV heads for 16
    # query heads, SDPA scale 1.0; six of them), contexts as the headline
    "gemma4-26b-full-b32": dict(kind="decode", layers=6, Hq=16, Hkv=2, D=512, B=32, lo=512, hi=8192,
                                scale=1.0),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--workload", default="qwen3-14b-b32", choices=sorted(WORKLOADS))
    ap.add_argument("--quant", default="affine_g64", choices=["affine_g64", "ref_row"])
    ap.add_argument("--split-blocks", type=int, default=0)
    ap.add_argument("--prefix-split", type=int, default=0,
                    help="shared-prefix workload: prefix blocks per workgroup of the prefix pass (0 = automatic)")
    ap.add_argument("--wave-stamps", action="store_true",
                    help="add the last decode launch's wave timeline (needs KRILL_LIBRARY=libkrillhip_stamps.so)")
    ap.add_argument("--rope-fill", action="store_true",
                    help="prefill K with RoPE fused into the append (krill_quantize_append_rope)")
    ap.add_argument("--window-rope", type=int, default=1,
                    help="sliding-window workload, fused step: 1 = RoPE of the queries and new K rows in the call, "
                         "0 = without")
    ap.add_argument("--unfused", action="store_true",
                    help="decode step as two calls per layer (quantize-append, then decode attention) instead of "
                         "the fused krill_decode_append_attention")
    ap.add_argument("--single-pass", action="store_true",
                    help="shared-prefix workload: one decode attention over the whole tables instead of the "
                         "prefix/suffix cascade")
    ap.add_argument("--kernel-reps", type=int, default=5, help="repetitions of the attention-only timing loop")
    ap.add_argument("--graph", type=int, default=1,
                    help="decode workloads: 1 = replay each step's table upload and per-layer calls from a HIP "
                         "graph (captured once per pinned table buffer); 0 = issue them from Python every step")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="1: time the CPU baseline sample on rank 0")
    ap.add_argument("--seed", type=int, default=None, help="default: 20261201 + the workload's configuration index")
    ap.add_argument("--copy-calibration", type=int, default=0,
                    help="MiB for a plain device copy (torch.neg of float32) run before the bench, so one "
                         "rocprofv3 --pmc run reads FETCH_SIZE/WRITE_SIZE of a kernel of known traffic too")
    args = ap.parse_args()
    if args.seed is None:
        args.seed = 20261201 + CONFIG_INDEX[args.workload]
    return args


def algorithmic_bytes_per_token_layer(Hkv, D, G):
    # int8 K and V payload + fp16 (scale, zero) for K and V per group
    return 2 * Hkv * D + 2 * Hkv * G * 4


class Env:
    """Pool, library handle, stream and RNG of one bench run."""

    def __init__(self, args, w, num_blocks, **pool_kw):
        import torch

        import krill_amd
        from krill_amd import _lib as KL

        self.torch, self.KL = torch, KL
        self.dev = torch.device("cuda:0")
        self.args, self.w = args, w
        self.G = w["D"] // 64 if args.quant == "affine_g64" else 1
        self.per_tok = algorithmic_bytes_per_token_layer(w["Hkv"], w["D"], self.G)
        self.pool = krill_amd.KVPool(w["layers"], w["Hkv"], w["D"], num_blocks, args.quant, "bf16",
                                     free_list_seed=args.seed, **pool_kw)
        if args.split_blocks:
            self.pool.set_option(KL.OPT_SPLIT_BLOCKS, args.split_blocks)
        if args.prefix_split:
            self.pool.set_option(KL.OPT_PREFIX_SPLIT, args.prefix_split)

        self.lib = KL.lib()
        self.h = self.pool.handle
        self.stream = torch.cuda.current_stream()
        self.sp = ctypes.c_void_p(self.stream.cuda_stream)
        self.rng_fill = Philox(args.seed, S_FILL, self.dev)
        self.rng_step = Philox(args.seed, S_STEP, self.dev)
        self.i32p = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))  # noqa: E731

    def randn_bf16(self, shape):
        t = self.torch
        return self.rng_step.normal(shape).to(t.bfloat16)

    def fill(self, seqs, counts, chunk=1024, outlier_frac=0.0, nrand=4):
        """Append counts[b] tokens to seqs[b] in every layer through the product path
        (reserve + strided quantize-append), cycling over nrand random chunks."""
        t, w = self.torch, self.w
        B, Hkv, D = len(seqs), w["Hkv"], w["D"]
        Tmax = int(max(counts)) if len(counts) else 0
        if Tmax == 0:
            return
        slots = np.full((B, Tmax), -1, np.int32)
        for b in range(B):
            if counts[b] > 0:
                slots[b, : counts[b]] = self.pool.reserve_append(seqs[b], int(counts[b]))
        slots_d = t.from_numpy(slots).to(self.dev)
        C = min(chunk, Tmax)
        scale = None
        if outlier_frac > 0:
            ch = Philox(self.args.seed, S_OUTLIERS).choice(Hkv * D, max(1, int(round(outlier_frac * Hkv * D))))
            s = np.ones(Hkv * D, np.float32)
            s[ch] = 20.0
            scale = t.from_numpy(s.reshape(1, Hkv, 1, D)).to(self.dev)
        pool_k, pool_v = [], []
        for _ in range(nrand):
            k = self.rng_fill.normal((B, Hkv, C, D))
            v = self.rng_fill.normal((B, Hkv, C, D))
            if scale is not None:
                k, v = k * scale, v * scale
            pool_k.append(k.to(t.bfloat16))
            pool_v.append(v.to(t.bfloat16))
        strides = (Hkv * C * D, C * D, D)
        rope = getattr(self.args, "rope_fill", False)
        if rope:
            from krill_amd.pool import rope_table

            cs = t.from_numpy(rope_table(Tmax, D, 1.0e6)).to(self.dev)  # Qwen3 rope_theta
            pos_d = t.arange(Tmax, dtype=t.int32, device=self.dev).expand(B, Tmax)
        n = 0
        for layer in range(w["layers"]):
            for t0 in range(0, Tmax, C):
                L = min(C, Tmax - t0)
                sm = slots_d[:, t0: t0 + L].contiguous()
                k, v = pool_k[n % nrand], pool_v[n % nrand]
                n += 1
                if rope:
                    ps = pos_d[:, t0: t0 + L].contiguous()
                    self.KL.check(self.lib.krill_quantize_append_rope(
                        self.h, layer, k.data_ptr(), v.data_ptr(), *strides, sm.data_ptr(), ps.data_ptr(),
                        cs.data_ptr(), Tmax, B, L, self.sp))
                else:
                    self.KL.check(self.lib.krill_quantize_append_strided(self.h, layer, k.data_ptr(), v.data_ptr(),
                                                                         *strides, sm.data_ptr(), B, L, self.sp))
        t.cuda.synchronize()


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one MI355X; --gpus {args.gpus} is not supported (the path would shard by "
              "sequence / KV head across GPUs)", file=sys.stderr)
        sys.exit(2)
    import torch

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device="cuda:0")
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)
        torch.cuda.synchronize()
        del x, y
    w = WORKLOADS[args.workload]
    rec = {"decode": run_decode, "verify": run_verify, "shared_prefix": run_shared_prefix,
           "continuous": run_continuous, "window": run_window}[w["kind"]](args, w)
    print(json.dumps(rec))


def _record(args, w, env, value, ms_step, config, roofline, extra, cpu=None):
    stats = env.pool.stats()
    rec = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "u8",
        "data": "synthetic",
        "config": config,
    }
    rec.update(extra)
    rec["host_ms_per_step"] = round(getattr(env, "host_loop_ms", 0.0), 4)
    rec["roofline"] = roofline
    rec["cpu_baseline"] = cpu
    rec["pool"] = {k: stats[k] for k in ("cow_copies", "blocks_used", "blocks_shared", "evicted_entries",
                                         "evicted_blocks", "num_blocks")}
    if args.wave_stamps:
        rec["wave_stamps"] = wave_stamp_summary(env)
    return rec


def wave_stamp_summary(env):
    """Timeline of the last decode-attention launch from a library built with
    `make stamps` (KRILL_LIBRARY=libkrillhip_stamps.so): per-wave start, first
    block ready, static part done and end (realtime clock, 100 MHz), with the
    XCD / CU / SIMD of each wave; and the launch's end time if the waves' work
    were balanced within each CU, within each XCD, or over the whole GPU (the
    mean end time of the group: total work kept, end times evened out)."""
    env.torch.cuda.synchronize()
    buf = np.zeros((65536, 6), np.uint64)
    n = env.lib.krill_diag_wave_stamps(buf.ctypes.data_as(ctypes.c_void_p), buf.shape[0])
    if n < 0:
        return {"error": env.KL.last_error()}
    a = buf[:n].astype(np.int64)
    a = a[a[:, 2] > 0]
    a = a[a[:, 0] >= a[:, 0].max() - 5000]  # the last launch: its waves start within 50 us
    t0 = a[:, 0].min()
    us = lambda t: (t - t0) / 100.0  # noqa: E731
    st, fr, en = us(a[:, 0]), us(a[:, 1]), us(a[:, 2])
    hw, xcc = a[:, 4] & 0xFFFFFFFF, (a[:, 4] >> 32) & 0xF
    simd, cu, sh, se = (hw >> 4) & 3, (hw >> 8) & 15, (hw >> 12) & 1, (hw >> 13) & 7
    cuid = xcc * 1000 + se * 100 + sh * 20 + cu
    cus = np.unique(cuid)
    cu_spread = np.array([np.ptp(en[cuid == c]) for c in cus])
    cu_mean = np.array([en[cuid == c].mean() for c in cus])
    xcds = np.unique(xcc)
    xcd_mean = np.array([en[xcc == x].mean() for x in xcds])
    grid = np.linspace(0.0, en.max(), 13)
    r2 = lambda x: round(float(x), 2)  # noqa: E731
    return {
        "waves": int(len(a)),
        "span_us": r2(en.max()),
        "start_spread_us": r2(np.ptp(st)),
        "first_ready_us": {"median": r2(np.median(fr - st)), "p90": r2(np.percentile(fr - st, 90))},
        "end_us": {"min": r2(en.min()), "p10": r2(np.percentile(en, 10)), "median": r2(np.median(en)),
                   "p90": r2(np.percentile(en, 90)), "max": r2(en.max())},
        "mean_wave_life_frac": r2((en - st).mean() / en.max()),
        "xcd_mean_end_us": [r2(x) for x in xcd_mean],
        "within_cu_end_spread_us_median": r2(np.median(cu_spread)),
        "balanced_end_us": {"within_cu": r2(cu_mean.max()), "within_xcd": r2(xcd_mean.max()),
                            "whole_gpu": r2(en.mean())},
        "alive_waves": [int(((st <= t) & (en > t)).sum()) for t in grid],
        "alive_at_us": [r2(t) for t in grid],
    }


def _timed(env, step, warmup, steps):
    t = env.torch
    for i in range(warmup):
        step(i)
    t.cuda.synchronize()
    # no collector pass inside the timed steps: a full pass over the interpreter's
    # objects stalls the host for tens of ms, which a native batcher never does
    gc.collect()
    gc.disable()
    try:
        return _timed_steps(env, step, warmup, steps)
    finally:
        gc.enable()


def _timed_steps(env, step, warmup, steps):
    t = env.torch
    t_start = t.cuda.Event(enable_timing=True)
    t_end = t.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t_start.record(env.stream)
    for i in range(steps):
        step(warmup + i)
    t_end.record(env.stream)
    env.host_loop_ms = (time.perf_counter() - wall0) * 1e3 / steps  # host side of a step (calls, table builds)
    t.cuda.synchronize()
    return t_start.elapsed_time(t_end) / steps, time.perf_counter() - wall0


def _time_calls(env, call, reps):
    """Average time of one call(layer) over reps passes of all layers (HIP events on the library's stream)."""
    t = env.torch
    layers = env.w["layers"]
    for layer in range(layers):
        call(layer)
    t.cuda.synchronize()
    e0 = t.cuda.Event(enable_timing=True)
    e1 = t.cuda.Event(enable_timing=True)
    e0.record(env.stream)
    for _ in range(reps):
        for layer in range(layers):
            call(layer)
    e1.record(env.stream)
    t.cuda.synchronize()
    return e0.elapsed_time(e1) / (reps * layers)


class StepTables:
    """Pinned host buffers (ring of 3) and device copies of the step's block tables, lengths and slots."""

    def __init__(self, env, B, max_blocks, slots_per_seq, prefix_blocks=0):
        t = env.torch
        self.env, self.B, self.mb, self.pb = env, B, max_blocks, prefix_blocks
        sw = max(max_blocks - prefix_blocks, 1)
        self.ring = [(t.empty((B, max(slots_per_seq, 1)), dtype=t.int32).pin_memory(),
                      t.empty((B, max_blocks), dtype=t.int32).pin_memory(),
                      t.empty((B,), dtype=t.int32).pin_memory(),
                      t.empty((B, sw), dtype=t.int32).pin_memory(),
                      t.empty((B,), dtype=t.int32).pin_memory()) for _ in range(3)]
        self.events = [None] * 3
        self.d_slots = t.empty((B, max(slots_per_seq, 1)), dtype=t.int32, device=env.dev)
        self.d_tables = t.empty((B, max_blocks), dtype=t.int32, device=env.dev)
        self.d_lens = t.empty((B,), dtype=t.int32, device=env.dev)
        # with a shared prefix of prefix_blocks blocks: each table from that column on, and the length after it
        self.suffix_width = sw
        self.d_suffix_tables = t.empty((B, sw), dtype=t.int32, device=env.dev)
        self.d_suffix_lens = t.empty((B,), dtype=t.int32, device=env.dev)

    def host(self, i):
        j = i % 3
        if self.events[j] is not None:
            self.events[j].synchronize()
        return j, self.ring[j][0].numpy(), self.ring[j][1].numpy(), self.ring[j][2].numpy()

    def upload(self, j, slots=True):
        ps, pt, pl, sfx_t, sfx_l = self.ring[j]
        if slots:
            self.d_slots.copy_(ps, non_blocking=True)
        if self.pb:
            sfx_t.numpy()[:] = pt.numpy()[:, self.pb:]
            sfx_l.numpy()[:] = pl.numpy() - 64 * self.pb
            self.d_suffix_tables.copy_(sfx_t, non_blocking=True)
            self.d_suffix_lens.copy_(sfx_l, non_blocking=True)
        else:
            self.d_tables.copy_(pt, non_blocking=True)
            self.d_lens.copy_(pl, non_blocking=True)
        self.mark(j)

    def mark(self, j):
        """Event after the work that reads ring buffer j (its next host() waits on it)."""
        ev = self.env.torch.cuda.Event()
        ev.record(self.env.stream)
        self.events[j] = ev


class StepGraphs:
    """A decode step replayed from HIP graphs: per pinned ring buffer j, the
    copy of its tables (and slots) to the device and every layer's calls,
    captured once on a side stream (default priority).  The calls are made
    with max_seq_len = the run's final longest sequence, an upper bound for
    every step (the kernels read the true lengths from the device), so one
    capture serves all steps."""

    def __init__(self, env, st, layers, step_layer, max_len_final, slots):
        t = env.torch
        self.graphs = []
        cap = t.cuda.Stream()
        scap = ctypes.c_void_p(cap.cuda_stream)
        t.cuda.synchronize()
        for j in range(3):
            ps, pt, pl = st.ring[j][0], st.ring[j][1], st.ring[j][2]
            g = t.cuda.CUDAGraph()
            with t.cuda.graph(g, stream=cap):
                if slots:
                    st.d_slots.copy_(ps, non_blocking=True)
                st.d_tables.copy_(pt, non_blocking=True)
                st.d_lens.copy_(pl, non_blocking=True)
                for layer in range(layers):
                    step_layer(layer, max_len_final, scap)
            self.graphs.append(g)
        t.cuda.synchronize()

    def replay(self, j):
        self.graphs[j].replay()


def _decode_calls(env, seqs, st, max_len_final, Hq):
    """The per-layer decode call(s) over the batch (fused unless --unfused)."""
    args, w, KL, lib, h, sp = env.args, env.w, env.KL, env.lib, env.h, env.sp
    B, Hkv, D, layers = len(seqs), w["Hkv"], w["D"], w["layers"]
    q_all = env.randn_bf16((layers, B, Hq, 1, D))
    k_new = env.randn_bf16((layers, B, Hkv, 1, D))
    v_new = env.randn_bf16((layers, B, Hkv, 1, D))
    out = env.torch.empty((B, Hq, 1, D), dtype=env.torch.bfloat16, device=env.dev)
    ws_bytes = env.pool.workspace_size(B, Hq, 1, max_len_final)
    ws = env.torch.empty(max(ws_bytes, 1), dtype=env.torch.uint8, device=env.dev)
    qp = [q_all[l].data_ptr() for l in range(layers)]
    kp = [k_new[l].data_ptr() for l in range(layers)]
    vp = [v_new[l].data_ptr() for l in range(layers)]
    scale = ctypes.c_float(w.get("scale", 1.0 / math.sqrt(D)))
    keep = (q_all, k_new, v_new, out, ws)

    def append(layer, s):
        KL.check(lib.krill_quantize_append(h, layer, kp[layer], vp[layer], st.d_slots.data_ptr(), B, 1, s))

    def attend(layer, mx, s=sp):
        KL.check(lib.krill_decode_attention(h, layer, qp[layer], st.d_tables.data_ptr(), st.d_lens.data_ptr(), B,
                                            st.mb, mx, Hq, scale, out.data_ptr(), KL.DTYPE_BF16, ws.data_ptr(),
                                            ws_bytes, s))

    def fused(layer, mx, s=sp):
        # the token at position len - 1 (its slot reserved by the step) is written, then attended over
        KL.check(lib.krill_decode_append_attention(h, layer, qp[layer], kp[layer], vp[layer], Hkv * D, D,
                                                   st.d_tables.data_ptr(), st.d_lens.data_ptr(), B, st.mb, mx, Hq,
                                                   scale, out.data_ptr(), KL.DTYPE_BF16, ws.data_ptr(), ws_bytes,
                                                   s))

    def step_layer(layer, mx, s=sp):
        if args.unfused:
            append(layer, s)
            attend(layer, mx, s)
        else:
            fused(layer, mx, s)

    def call_only(layer, mx):  # the dominant call alone; the fused one rewrites the same token
        if args.unfused:
            attend(layer, mx)
        else:
            fused(layer, mx)

    return step_layer, call_only, keep


def _cascade_calls(env, seqs, st, max_len_final, Hq, prefix_table):
    """Per layer the shared-prefix cascade (prefix pass over the P shared
    blocks for all B sequences, suffix pass, merge) with the new token's
    append fused into the suffix pass (--unfused: quantize-append, then the
    cascade)."""
    KL, lib, h, sp, w = env.KL, env.lib, env.h, env.sp, env.w
    B, Hkv, D, layers = len(seqs), w["Hkv"], w["D"], w["layers"]
    Pb = st.pb
    q_all = env.randn_bf16((layers, B, Hq, 1, D))
    k_new = env.randn_bf16((layers, B, Hkv, 1, D))
    v_new = env.randn_bf16((layers, B, Hkv, 1, D))
    out = env.torch.empty((B, Hq, 1, D), dtype=env.torch.bfloat16, device=env.dev)
    need = ctypes.c_size_t()
    KL.check(lib.krill_shared_prefix_workspace_size(h, B, Hq, Pb, max_len_final - 64 * Pb, ctypes.byref(need)))
    ws = env.torch.empty(max(need.value, 1), dtype=env.torch.uint8, device=env.dev)
    qp = [q_all[l].data_ptr() for l in range(layers)]
    kp = [k_new[l].data_ptr() for l in range(layers)]
    vp = [v_new[l].data_ptr() for l in range(layers)]
    scale = ctypes.c_float(1.0 / math.sqrt(D))
    keep = (q_all, k_new, v_new, out, ws, prefix_table)

    def attend(layer, mx):
        KL.check(lib.krill_decode_attention_shared_prefix(
            h, layer, qp[layer], prefix_table.data_ptr(), Pb, st.d_suffix_tables.data_ptr(),
            st.d_suffix_lens.data_ptr(), B, st.suffix_width, mx - 64 * Pb, Hq, scale, out.data_ptr(),
            KL.DTYPE_BF16, ws.data_ptr(), need.value, sp))

    def fused(layer, mx):
        KL.check(lib.krill_decode_append_attention_shared_prefix(
            h, layer, qp[layer], kp[layer], vp[layer], Hkv * D, D, prefix_table.data_ptr(), Pb,
            st.d_suffix_tables.data_ptr(), st.d_suffix_lens.data_ptr(), B, st.suffix_width, mx - 64 * Pb, Hq, scale,
            out.data_ptr(), KL.DTYPE_BF16, ws.data_ptr(), need.value, sp))

    def step_layer(layer, mx):
        if env.args.unfused:
            KL.check(lib.krill_quantize_append(h, layer, kp[layer], vp[layer], st.d_slots.data_ptr(), B, 1, sp))
            attend(layer, mx)
        else:
            fused(layer, mx)

    return step_layer, (attend if env.args.unfused else fused), keep


def run_decode(args, w):
    layers, Hq, Hkv, D, B = w["layers"], w["Hq"], w["Hkv"], w["D"], w["B"]
    rng = Philox(args.seed, S_LENGTHS)
    lens0 = rng.integers(w["lo"], w["hi"] + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1 + (3 if args.graph else 0)
    blocks_needed = int(sum((int(T) + total_steps + 63) // 64 for T in lens0))
    num_blocks = blocks_needed + max(16, blocks_needed // 8)
    max_len_final = int(lens0.max()) + total_steps
    max_blocks = (max_len_final + 63) // 64
    env = Env(args, w, num_blocks)
    seqs = [env.pool.seq_create() for _ in range(B)]
    env.fill(seqs, [int(x) for x in lens0], outlier_frac=w.get("outlier_frac", 0.0))

    st = StepTables(env, B, max_blocks, 1)
    step_layer, call_only, keep = _decode_calls(env, seqs, st, max_len_final, Hq)
    seqs_np = np.array(seqs, np.int32)
    one = np.empty(1, np.int32)
    cur_len = [int(x) for x in lens0]
    graphs = None

    def step(i):
        j, ps, pt, pl = st.host(i)
        for b in range(B):
            env.KL.check(env.lib.krill_seq_reserve_append(env.h, seqs[b], 1, env.i32p(one)))
            ps[b, 0] = one[0]
            cur_len[b] += 1
        env.KL.check(env.lib.krill_batch_tables(env.h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
        if graphs is not None:
            graphs.replay(j)
            st.mark(j)
            return
        st.upload(j, slots=args.unfused)
        mx = max(cur_len)
        for layer in range(layers):
            step_layer(layer, mx)

    for i in range(args.warmup):
        step(i)
    if args.graph:
        graphs = StepGraphs(env, st, layers, step_layer, max_len_final, args.unfused)
        for i in range(3):  # one replay of each graph before the timed steps
            step(args.warmup + i)
    lens_start = None
    # timed steps (lengths at their start recorded for the byte count)
    env.torch.cuda.synchronize()
    lens_start = list(cur_len)
    ms_step, wall = _timed(env, lambda i: step(args.warmup + i), 0, args.steps)

    per_tok = env.per_tok
    avg_ctx = [(lens_start[b] + cur_len[b] + 1) / 2.0 for b in range(B)]
    kv_bytes_layer = sum(avg_ctx) * per_tok
    qo_bytes_layer = B * Hq * D * 2 * 2
    step_bytes = layers * (kv_bytes_layer + qo_bytes_layer)
    gbs_step = step_bytes / (ms_step * 1e-3) / 1e9

    mx = max(cur_len)
    attn_ms = _time_calls(env, lambda layer: call_only(layer, mx), args.kernel_reps)
    launch_bytes = sum(cur_len) * per_tok + qo_bytes_layer
    if not args.unfused:  # the new token: bf16 K/V rows in, quantized bytes out
        launch_bytes += B * (2 * Hkv * D * 2 + per_tok)
    achieved = launch_bytes / (attn_ms * 1e-3) / 1e9

    cpu = None
    if args.cpu_baseline and w["kind"] == "decode" and max(lens0) <= 16384:
        cpu = cpu_baseline(args, w, lens0, per_tok)

    config = {
        "workload": f"{args.workload}: {layers} layers, Hq {Hq}, Hkv {Hkv}, D {D}, B {B}, "
                    f"context U[{w['lo']},{w['hi']}], 64-token blocks (permuted pool), {args.quant} int8, "
                    "bf16 N(0,1) inputs"
                    + (f" ({w['outlier_frac']:.0%} of channels x20)" if w.get("outlier_frac") else "")
                    + (f", softmax scale {w['scale']}" if "scale" in w else "")
                    + "; step = per layer quantize-append 1 token/seq + paged decode attention"
                    + (" (two calls)" if args.unfused else " (one fused call)")
                    + ("; each step's table upload and calls replayed from a HIP graph" if args.graph else ""),
        "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "quant": args.quant,
        "context_mean": float(np.mean(lens0)), "num_blocks": num_blocks,
    }
    call = "decode_attn" if args.unfused else "decode_append_attn"
    roofline = {
        "bound": "hbm",
        "kernel": ("paged decode attention call (k_attn_valu + k_attn_merge_flat), one layer" if args.unfused
                   else "fused append + paged decode attention call (k_attn_valu + k_attn_merge_flat), one layer"),
        "achieved": round(achieved, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(achieved / HBM_PEAK_GBS, 4),
        "traffic": measured_traffic(args, call),
        "traffic_source": traffic_source(args, call),
        "bytes_per_launch": int(launch_bytes),
        "avg_launch_ms": round(attn_ms, 5),
    }
    extra = {"tokens_per_s": round(B / (ms_step * 1e-3), 1), "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4),
             "step_bytes": int(step_bytes), "wall_s_timed": round(wall, 4)}
    rec = _record(args, w, env, gbs_step, ms_step, config, roofline, extra, cpu)
    del keep
    env.pool.close()
    return rec


def run_continuous(args, w):
    """Continuous batching without epochs: at every step `churn` rows leave
    (their blocks freed) and as many requests join, each with its prompt's
    K/V (prefilled by the caller's model) appended into a fresh sequence; then
    one fused decode step of all B rows.  The running rows are never copied.
    The reference batcher instead restacks every row's cache left-padded when
    the active set changes and scatters it back after the epoch; both copies
    are timed on the same pool after the steps for comparison."""
    t = None
    layers, Hq, Hkv, D, B, churn = w["layers"], w["Hq"], w["Hkv"], w["D"], w["B"], w["churn"]
    rng = Philox(args.seed, S_LENGTHS)
    lens0 = rng.integers(w["lo"], w["hi"] + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1
    new_lens = rng.integers(w["lo"], w["hi"] + 1, size=total_steps * churn).astype(np.int64)
    leave = rng.integers(0, B, size=total_steps * churn)
    max_len_final = w["hi"] + total_steps
    max_blocks = (max_len_final + 63) // 64
    num_blocks = B * (max_blocks + 1) + 64
    env = Env(args, w, num_blocks)
    t = env.torch
    seqs = [env.pool.seq_create() for _ in range(B)]
    env.fill(seqs, [int(x) for x in lens0])
    st = StepTables(env, B, max_blocks, 1)
    step_layer, call_only, keep = _decode_calls(env, seqs, st, max_len_final, Hq)
    # prompt K/V of the joining requests (the same random rows for every one; the bytes are what count)
    Tp = w["hi"]
    kp = env.randn_bf16((1, Hkv, Tp, D))
    vp = env.randn_bf16((1, Hkv, Tp, D))
    strides = (Hkv * Tp * D, Tp * D, D)
    ring = [t.empty((churn, Tp), dtype=t.int32).pin_memory() for _ in range(3)]
    d_new = t.empty((churn, Tp), dtype=t.int32, device=env.dev)
    cur_len = [int(x) for x in lens0]
    one = np.empty(1, np.int32)
    joined_tokens = [0]

    def step(i):
        j, ps, pt, pl = st.host(i)
        ns = ring[j].numpy()
        news = []
        for c in range(churn):
            r = int(leave[i * churn + c])
            env.KL.check(env.lib.krill_seq_free(env.h, seqs[r]))
            sid = ctypes.c_int32()
            env.KL.check(env.lib.krill_seq_create(env.h, ctypes.byref(sid)))
            T = int(new_lens[i * churn + c])
            env.KL.check(env.lib.krill_seq_reserve_append(env.h, sid.value, T, env.i32p(ns[c])))
            seqs[r] = sid.value
            cur_len[r] = T
            news.append(T)
            joined_tokens[0] += T
        d_new.copy_(ring[j], non_blocking=True)
        for b in range(B):
            env.KL.check(env.lib.krill_seq_reserve_append(env.h, seqs[b], 1, env.i32p(one)))
            ps[b, 0] = one[0]
            cur_len[b] += 1
        seqs_np = np.array(seqs, np.int32)
        env.KL.check(env.lib.krill_batch_tables(env.h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
        st.upload(j, slots=args.unfused)
        mx = max(cur_len)
        for layer in range(layers):
            for c, T in enumerate(news):  # the joining requests' prompts, then the batch's decode
                env.KL.check(env.lib.krill_quantize_append_strided(
                    env.h, layer, kp.data_ptr(), vp.data_ptr(), *strides, d_new[c].data_ptr(), 1, T, env.sp))
            step_layer(layer, mx)

    for i in range(args.warmup):
        step(i)
    t.cuda.synchronize()
    lens_start = list(cur_len)
    j0 = joined_tokens[0]
    ms_step, wall = _timed(env, lambda i: step(args.warmup + i), 0, args.steps)
    per_tok = env.per_tok
    joined = (joined_tokens[0] - j0) / args.steps  # prompt tokens appended per step
    # decode bytes: each row's cache at the step (rows replaced mid-run counted at their new length)
    avg_ctx = sum((a + b_) / 2.0 for a, b_ in zip(lens_start, cur_len))
    qo_layer = B * Hq * D * 2 * 2
    step_bytes = layers * (avg_ctx * per_tok + qo_layer + joined * (2 * Hkv * D * 2 + per_tok)
                           + B * (2 * Hkv * D * 2 + per_tok))
    gbs_step = step_bytes / (ms_step * 1e-3) / 1e9
    mx = max(cur_len)
    attn_ms = _time_calls(env, lambda layer: call_only(layer, mx), args.kernel_reps)
    launch_bytes = sum(cur_len) * per_tok + qo_layer + B * (2 * Hkv * D * 2 + per_tok)

    # the reference's epoch copies on this batch: stack every row left-padded, scatter it back
    tabs, lns = env.pool.batch_tables(seqs, max_blocks)
    S = int(lns.max())
    d_tabs = t.from_numpy(np.ascontiguousarray(tabs)).to(env.dev)
    d_lns = t.from_numpy(np.ascontiguousarray(lns)).to(env.dev)
    tok = np.arange(S)
    slot_map = np.where(tok[None, :] < lns[:, None],
                        np.take_along_axis(tabs, np.minimum(tok[None, :] // 64, max_blocks - 1).repeat(B, 0), 1) * 64
                        + tok[None, :] % 64, -1).astype(np.int32)
    d_slots = t.from_numpy(slot_map).to(env.dev)
    d_start = t.from_numpy((S - lns).astype(np.int32)).to(env.dev)
    snap = env.pool.gather(0, d_tabs, d_lns, S, left_pad=True, stream=env.stream)
    t.cuda.synchronize()
    e = [t.cuda.Event(enable_timing=True) for _ in range(3)]
    reps = 3
    e[0].record(env.stream)
    for _ in range(reps):
        env.pool.gather(0, d_tabs, d_lns, S, left_pad=True, stream=env.stream)
    e[1].record(env.stream)
    for _ in range(reps):
        env.pool.scatter(0, snap, d_start, d_slots, stream=env.stream)
    e[2].record(env.stream)
    t.cuda.synchronize()
    gather_ms, scatter_ms = e[0].elapsed_time(e[1]) / reps, e[1].elapsed_time(e[2]) / reps
    stack_bytes = 2 * int(lns.sum()) * per_tok  # read + write of every row's cache

    config = {
        "workload": f"{args.workload}: {layers} layers, Hq {Hq}, Hkv {Hkv}, D {D}, B {B}, context "
                    f"U[{w['lo']},{w['hi']}], {churn} request(s) leaving and joining per step (prompt "
                    f"U[{w['lo']},{w['hi']}] tokens of K/V appended into a fresh sequence), {args.quant} int8; "
                    "step = the joining prompts' appends + per layer one fused append + decode attention call "
                    "over all rows (no restack)",
        "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "quant": args.quant, "churn": churn,
        "num_blocks": num_blocks,
    }
    roofline = {
        "bound": "hbm",
        "kernel": "fused append + paged decode attention call (k_attn_valu + k_attn_merge_flat), one layer",
        "achieved": round(launch_bytes / (attn_ms * 1e-3) / 1e9, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(launch_bytes / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": None,
        "bytes_per_launch": int(launch_bytes),
        "avg_launch_ms": round(attn_ms, 5),
    }
    extra = {"tokens_per_s": round(B / (ms_step * 1e-3), 1), "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4),
             "prompt_tokens_joined_per_step": joined, "wall_s_timed": round(wall, 4),
             "epoch_restack": {"gather_left_padded_ms_per_layer": round(gather_ms, 4),
                               "scatter_back_ms_per_layer": round(scatter_ms, 4),
                               "ms_per_change_all_layers": round((gather_ms + scatter_ms) * layers, 3),
                               "gbs": round(stack_bytes / ((gather_ms + scatter_ms) * 1e-3) / 1e9, 1),
                               "rows_tokens": int(lns.sum())}}
    rec = _record(args, w, env, gbs_step, ms_step, config, roofline, extra)
    del keep, snap
    env.pool.close()
    return rec


def run_window(args, w):
    """Decode steps of sliding-window layers: a pool with the window option
    (each append first drops the blocks below the sequence's last window - 1
    tokens), per layer one launch that turns the queries and the new K row by
    the token's position (RoPE), appends the token and attends the retained
    window (--unfused: quantize-append, then windowed attention, no RoPE)."""
    layers, Hq, Hkv, D, B, W = w["layers"], w["Hq"], w["Hkv"], w["D"], w["B"], w["window"]
    t = None
    rng = Philox(args.seed, S_LENGTHS)
    lens0 = rng.integers(w["lo"], w["hi"] + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1
    max_len_final = int(lens0.max()) + total_steps
    max_blocks = (max_len_final + 63) // 64
    num_blocks = int(sum((int(x) + 63) // 64 for x in lens0)) + B * 4 + 16
    env = Env(args, w, num_blocks)
    t = env.torch
    env.pool.set_option(env.KL.OPT_WINDOW, W)
    seqs = [env.pool.seq_create() for _ in range(B)]
    env.fill(seqs, [int(x) for x in lens0])
    st = StepTables(env, B, max_blocks, 1)
    starts_ring = [t.empty((B,), dtype=t.int32).pin_memory() for _ in range(3)]
    d_starts = t.empty((B,), dtype=t.int32, device=env.dev)
    q_all = env.randn_bf16((layers, B, Hq, 1, D))
    k_new = env.randn_bf16((layers, B, Hkv, 1, D))
    v_new = env.randn_bf16((layers, B, Hkv, 1, D))
    out = t.empty((B, Hq, 1, D), dtype=t.bfloat16, device=env.dev)
    need = ctypes.c_size_t()
    env.KL.check(env.lib.krill_window_workspace_size(env.h, B, Hq, 1, max_blocks, max_len_final, W,
                                                     ctypes.byref(need)))
    ws = t.empty(max(need.value, 1), dtype=t.uint8, device=env.dev)
    scale = ctypes.c_float(1.0 / math.sqrt(D))
    seqs_np = np.array(seqs, np.int32)
    one = np.empty(1, np.int32)
    cur_len = [int(x) for x in lens0]
    KL, lib, h, sp = env.KL, env.lib, env.h, env.sp
    from krill_amd.pool import rope_table

    cs = t.from_numpy(rope_table(max_len_final + 1, D, 1.0e4)).to(env.dev)

    def attend(layer, mx):
        KL.check(lib.krill_attention_windowed(h, layer, q_all[layer].data_ptr(), 1, st.d_tables.data_ptr(),
                                              st.d_lens.data_ptr(), d_starts.data_ptr(), W, B, max_blocks, mx, Hq,
                                              scale, out.data_ptr(), KL.DTYPE_BF16, ws.data_ptr(), need.value, sp))

    def fused(layer, mx):  # RoPE + append + windowed attention, one launch
        KL.check(lib.krill_decode_append_attention_windowed(
            h, layer, q_all[layer].data_ptr(), k_new[layer].data_ptr(), v_new[layer].data_ptr(), Hkv * D, D,
            st.d_tables.data_ptr(), st.d_lens.data_ptr(), d_starts.data_ptr(), W, B, max_blocks, mx, Hq, scale,
            cs.data_ptr() if args.window_rope else None, cs.shape[0], out.data_ptr(), KL.DTYPE_BF16, ws.data_ptr(),
            need.value, sp))

    def step(i):
        j, ps, pt, pl = st.host(i)
        for b in range(B):
            KL.check(lib.krill_seq_reserve_append(h, seqs[b], 1, env.i32p(one)))
            ps[b, 0] = one[0]
            cur_len[b] += 1
        KL.check(lib.krill_batch_tables(h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
        KL.check(lib.krill_batch_starts(h, env.i32p(seqs_np), B, env.i32p(starts_ring[j].numpy())))
        d_starts.copy_(starts_ring[j], non_blocking=True)
        st.upload(j, slots=True)
        mx = max(cur_len)
        for layer in range(layers):
            if args.unfused:
                KL.check(lib.krill_quantize_append(h, layer, k_new[layer].data_ptr(), v_new[layer].data_ptr(),
                                                   st.d_slots.data_ptr(), B, 1, sp))
                attend(layer, mx)
            else:
                fused(layer, mx)

    for i in range(args.warmup):
        step(i)
    t.cuda.synchronize()
    ms_step, wall = _timed(env, lambda i: step(args.warmup + i), 0, args.steps)
    per_tok = env.per_tok
    vis = sum(min(n, W) for n in cur_len)  # keys each decode row sees
    qo_layer = B * Hq * D * 2 * 2
    app_layer = B * (2 * Hkv * D * 2 + per_tok)
    step_bytes = layers * (vis * per_tok + qo_layer + app_layer)
    gbs_step = step_bytes / (ms_step * 1e-3) / 1e9
    mx = max(cur_len)
    call = attend if args.unfused else fused  # the fused call rewrites the same newest token
    attn_ms = _time_calls(env, lambda layer: call(layer, mx), args.kernel_reps)
    launch_bytes = vis * per_tok + qo_layer + (0 if args.unfused else app_layer)
    stats = env.pool.stats()
    config = {
        "workload": f"{args.workload}: {layers} sliding-window layers, window {W}, Hq {Hq}, Hkv {Hkv}, D {D}, B {B}, "
                    f"context U[{w['lo']},{w['hi']}], {args.quant} int8, pool with the window option (blocks below "
                    "each window freed); step = per layer "
                    + ("quantize-append 1 token/seq + windowed decode attention (two calls)" if args.unfused else
                       ("RoPE of the queries and new K rows + " if args.window_rope else "")
                       + "append 1 token/seq + windowed decode attention (one fused call)"),
        "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "quant": args.quant, "window": W,
        "context_mean": float(np.mean(lens0)), "num_blocks": num_blocks,
    }
    roofline = {
        "bound": "hbm",
        "kernel": ("windowed decode attention call" if args.unfused else
                   "fused " + ("RoPE + " if args.window_rope else "") + "append + windowed decode attention call")
                  + (" (k_attn_valu window variant, one workgroup per (sequence, KV head), partials merged in"
                     " LDS)" if D <= 256 else " (k_attn_valu window variant + k_attn_merge_flat)")
                  + ", one layer; bytes of the keys the rows see"
                  + ("" if args.unfused else ", q/o and the new token"),
        "achieved": round(launch_bytes / (attn_ms * 1e-3) / 1e9, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(launch_bytes / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": None,
        "bytes_per_launch": int(launch_bytes),
        "avg_launch_ms": round(attn_ms, 5),
    }
    extra = {"tokens_per_s": round(B / (ms_step * 1e-3), 1), "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4),
             "blocks_held_after": stats["blocks_used"],
             "blocks_full_history": int(sum((n + 63) // 64 for n in cur_len)), "wall_s_timed": round(wall, 4)}
    rec = _record(args, w, env, gbs_step, ms_step, config, roofline, extra)
    del q_all, k_new, v_new, out, ws
    env.pool.close()
    return rec


def run_shared_prefix(args, w):
    """Decode steps of B sequences forked from one refcounted prefix.  The pool
    is sized so that occupancy sits just under the 90 % watermark when the
    timed steps start, with unreferenced prefix entries (stale cached
    prompts) holding the slack: new blocks then evict them oldest first."""
    layers, Hq, Hkv, D, B = w["layers"], w["Hq"], w["Hkv"], w["D"], w["B"]
    rng = Philox(args.seed, S_LENGTHS)
    P = w["prefix"]
    suffix = rng.integers(w["lo"], w["hi"] + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1
    pblocks = (P + 63) // 64
    # blocks the live sequences end with: shared prefix blocks + each fork's own blocks (incl. its COW copy)
    own = [((P + int(s) + total_steps + 63) // 64) - (P // 64) for s in suffix]
    live_end = pblocks + sum(own)
    live_start = pblocks + sum(((P + int(s) + 63) // 64) - (P // 64) if s > 0 else 0 for s in suffix)
    stale_entries, stale_tokens = 8, 1024
    stale_blocks = stale_entries * (stale_tokens // 64)
    # num_blocks: (live_start + stale) just under 90 %; growth beyond it evicts stale entries
    num_blocks = int(math.ceil((live_start + stale_blocks) / 0.895)) + 1
    num_blocks = max(num_blocks, int(math.ceil(live_end / 0.9)) + 8)
    env = Env(args, w, num_blocks, evict_watermark=0.9, max_prefix_entries=stale_entries + 4)
    pool = env.pool
    # stale cached prompts, unreferenced once their sequences are freed
    for e in range(stale_entries):
        s = pool.seq_create()
        env.fill([s], [stale_tokens], chunk=stale_tokens, nrand=1)
        assert pool.prefix_store(s, np.arange(stale_tokens) + 1000003 * (e + 1))
        pool.seq_free(s)
    # the shared prefix, stored as an entry too (the prompt cache of the reference)
    base = pool.seq_create()
    env.fill([base], [P], chunk=1024, nrand=2)
    assert pool.prefix_store(base, np.arange(P))
    seqs = [pool.seq_fork(base, P) for _ in range(B)]
    pool.seq_free(base)
    env.fill(seqs, [int(s) for s in suffix], chunk=256, nrand=2)  # first appends copy the shared partial block
    lens0 = P + suffix
    max_len_final = int(lens0.max()) + total_steps
    max_blocks = (max_len_final + 63) // 64
    cascade = not args.single_pass
    Pb = P // 64
    st = StepTables(env, B, max_blocks, 1, prefix_blocks=Pb if cascade else 0)
    if cascade:
        # the P full prefix blocks: the same first Pb table entries in every fork
        t0, _ = pool.batch_tables(seqs, max_blocks)
        assert (t0[:, :Pb] == t0[0, :Pb]).all()
        prefix_table = env.torch.as_tensor(np.ascontiguousarray(t0[0, :Pb]), device=env.dev)
        step_layer, call_only, keep = _cascade_calls(env, seqs, st, max_len_final, Hq, prefix_table)
    else:
        step_layer, call_only, keep = _decode_calls(env, seqs, st, max_len_final, Hq)
    seqs_np = np.array(seqs, np.int32)
    one = np.empty(1, np.int32)
    cur_len = [int(x) for x in lens0]
    stats0 = pool.stats()

    def step(i):
        j, ps, pt, pl = st.host(i)
        for b in range(B):
            env.KL.check(env.lib.krill_seq_reserve_append(env.h, seqs[b], 1, env.i32p(one)))
            ps[b, 0] = one[0]
            cur_len[b] += 1
        env.KL.check(env.lib.krill_batch_tables(env.h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
        st.upload(j, slots=args.unfused)
        mx = max(cur_len)
        for layer in range(layers):
            step_layer(layer, mx)

    for i in range(args.warmup):
        step(i)
    env.torch.cuda.synchronize()
    lens_start = list(cur_len)
    ms_step, wall = _timed(env, lambda i: step(args.warmup + i), 0, args.steps)
    per_tok = env.per_tok
    avg_ctx = [(lens_start[b] + cur_len[b] + 1) / 2.0 for b in range(B)]
    logical_layer = sum(avg_ctx) * per_tok
    unique_layer = (P + sum(c - P for c in avg_ctx)) * per_tok
    qo_layer = B * Hq * D * 2 * 2
    unique_gbs = layers * (unique_layer + qo_layer) / (ms_step * 1e-3) / 1e9
    logical_gbs = layers * (logical_layer + qo_layer) / (ms_step * 1e-3) / 1e9
    mx = max(cur_len)
    attn_ms = _time_calls(env, lambda layer: call_only(layer, mx), args.kernel_reps)
    uniq_launch = (P + sum(c - P for c in cur_len)) * per_tok + qo_layer
    stats1 = pool.stats()
    config = {
        "workload": f"{args.workload}: {layers} layers, Hq {Hq}, Hkv {Hkv}, D {D}, {B} sequences forked from one "
                    f"{P}-token prefix (refcounted; last block shared while partly filled -> copy-on-write), "
                    f"unique suffixes U[{w['lo']},{w['hi']}], {args.quant} int8, pool at the 90 % LRU watermark "
                    f"with {stale_entries} unreferenced {stale_tokens}-token prefix entries; step = per layer "
                    "quantize-append 1 token/seq + paged decode attention"
                    + (f" as a cascade (the {Pb} full prefix blocks attended once for all {B} sequences, each "
                       "suffix on its own, partials merged)" if cascade else "")
                    + (" (two calls)" if args.unfused else " (one fused call)"),
        "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "quant": args.quant,
        "prefix": P, "cascade": cascade, "suffix_mean": float(np.mean(suffix)), "num_blocks": num_blocks,
    }
    if cascade:
        call_name = "shared-prefix cascade call (prefix pass + suffix pass + merge" + (
            ")" if args.unfused else ", append fused)")
    else:
        call_name = "paged decode attention call" if args.unfused else "fused append + paged decode attention call"
    roofline = {
        "bound": "hbm",
        "kernel": call_name + ", one layer; unique bytes (shared prefix once)",
        "achieved": round(uniq_launch / (attn_ms * 1e-3) / 1e9, 2),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(uniq_launch / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "traffic": None,
        "bytes_per_launch": int(uniq_launch),
        "avg_launch_ms": round(attn_ms, 5),
    }
    extra = {"tokens_per_s": round(B / (ms_step * 1e-3), 1), "hbm_frac_step": round(unique_gbs / HBM_PEAK_GBS, 4),
             "effective_gbs_logical": round(logical_gbs, 2), "wall_s_timed": round(wall, 4),
             "evictions_during_steps": {"entries": stats1["evicted_entries"] - stats0["evicted_entries"],
                                        "blocks": stats1["evicted_blocks"] - stats0["evicted_blocks"]},
             "occupancy_before_steps": round(stats0["blocks_used"] / num_blocks, 4)}
    rec = _record(args, w, env, unique_gbs, ms_step, config, roofline, extra)
    del keep
    pool.close()
    return rec


def run_verify(args, w):
    """Speculative verify: k draft tokens appended per sequence, causal verify
    attention of the k rows (MFMA path), then rollback to the accepted length
    (a ~ U[0, k] accepted: keep a + 1 rows on rejection, all k on full accept)."""
    layers, Hq, Hkv, D, B, k = w["layers"], w["Hq"], w["Hkv"], w["D"], w["B"], w["draft"]
    rollback = w.get("rollback", True)
    rng = Philox(args.seed, S_LENGTHS)
    lens0 = rng.integers(w["lo"], w["hi"] + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1
    blocks_needed = int(sum((int(T) + k * total_steps + 63) // 64 for T in lens0))
    num_blocks = blocks_needed + max(16, blocks_needed // 8)
    max_len_final = int(lens0.max()) + k * total_steps
    max_blocks = (max_len_final + 63) // 64
    env = Env(args, w, num_blocks)
    KL, lib, h, sp, t = env.KL, env.lib, env.h, env.sp, env.torch
    seqs = [env.pool.seq_create() for _ in range(B)]
    env.fill(seqs, [int(x) for x in lens0])
    st = StepTables(env, B, max_blocks, k)
    q_all = env.randn_bf16((layers, B, Hq, k, D))
    k_new = env.randn_bf16((layers, B, Hkv, k, D))
    v_new = env.randn_bf16((layers, B, Hkv, k, D))
    out = t.empty((B, Hq, k, D), dtype=t.bfloat16, device=env.dev)
    ws_bytes = env.pool.workspace_size(B, Hq, k, max_len_final)
    ws = t.empty(max(ws_bytes, 1), dtype=t.uint8, device=env.dev)
    scale = ctypes.c_float(1.0 / math.sqrt(D))
    seqs_np = np.array(seqs, np.int32)
    slots_h = np.empty(k, np.int32)
    cur_len = [int(x) for x in lens0]
    # accepted drafts per (step, sequence), drawn before the steps (no
    # generator work inside the timed loop)
    acc_draws = Philox(args.seed, S_ACCEPT).integers(0, k + 1, size=(args.warmup + args.steps + 1) * B)
    acc_pos = [0]
    accepted_total = [0]

    def verify(layer, mx):
        KL.check(lib.krill_verify_attention(h, layer, q_all[layer].data_ptr(), k, st.d_tables.data_ptr(),
                                            st.d_lens.data_ptr(), B, max_blocks, mx, Hq, scale, out.data_ptr(),
                                            KL.DTYPE_BF16, ws.data_ptr(), ws_bytes, sp))

    def step(i):
        j, ps, pt, pl = st.host(i)
        for b in range(B):
            KL.check(lib.krill_seq_reserve_append(h, seqs[b], k, env.i32p(slots_h)))
            ps[b, :] = slots_h
            cur_len[b] += k
        KL.check(lib.krill_batch_tables(h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
        st.upload(j)
        mx = max(cur_len)
        for layer in range(layers):
            KL.check(lib.krill_quantize_append(h, layer, k_new[layer].data_ptr(), v_new[layer].data_ptr(),
                                               st.d_slots.data_ptr(), B, k, sp))
            verify(layer, mx)
        # rollback (SpeculativeDecoder.swift:309-318): keep a + 1 rows on rejection, k on full accept
        for b in range(B):
            if not rollback:  # chunked prefill keeps every row
                accepted_total[0] += k
                continue
            a = int(acc_draws[acc_pos[0]])
            acc_pos[0] += 1
            keep_rows = a + 1 if a < k else k
            cur_len[b] += keep_rows - k
            accepted_total[0] += keep_rows
            KL.check(lib.krill_seq_truncate(h, seqs[b], cur_len[b]))

    for i in range(args.warmup):
        step(i)
    t.cuda.synchronize()
    lens_start = list(cur_len)
    acc0 = accepted_total[0]
    ms_step, wall = _timed(env, lambda i: step(args.warmup + i), 0, args.steps)
    per_tok = env.per_tok
    # per step: each sequence reads (len + k) tokens per layer
    avg_ctx = [(lens_start[b] + cur_len[b]) / 2.0 + k for b in range(B)]
    qo_layer = B * Hq * k * D * 2 * 2
    step_bytes = layers * (sum(avg_ctx) * per_tok + qo_layer)
    gbs_step = step_bytes / (ms_step * 1e-3) / 1e9

    # the verify call alone at the current lengths (the drafts of the last step are still cached)
    for b in range(B):
        KL.check(lib.krill_seq_reserve_append(h, seqs[b], k, env.i32p(slots_h)))
        cur_len[b] += k
    j, ps, pt, pl = st.host(10 ** 6)
    KL.check(lib.krill_batch_tables(h, env.i32p(seqs_np), B, max_blocks, env.i32p(pt), env.i32p(pl)))
    st.upload(j, slots=False)
    mx = max(cur_len)
    attn_ms = _time_calls(env, lambda layer: verify(layer, mx), args.kernel_reps)
    kv_launch = sum(cur_len) * per_tok + qo_layer
    # causal: row r of sequence b sees len_b - k + r + 1 tokens; QK^T and PV 2 FLOP per MAC each
    flops = sum(4.0 * Hq * D * sum(c - k + r + 1 for r in range(k)) for c in cur_len)
    tflops = flops / (attn_ms * 1e-3) / 1e12
    what = (f"{k} draft rows/seq (causal inside the window, {Hq // Hkv * k} query rows per KV head -> MFMA "
            f"path), accepted a ~ U[0,{k}] then rollback" if rollback else
            f"a {k}-token prefill chunk per sequence (causal inside the chunk, {Hq // Hkv * k} query rows per KV "
            "head in row groups of 32 -> MFMA path), every row kept")
    config = {
        "workload": f"{args.workload}: {layers} layers, Hq {Hq}, Hkv {Hkv}, D {D}, B {B}, context "
                    f"U[{w['lo']},{w['hi']}], {what}, {args.quant} int8; step = per layer quantize-append {k} "
                    "tokens/seq + causal attention of those rows",
        "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "draft": k, "quant": args.quant,
        "context_mean": float(np.mean(lens0)), "num_blocks": num_blocks,
    }
    ai = flops / kv_launch
    hbm = {"achieved": round(kv_launch / (attn_ms * 1e-3) / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
           "frac": round(kv_launch / (attn_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes_per_launch": int(kv_launch)}
    mfma = {"achieved": round(tflops, 2), "peak": MFMA_F16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4), "flops_per_launch": flops,
            "arith_intensity": round(ai, 1)}
    compute_bound = ai > MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)  # above the ridge (~312 FLOP/B)
    roofline = {
        "bound": "mfma" if compute_bound else "hbm",
        "kernel": ("chunked-prefill" if not rollback else "verify") + " attention call (k_attn_mfma + "
                  "k_attn_merge_flat), one layer",
        "achieved": mfma["achieved"] if compute_bound else hbm["achieved"],
        "peak": MFMA_F16_PEAK_TFLOPS if compute_bound else HBM_PEAK_GBS,
        "unit": "TFLOP/s" if compute_bound else "GB/s",
        "frac": mfma["frac"] if compute_bound else hbm["frac"],
        "traffic": measured_traffic(args, "verify_attn") if rollback else None,
        "traffic_source": traffic_source(args, "verify_attn") if rollback else None,
        "bytes_per_launch": int(kv_launch),
        "avg_launch_ms": round(attn_ms, 5),
        "mfma" if not compute_bound else "hbm": mfma if not compute_bound else hbm,
    }
    accepted = accepted_total[0] - acc0
    extra = {"tokens_per_s": round(accepted / args.steps / (ms_step * 1e-3), 1),
             "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4), "step_bytes": int(step_bytes),
             "wall_s_timed": round(wall, 4)}
    rec = _record(args, w, env, gbs_step, ms_step, config, roofline, extra)
    del q_all, k_new, v_new, out, ws
    env.pool.close()
    return rec


def measured_traffic(args, call):
    """HBM bytes per call of the timed entry point from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated against a plain
    copy), when it was taken on this workload; None otherwise.  Not measured
    in this run: the counters need their own rocprofv3 --pmc runs."""
    name = f"{call}_{args.workload}_{args.quant}_traffic.json"
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec.get("traffic_bytes_per_call")


def traffic_source(args, call):
    """Where roofline.traffic comes from (None when there is no figure)."""
    name = f"{call}_{args.workload}_{args.quant}_traffic.json"
    if measured_traffic(args, call) is None:
        return None
    return (f"profiles/{name}: rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE of this call in their own runs, "
            "scaled by a plain copy's counters; committed, not measured in this run")


def cpu_baseline(args, w, lens0, per_tok):
    """Time the oracle's restatement of the reference step (quantize row ->
    concat -> full-cache fp16 dequant -> SDPA as MLX's composed ops, float32 for
    bf16 queries) on a bounded sample."""
    from oracle import oracle as O

    Hq, Hkv, D = w["Hq"], w["Hkv"], w["D"]
    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    sample_layers = 2
    B = len(lens0)
    rng = Philox(args.seed, S_CPU)
    base = O.Baseline(sample_layers, B, Hkv, Hq, D, lens0.astype(np.int32), seed=args.seed)
    threads = base.threads
    q = O.f32_to_bf16_bits(rng.normal((sample_layers, B, Hq, D)).numpy())
    k = O.f32_to_bf16_bits(rng.normal((sample_layers, B, Hkv, D)).numpy())
    v = O.f32_to_bf16_bits(rng.normal((sample_layers, B, Hkv, D)).numpy())
    out = np.empty((sample_layers, B, Hq, D), np.float32)
    sc = w.get("scale", 1.0 / math.sqrt(D))
    base.step(q, k, v, O.DT_BF16, sc, out)  # warm (allocations)
    reps = 0
    t0 = time.perf_counter()
    while True:
        base.step(q, k, v, O.DT_BF16, sc, out)
        reps += 1
        el = time.perf_counter() - t0
        if el > 12.0 or reps >= 100000:
            break
    per_layer_s = el / (reps * sample_layers)
    # the same restatement on one thread: one step of one layer
    base.set_threads(1)
    one_reps = 0
    t1 = time.perf_counter()
    while True:
        base.step(q, k, v, O.DT_BF16, sc, out, layers_to_run=1)
        one_reps += 1
        one_el = time.perf_counter() - t1
        if one_el > 2.0 or one_reps >= 100000:
            break
    one_s = one_el / one_reps
    base.close()
    ctx = float(np.sum(lens0)) + 1.5 * B
    # the restatement stores the reference's row layout: per token and layer
    # 2 Hkv D payload bytes + one fp16 (scale, zero) pair per head for K and V
    per_tok = algorithmic_bytes_per_token_layer(Hkv, D, 1)
    gbs = ctx * per_tok / per_layer_s / 1e9
    layers = w["layers"]
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "tokens_per_s": round(B / (per_layer_s * layers), 3),
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} decode steps x {sample_layers} layers of the same batch ({B} seqs, same lengths) "
                  f"through the CPU restatement of the reference step (row quantize, concat, full fp16 dequant, "
                  f"SDPA as MLX's composed ops, float32 for bf16 queries); {el:.1f} s; GB/s on the row layout's {per_tok} B per token and layer; "
                  f"tokens/s extrapolated to {layers} layers",
        "single_thread": {"value": round(ctx * per_tok / one_s / 1e9, 3), "unit": "GB/s",
                          "tokens_per_s": round(B / (one_s * layers), 4),
                          "sample": f"{one_reps} decode steps of one layer on one thread, {one_el:.1f} s"},
    }


if __name__ == "__main__":
    main()
