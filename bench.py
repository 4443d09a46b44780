"""Benchmark of the int8 paged KV hot path on one MI355X.

A step is one decode pass of the hot path over one batch: for every layer,
quantize-append one new token per sequence into the paged pool, then paged
int8 decode attention over each sequence's whole cache (split-K merge
included); plus the host block-manager work of the step (slot reservation,
block tables) and its small host->device copies.

Default workload: Qwen3-14B-shaped KV (40 layers, 40 query / 8 KV heads,
head_dim 128), affine int8 in groups of 64 with fp16 scale/bias, batch 32,
context lengths uniform in [512, 8192], 64-token blocks whose ids are a
seeded random permutation of the pool, bf16 N(0,1) inputs resident in HBM.

Prints one JSON line (see README/DESIGN for the fields).
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "int8-KV paged decode-attn GB/s (% HBM peak) + tokens/s, B=32 Qwen3-14B shape"

WORKLOADS = {
    # name: (layers, Hq, Hkv, D, B, lo, hi)
    "qwen3-14b-b32": (40, 40, 8, 128, 32, 512, 8192),
    "llama-3.2-1b-b1": (16, 32, 8, 64, 1, 2048, 2048),
    "qwen3-30b-a3b-b8-128k": (48, 32, 4, 128, 8, 131072, 131072),
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--workload", default="qwen3-14b-b32", choices=sorted(WORKLOADS))
    ap.add_argument("--quant", default="affine_g64", choices=["affine_g64", "ref_row"])
    ap.add_argument("--split-blocks", type=int, default=0)
    ap.add_argument("--unfused", action="store_true",
                    help="step as two calls per layer (quantize-append, then decode attention) instead of the "
                         "fused krill_decode_append_attention")
    ap.add_argument("--kernel-reps", type=int, default=5, help="repetitions of the attention-only timing loop")
    ap.add_argument("--cpu-baseline", type=int, default=1, help="1: time the CPU baseline sample on rank 0")
    ap.add_argument("--seed", type=int, default=20261203)
    ap.add_argument("--copy-calibration", type=int, default=0,
                    help="MiB for a plain device copy (torch.neg of float32) run before the bench, so one "
                         "rocprofv3 --pmc run reads FETCH_SIZE/WRITE_SIZE of a kernel of known traffic too")
    return ap.parse_args()


def algorithmic_bytes_per_token_layer(Hkv, D, G):
    # int8 K and V payload + fp16 (scale, zero) for K and V per group
    return 2 * Hkv * D + 2 * Hkv * G * 4


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: every box in this setup has one MI355X; --gpus {args.gpus} is not "
              "supported (the path would shard by sequence / KV head, see DESIGN.md)", file=sys.stderr)
        sys.exit(2)

    import torch

    import krill_amd
    from krill_amd import _lib as KL

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    layers, Hq, Hkv, D, B, lo, hi = WORKLOADS[args.workload]
    G = D // 64 if args.quant == "affine_g64" else 1
    R = Hq // Hkv
    rng = np.random.default_rng(args.seed)
    lens0 = rng.integers(lo, hi + 1, size=B).astype(np.int64)
    total_steps = args.warmup + args.steps + 1
    blocks_needed = int(sum((int(T) + total_steps + 63) // 64 for T in lens0))
    num_blocks = blocks_needed + max(16, blocks_needed // 8)
    max_len_final = int(lens0.max()) + total_steps
    max_blocks = (max_len_final + 63) // 64

    pool = krill_amd.KVPool(layers, Hkv, D, num_blocks, args.quant, "bf16", free_list_seed=args.seed)
    if args.split_blocks:
        pool.set_option(KL.OPT_SPLIT_BLOCKS, args.split_blocks)
    lib = KL.lib()
    h = pool.handle
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    gen = torch.Generator(device=dev)
    gen.manual_seed(args.seed)

    if args.copy_calibration:
        n = args.copy_calibration * (1 << 20) // 4
        x = torch.ones(n, dtype=torch.float32, device=dev)
        y = torch.empty_like(x)
        for _ in range(3):
            torch.neg(x, out=y)
        torch.cuda.synchronize()
        del x, y

    # ---- fill every layer with the initial contexts (product path: reserve + quantize-append)
    seqs = [pool.seq_create() for _ in range(B)]
    Tmax = int(lens0.max())
    slots = np.full((B, Tmax), -1, np.int32)
    for b in range(B):
        slots[b, : lens0[b]] = pool.reserve_append(seqs[b], int(lens0[b]))
    slots_d = torch.from_numpy(slots).to(dev)
    chunk = 1024
    for layer in range(layers):
        for t0 in range(0, Tmax, chunk):
            L = min(chunk, Tmax - t0)
            k = torch.randn((B, Hkv, L, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
            v = torch.randn((B, Hkv, L, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
            sm = slots_d[:, t0: t0 + L].contiguous()
            KL.check(lib.krill_quantize_append(h, layer, k.data_ptr(), v.data_ptr(), sm.data_ptr(), B, L, sp))
    del slots_d
    torch.cuda.synchronize()

    # ---- per-step inputs, resident in HBM
    q_all = torch.randn((layers, B, Hq, 1, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    k_new = torch.randn((layers, B, Hkv, 1, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    v_new = torch.randn((layers, B, Hkv, 1, D), generator=gen, device=dev, dtype=torch.float32).to(torch.bfloat16)
    out = torch.empty((B, Hq, 1, D), dtype=torch.bfloat16, device=dev)
    ws_bytes = pool.workspace_size(B, Hq, 1, max_len_final)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    scale = 1.0 / math.sqrt(D)

    NBUF = 3
    pin_slots = [torch.empty((B, 1), dtype=torch.int32).pin_memory() for _ in range(NBUF)]
    pin_tables = [torch.empty((B, max_blocks), dtype=torch.int32).pin_memory() for _ in range(NBUF)]
    pin_lens = [torch.empty((B,), dtype=torch.int32).pin_memory() for _ in range(NBUF)]
    buf_events = [None] * NBUF
    d_slots = torch.empty((B, 1), dtype=torch.int32, device=dev)
    d_tables = torch.empty((B, max_blocks), dtype=torch.int32, device=dev)
    d_lens = torch.empty((B,), dtype=torch.int32, device=dev)
    seqs_np = np.array(seqs, np.int32)
    one_slot = np.empty(1, np.int32)
    i32p = lambda a: a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))  # noqa: E731
    qp = [q_all[l].data_ptr() for l in range(layers)]
    kp = [k_new[l].data_ptr() for l in range(layers)]
    vp = [v_new[l].data_ptr() for l in range(layers)]
    outp, wsp = out.data_ptr(), ws.data_ptr()
    cur_len = [int(x) for x in lens0]

    def fused_call(layer, mx):
        # the token at position len - 1 (its slot reserved above) is written, then attended over
        KL.check(lib.krill_decode_append_attention(h, layer, qp[layer], kp[layer], vp[layer], Hkv * D, D,
                                                   d_tables.data_ptr(), d_lens.data_ptr(), B, max_blocks, mx, Hq,
                                                   ctypes.c_float(scale), outp, KL.DTYPE_BF16, wsp, ws_bytes, sp))

    def attn_call(layer, mx):
        if args.unfused:
            KL.check(lib.krill_decode_attention(h, layer, qp[layer], d_tables.data_ptr(), d_lens.data_ptr(), B,
                                                max_blocks, mx, Hq, ctypes.c_float(scale), outp, KL.DTYPE_BF16,
                                                wsp, ws_bytes, sp))
        else:
            fused_call(layer, mx)  # rewrites the same token: the pool does not change

    def step(i):
        j = i % NBUF
        if buf_events[j] is not None:
            buf_events[j].synchronize()
        ps, pt, pl = pin_slots[j].numpy(), pin_tables[j].numpy(), pin_lens[j].numpy()
        for b in range(B):
            KL.check(lib.krill_seq_reserve_append(h, seqs[b], 1, i32p(one_slot)))
            ps[b, 0] = one_slot[0]
            cur_len[b] += 1
        KL.check(lib.krill_batch_tables(h, i32p(seqs_np), B, max_blocks, i32p(pt), i32p(pl)))
        if args.unfused:
            d_slots.copy_(pin_slots[j], non_blocking=True)
        d_tables.copy_(pin_tables[j], non_blocking=True)
        d_lens.copy_(pin_lens[j], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        buf_events[j] = ev
        mx = max(cur_len)
        for layer in range(layers):
            if args.unfused:
                KL.check(lib.krill_quantize_append(h, layer, kp[layer], vp[layer], d_slots.data_ptr(), B, 1, sp))
                KL.check(lib.krill_decode_attention(h, layer, qp[layer], d_tables.data_ptr(), d_lens.data_ptr(),
                                                    B, max_blocks, mx, Hq, ctypes.c_float(scale), outp,
                                                    KL.DTYPE_BF16, wsp, ws_bytes, sp))
            else:
                fused_call(layer, mx)

    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    lens_start = list(cur_len)
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    t_start.record(stream)
    for i in range(args.steps):
        step(args.warmup + i)
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_step = t_start.elapsed_time(t_end) / args.steps

    per_tok = algorithmic_bytes_per_token_layer(Hkv, D, G)
    # attention reads each sequence's cache (incl. the appended token); average over timed steps
    avg_ctx = [(lens_start[b] + cur_len[b] + 1) / 2.0 for b in range(B)]
    kv_bytes_layer = sum(avg_ctx) * per_tok
    qo_bytes_layer = B * Hq * D * 2 * 2
    step_bytes = layers * (kv_bytes_layer + qo_bytes_layer)
    gbs_step = step_bytes / (ms_step * 1e-3) / 1e9
    tok_s = B / (ms_step * 1e-3)

    # ---- dominant kernel alone: paged decode attention (+ its split merge; with the append fused unless
    # --unfused), all layers
    mx = max(cur_len)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for layer in range(layers):  # warm
        attn_call(layer, mx)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(args.kernel_reps):
        for layer in range(layers):
            attn_call(layer, mx)
    e1.record(stream)
    torch.cuda.synchronize()
    attn_ms = e0.elapsed_time(e1) / (args.kernel_reps * layers)
    launch_bytes = sum(cur_len) * per_tok + qo_bytes_layer
    if not args.unfused:  # the new token: bf16 K/V rows in, quantized bytes out
        launch_bytes += B * (2 * Hkv * D * 2 + per_tok)
    achieved = launch_bytes / (attn_ms * 1e-3) / 1e9

    # ---- CPU baseline: the reference's per-step algorithm on the host cores
    cpu = None
    if args.cpu_baseline:
        cpu = cpu_baseline(args, Hq, Hkv, D, lens0, per_tok)

    stats = pool.stats()
    pool.close()
    rec = {
        "metric": METRIC,
        "value": round(gbs_step, 2),
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
        "config": {
            "workload": f"{args.workload}: {layers} layers, Hq {Hq}, Hkv {Hkv}, D {D}, B {B}, "
                        f"context U[{lo},{hi}], 64-token blocks (permuted pool), {args.quant} int8, "
                        "bf16 N(0,1) inputs; step = per layer quantize-append 1 token/seq + paged decode attention"
                        + (" (two calls)" if args.unfused else " (one fused call)"),
            "layers": layers, "Hq": Hq, "Hkv": Hkv, "head_dim": D, "batch": B, "quant": args.quant,
            "context_mean": float(np.mean(lens0)), "num_blocks": num_blocks,
        },
        "tokens_per_s": round(tok_s, 1),
        "hbm_frac_step": round(gbs_step / HBM_PEAK_GBS, 4),
        "step_bytes": int(step_bytes),
        "wall_s_timed": round(wall, 4),
        "roofline": {
            "bound": "hbm",
            "kernel": ("paged decode attention call (k_attn_valu + k_attn_merge_flat), one layer" if args.unfused
                       else "fused append + paged decode attention call (k_attn_valu + k_attn_merge_flat), "
                            "one layer"),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args),
            "bytes_per_launch": int(launch_bytes),
            "avg_launch_ms": round(attn_ms, 5),
        },
        "cpu_baseline": cpu,
        "pool": {"cow_copies": stats["cow_copies"], "blocks_used": stats["blocks_used"]},
    }
    print(json.dumps(rec))


def measured_traffic(args):
    """HBM bytes per call of the timed entry point from the committed
    rocprofv3 PMC summary (FETCH_SIZE + WRITE_SIZE, calibrated against a plain
    copy), when it was taken on this workload; None otherwise."""
    call = "decode_attn" if args.unfused else "decode_append_attn"
    path = os.path.join(ROOT, "profiles", f"{call}_{args.workload}_{args.quant}_traffic.json")
    try:
        with open(path) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    return rec.get("traffic_bytes_per_call")


def cpu_baseline(args, Hq, Hkv, D, lens0, per_tok):
    """Time the oracle's restatement of the reference step (quantize row ->
    concat -> full-cache fp16 dequant -> fp32 SDPA) on a bounded sample."""
    from oracle import oracle as O

    cores = len(os.sched_getaffinity(0))
    os.environ.setdefault("OMP_NUM_THREADS", str(cores))
    sample_layers = 2
    B = len(lens0)
    rng = np.random.default_rng(args.seed + 1)
    base = O.Baseline(sample_layers, B, Hkv, Hq, D, lens0.astype(np.int32), seed=args.seed)
    threads = base.threads
    q = O.f32_to_bf16_bits(rng.standard_normal((sample_layers, B, Hq, D)).astype(np.float32))
    k = O.f32_to_bf16_bits(rng.standard_normal((sample_layers, B, Hkv, D)).astype(np.float32))
    v = O.f32_to_bf16_bits(rng.standard_normal((sample_layers, B, Hkv, D)).astype(np.float32))
    out = np.empty((sample_layers, B, Hq, D), np.float32)
    base.step(q, k, v, O.DT_BF16, 1.0 / math.sqrt(D), out)  # warm (allocations)
    reps = 0
    t0 = time.perf_counter()
    while True:
        base.step(q, k, v, O.DT_BF16, 1.0 / math.sqrt(D), out)
        reps += 1
        el = time.perf_counter() - t0
        if el > 12.0 or reps >= 500:
            break
    per_layer_s = el / (reps * sample_layers)
    base.close()
    ctx = float(np.sum(lens0)) + 1.5 * B
    gbs = ctx * per_tok / per_layer_s / 1e9
    layers = WORKLOADS[args.workload][0]
    return {
        "value": round(gbs, 3),
        "unit": "GB/s",
        "tokens_per_s": round(B / (per_layer_s * layers), 3),
        "cores": threads,
        "kind": "port",
        "sample": f"{reps} decode steps x {sample_layers} layers of the same batch ({B} seqs, same lengths) "
                  f"through the CPU restatement of the reference step (row quantize, concat, full fp16 dequant, "
                  f"fp32 SDPA); {el:.1f} s; tokens/s extrapolated to {layers} layers",
    }


if __name__ == "__main__":
    main()
