"""Shared helpers for the GPU parity tests: seeded inputs, filling a pool
through the product path, and the oracle's view of the same inputs."""
from __future__ import annotations

import numpy as np

from oracle import oracle as O

DT = {"bf16": O.DT_BF16, "f16": O.DT_F16}
MODE = {"ref_row": 0, "affine_g64": 1}


def rand_bits(rng, shape, dt: str, scale: float = 1.0, outlier_frac: float = 0.0, outlier_mul: float = 20.0):
    x = rng.standard_normal(shape).astype(np.float32) * scale
    if outlier_frac > 0:
        # a fixed set of channels (last axis) scaled up, as in the long-context config
        D = shape[-1]
        ch = rng.choice(D, size=max(1, int(round(outlier_frac * D))), replace=False)
        x[..., ch] *= outlier_mul
    return O.f32_to_bf16_bits(x) if dt == "bf16" else O.f32_to_f16_bits(x)


def to_dev(bits: np.ndarray, dt: str, device="cuda"):
    import torch

    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy())
    return t.view(torch.bfloat16 if dt == "bf16" else torch.float16).to(device)


def i32(a, device="cuda"):
    import torch

    return torch.as_tensor(np.ascontiguousarray(a, np.int32), device=device)


class Filled:
    """B sequences appended in random chunks to `layers` of a pool."""

    def __init__(self, pool, lens, rng, dt: str, layers=(0,), max_chunk: int = 70, scale: float = 1.0,
                 outlier_frac: float = 0.0, seqs=None):
        self.pool, self.lens, self.dt, self.layers = pool, list(lens), dt, tuple(layers)
        H, D = pool.num_kv_heads, pool.head_dim
        self.seqs = list(seqs) if seqs is not None else [pool.seq_create() for _ in self.lens]
        self.k = {l: [rand_bits(rng, (H, T, D), dt, scale, outlier_frac) for T in self.lens] for l in self.layers}
        self.v = {l: [rand_bits(rng, (H, T, D), dt, scale, outlier_frac) for T in self.lens] for l in self.layers}
        done = [0] * len(self.lens)
        B = len(self.lens)
        while any(done[b] < self.lens[b] for b in range(B)):
            L = int(rng.integers(1, max_chunk + 1))
            slots = np.full((B, L), -1, np.int32)
            take = [min(L, self.lens[b] - done[b]) for b in range(B)]
            for b in range(B):
                if take[b] > 0:
                    slots[b, : take[b]] = self.pool.reserve_append(self.seqs[b], take[b])
            for l in self.layers:
                kb = np.zeros((B, H, L, D), np.uint16)
                vb = np.zeros((B, H, L, D), np.uint16)
                for b in range(B):
                    if take[b] > 0:
                        kb[b, :, : take[b]] = self.k[l][b][:, done[b]: done[b] + take[b]]
                        vb[b, :, : take[b]] = self.v[l][b][:, done[b]: done[b] + take[b]]
                self.pool.quantize_append(l, to_dev(kb, dt), to_dev(vb, dt), i32(slots))
            for b in range(B):
                done[b] += take[b]

    def tables(self, extra_blocks: int = 0):
        mb = max((T + 63) // 64 for T in self.lens) + extra_blocks
        t, n = self.pool.batch_tables(self.seqs, max(mb, 1))
        return i32(t), i32(n), max(mb, 1)

    def expected(self, layer: int, b: int):
        """Oracle quantization of sequence b: (kq, ks, kz, vq, vs, vz), [H, T, ...]."""
        mode = MODE[self.pool.quant_mode]
        kq, ks, kz = O.quantize(self.k[layer][b], DT[self.dt], mode)
        vq, vs, vz = O.quantize(self.v[layer][b], DT[self.dt], mode)
        return kq, ks, kz, vq, vs, vz


def oracle_attention(pool, filled: Filled, layer: int, q_bits: np.ndarray, dt: str, scale: float):
    """Reference outputs [B, Hq, Lq, D] (float64) for q_bits [B, Hq, Lq, D]."""
    B, Hq, Lq, D = q_bits.shape
    H = pool.num_kv_heads
    R = Hq // H
    mode = MODE[pool.quant_mode]
    qf = O.bits_to_f32(q_bits, DT[dt]).astype(np.float64)
    out = np.zeros((B, Hq, Lq, D), np.float64)
    for b in range(B):
        T = filled.lens[b]
        kq, ks, kz, vq, vs, vz = filled.expected(layer, b)
        kd = O.dequant_f64(kq, ks, kz, mode)
        vd = O.dequant_f64(vq, vs, vz, mode)
        for hk in range(H):
            rows = np.stack([qf[b, hk * R + (r % R), r // R] for r in range(R * Lq)])
            lim = [T - Lq + r // R + 1 for r in range(R * Lq)]
            o = O.attention_f64(rows, kd[hk], vd[hk], lim, scale)
            for r in range(R * Lq):
                out[b, hk * R + (r % R), r // R] = o[r]
    return out


def check_snapshot(snap, filled, layer, left_pad=False):
    """A gathered snapshot equals the oracle's quantization of `filled`, byte
    for byte, with zero bytes in the padding."""
    S = snap["keys"].shape[2]
    got = {k: v.cpu().numpy() for k, v in snap.items()}
    for b, T in enumerate(filled.lens):
        kq, ks, kz, vq, vs, vz = filled.expected(layer, b)
        sl = slice(S - T, S) if left_pad else slice(0, T)
        pad = slice(0, S - T) if left_pad else slice(T, S)
        np.testing.assert_array_equal(got["keys"][b, :, sl], kq)
        np.testing.assert_array_equal(got["values"][b, :, sl], vq)
        np.testing.assert_array_equal(got["key_scales"][b, :, sl].view(np.uint16), ks)
        np.testing.assert_array_equal(got["key_zeros"][b, :, sl].view(np.uint16), kz)
        np.testing.assert_array_equal(got["value_scales"][b, :, sl].view(np.uint16), vs)
        np.testing.assert_array_equal(got["value_zeros"][b, :, sl].view(np.uint16), vz)
        for name in got:
            assert not np.any(got[name][b, :, pad].view(np.uint8)), f"{name} padding not zero"
