"""Writes tests/golden/quantize_golden.npz: inputs and oracle outputs of the
two quantizers.  The reference (Swift + mlx-swift) cannot run here, so these
vectors pin the oracle against regressions; their correctness rests on the
independent checks in tests/test_oracle.py.  Inputs:
  * the Weyl-sequence fp16 tensors of QuantizedKVCacheUnitTests.swift:17-27
    ([1,4,8,16], ranges of the tests at :38-84);
  * seeded N(0,1) bf16 rows with 1% outlier channels x20;
  * edge rows: constant, two-valued, mixed sign, tiny magnitudes.
Run: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)
from oracle import oracle as O  # noqa: E402


def weyl(shape, lo, hi):
    total = int(np.prod(shape))
    span = np.float32(max(np.float32(hi) - np.float32(lo), np.float32(1e-3)))
    i = np.arange(total).astype(np.float32)
    prod = (i * np.float32(0.6180339887)).astype(np.float32)
    frac = (prod - np.trunc(prod).astype(np.float32)).astype(np.float32)
    vals = (np.float32(lo) + (frac * span).astype(np.float32)).astype(np.float32)
    return vals.reshape(shape).astype(np.float16).view(np.uint16)


def main():
    rng = np.random.default_rng(20261201)
    cases = {}
    for lo, hi in [(0.0, 10.0), (0.0, 5.0), (-64.0, 64.0), (-32.0, 64.0), (-2.0, 2.0)]:
        cases[f"weyl_{lo}_{hi}_ref"] = (weyl([1, 4, 8, 16], lo, hi), 0, 0)
    x = rng.standard_normal((8, 128)).astype(np.float32)
    x[:, rng.choice(128, 2, replace=False)] *= 20
    cases["normal_bf16_ref"] = (O.f32_to_bf16_bits(x), 1, 0)
    cases["normal_bf16_affine"] = (O.f32_to_bf16_bits(x), 1, 1)
    cases["normal_f16_affine"] = (O.f32_to_f16_bits(x), 0, 1)
    edge = np.zeros((6, 64), np.float32)
    edge[0] = 3.25
    edge[1, ::2] = -1.0
    edge[1, 1::2] = 1.0
    edge[2] = np.linspace(-7, 3, 64)
    edge[3] = np.linspace(1e-3, 2e-3, 64)
    edge[4] = np.linspace(-300, -299, 64)
    edge[5] = 0.0
    for dt, name in [(0, "f16"), (1, "bf16")]:
        bits = O.f32_to_f16_bits(edge) if dt == 0 else O.f32_to_bf16_bits(edge)
        cases[f"edge_{name}_ref"] = (bits, dt, 0)
        cases[f"edge_{name}_affine"] = (bits, dt, 1)
    out = {}
    for name, (x, dt, mode) in cases.items():
        q, s, z = O.quantize(x, dt, mode)
        out[name + "__x"] = x
        out[name + "__dt"] = np.array(dt)
        out[name + "__mode"] = np.array(mode)
        out[name + "__q"] = q
        out[name + "__s"] = s
        out[name + "__z"] = z
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "quantize_golden.npz")
    np.savez_compressed(path, **out)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(cases)} cases)")


if __name__ == "__main__":
    main()
