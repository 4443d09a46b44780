"""The benchmark's synthetic inputs: Philox4x32-10 against the known-answer
vectors of its authors' Random123 library (kat_vectors: counter and key all
zero, all ones, and the digits of pi), and the streams built on it
(reproducible, integers in range, Box-Muller normals with mean 0 and
variance 1)."""
import importlib.util
import os

import numpy as np
import pytest

torch = pytest.importorskip("torch")

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
_spec = importlib.util.spec_from_file_location("bench_inputs", os.path.join(ROOT, "bench.py"))
bench = importlib.util.module_from_spec(_spec)
_spec.loader.exec_module(bench)


@pytest.mark.parametrize("ctr,key,want", [
    ((0, 0, 0, 0), (0, 0), (0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8)),
    ((0xFFFFFFFF,) * 4, (0xFFFFFFFF, 0xFFFFFFFF), (0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD)),
    ((0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344), (0xA4093822, 0x299F31D0),
     (0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1)),
])
def test_philox4x32_10_known_answers(ctr, key, want):
    t = [torch.tensor([c], dtype=torch.int64) for c in ctr]
    got = tuple(int(x.item()) for x in bench.philox4x32_10(*t, key[0], key[1]))
    assert got == want


def test_streams_are_reproducible_and_in_range():
    a = bench.Philox(20261202, bench.S_LENGTHS).integers(512, 8193, size=1000)
    b = bench.Philox(20261202, bench.S_LENGTHS).integers(512, 8193, size=1000)
    assert np.array_equal(a, b)
    assert a.min() >= 512 and a.max() <= 8192 and len(np.unique(a)) > 900
    # another stream of the same seed is another sequence
    c = bench.Philox(20261202, bench.S_FILL).integers(512, 8193, size=1000)
    assert not np.array_equal(a, c)
    # draws continue the counter: a draw of 6 words takes 2 counters, so the
    # next draw starts at counter 2
    r = bench.Philox(7, 0)
    h = np.concatenate([r.integers(0, 100, size=6), r.integers(0, 100, size=6)])
    assert np.array_equal(h[:6], bench.Philox(7, 0).integers(0, 100, size=6))
    s = bench.Philox(7, 0)
    s.uniform(8)
    assert np.array_equal(h[6:], s.integers(0, 100, size=6))
    k = bench.Philox(3, bench.S_OUTLIERS).choice(1024, 100)
    assert len(set(k.tolist())) == 100 and k.min() >= 0 and k.max() < 1024


def test_box_muller_normals():
    z = bench.Philox(20261202, bench.S_STEP).normal((1 << 20,)).double().numpy()
    assert abs(z.mean()) < 5e-3 and abs(z.var() - 1.0) < 5e-3
    # tails of a normal: P(|z| > 3) = 0.0027
    assert 0.0022 < np.mean(np.abs(z) > 3.0) < 0.0032
    # each counter gives two Box-Muller pairs: z0^2 + z1^2 = -2 ln u1 > 0
    assert np.all(np.isfinite(z))
