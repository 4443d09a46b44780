"""CPU: the on-disk prefix-entry format (``<key>.q8.safetensors``, key names
and layout of PrefixCache.swift:553-627) and the disk tier's byte budget
(PrefixCache.swift:600-695).  The file is checked byte-level against the
safetensors layout (8-byte little-endian header length, JSON header with
dtype / shape / data_offsets per tensor, raw little-endian data), not only
through the safetensors reader."""
import json
import os
import struct

import numpy as np
import pytest

from krill_amd import q8file


def _layers(n_layers=2, H=2, T=5, D=64, G=1, seed=0):
    rng = np.random.default_rng(seed)
    out = []
    for _ in range(n_layers):
        out.append({
            "keys": rng.integers(0, 256, (1, H, T, D), dtype=np.uint8),
            "values": rng.integers(0, 256, (1, H, T, D), dtype=np.uint8),
            "key_scales": rng.standard_normal((1, H, T, G)).astype(np.float16),
            "key_zeros": rng.standard_normal((1, H, T, G)).astype(np.float16),
            "value_scales": rng.standard_normal((1, H, T, G)).astype(np.float16),
            "value_zeros": rng.standard_normal((1, H, T, G)).astype(np.float16),
        })
    return out


def _raw(path):
    data = open(path, "rb").read()
    (hlen,) = struct.unpack("<Q", data[:8])
    header = json.loads(data[8:8 + hlen])
    return header, data[8 + hlen:]


def test_file_layout_matches_reference_key_convention(tmp_path):
    layers = _layers(n_layers=3, G=2)
    p = tmp_path / ("%016x" % 0x0123456789ABCDEF + q8file.SUFFIX)
    q8file.save_entry(p, layers, metadata={"format": "mlx"})
    header, body = _raw(p)
    assert header.pop("__metadata__") == {"format": "mlx"}
    want = {f"layer_{i}_{t}" for i in range(3) for t in ("qk", "qv", "ks", "kz", "vs", "vz")}
    assert set(header) == want
    for i, snap in enumerate(layers):
        for field, tag in q8file.NAMES:
            h = header[f"layer_{i}_{tag}"]
            a = snap[field]
            assert h["dtype"] == ("U8" if a.dtype == np.uint8 else "F16")
            assert h["shape"] == list(a.shape)
            lo, hi = h["data_offsets"]
            assert body[lo:hi] == a.tobytes()  # little-endian, C order
    back = q8file.load_entry(p)
    assert len(back) == 3
    for a, b in zip(layers, back):
        for f, _ in q8file.NAMES:
            np.testing.assert_array_equal(a[f], b[f])
            assert a[f].dtype == b[f].dtype


def test_layers_stop_at_first_incomplete_layer():
    arrays = q8file.entry_arrays(_layers(n_layers=3))
    del arrays["layer_1_vz"]
    assert len(q8file.layers_of(arrays)) == 1
    del arrays["layer_0_qk"]
    assert q8file.layers_of(arrays) == []


def test_entry_bytes_is_the_six_arrays():
    layers = _layers(n_layers=2, H=2, T=5, D=64, G=1)
    assert q8file.entry_bytes(layers) == 2 * (2 * 2 * 5 * 64 + 4 * 2 * 5 * 1 * 2)


def test_disk_budget_evicts_oldest_to_low_water(tmp_path):
    layers = _layers(n_layers=1, H=2, T=16, D=64)  # ~4.8 kB per file
    size = len(q8file.entry_arrays(layers)["layer_0_qk"].tobytes())
    tier = q8file.DiskTier(tmp_path, disk_budget_gb=12_000 / 1e9)  # 12 kB, low water 10.8 kB
    t0 = 1_700_000_000
    tier.write(1, layers)
    os.utime(tier.path(1), (t0, t0))
    tier.write(2, layers)
    os.utime(tier.path(2), (t0 + 10, t0 + 10))
    assert tier.count == 2
    one = tier.path(1).stat().st_size
    assert 2 * size < one < 2 * size + 1024  # both payload arrays, the scales and the header
    # the third file crosses 12 kB: the oldest goes, down to <= 10.8 kB
    tier.write(3, layers)
    assert not tier.path(1).exists() and tier.path(2).exists() and tier.path(3).exists()
    # a load refreshes the file's time: 2 is now newer than 3, so 3 goes next
    os.utime(tier.path(3), (t0 + 20, t0 + 20))
    os.utime(tier.path(2), (t0 + 5, t0 + 5))
    assert tier.load(2) is not None
    tier.write(4, layers)
    assert tier.path(2).exists() and not tier.path(3).exists() and tier.path(4).exists()


def test_disk_budget_zero_disables_and_negative_never_evicts(tmp_path):
    layers = _layers(n_layers=1)
    off = q8file.DiskTier(tmp_path / "off", disk_budget_gb=0)
    assert not off.write(1, layers) and off.load(1) is None and off.count == 0
    inf = q8file.DiskTier(tmp_path / "inf", disk_budget_gb=-1)
    for k in range(5):
        inf.write(k, layers)
    assert inf.count == 5


def test_unreadable_file_is_a_miss(tmp_path):
    tier = q8file.DiskTier(tmp_path, disk_budget_gb=1)
    tier.path(7).write_bytes(b"not a safetensors file")
    assert tier.load(7) is None


@pytest.mark.parametrize("env,expect", [("0.5", 500_000_000), ("-1", -1), ("junk", 2_000_000_000)])
def test_budget_from_environment(tmp_path, monkeypatch, env, expect):
    monkeypatch.setenv("KRILL_PREFIX_CACHE_GB", env)
    assert q8file.DiskTier(tmp_path).budget == expect


def test_write_behind_runs_in_order_and_loads_wait_for_it(tmp_path, monkeypatch):
    """Background writes (PrefixCache.swift:397-399): queued in order on one
    writer; a load of a queued file waits for the queue; clear drains it."""
    import threading

    layers = _layers(n_layers=2)
    tier = q8file.DiskTier(tmp_path, disk_budget_gb=1)
    gate = threading.Event()
    order = []
    real = q8file.save_entry

    def slow_save(path, lay, metadata=None):
        gate.wait(10)  # the first write holds the writer until the test lets it go
        order.append(path.name)
        real(path, lay, metadata)

    monkeypatch.setattr(q8file, "save_entry", slow_save)
    assert tier.write(1, layers, background=True)
    assert tier.write(2, layers, background=True)
    assert not tier.path(1).exists()  # still queued behind the gate
    threading.Timer(0.2, gate.set).start()
    got = tier.load(2)  # waits for both writes
    assert got is not None and len(got) == 2
    assert order == [tier.path(1).name, tier.path(2).name]
    for f, _ in q8file.NAMES:
        np.testing.assert_array_equal(got[1][f], layers[1][f])
    tier.write(3, layers, background=True)
    tier.clear()  # the queued write lands before the directory is cleared
    assert tier.count == 0
    q8file.wait_for_disk_writes()
    assert q8file._WRITER.errors == 0
