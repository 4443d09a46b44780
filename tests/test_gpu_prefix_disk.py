"""GPU: the prefix cache's disk tier end to end.  A stored entry is written
as ``<key>.q8.safetensors`` (key: the library's FNV-1a v3 prefix key); after
the memory entries are gone, a lookup restores it from the file into fresh
blocks, and the restored sequence holds the original bytes (every layer,
token, scale and zero) and gives the same attention output bit for bit.
The file's arrays equal the oracle's quantization of the stored rows (shape
[1, Hkv, T, ...] per layer, as PrefixCache.swift:600-627 writes them), so a
row-mode pool writes the reference's on-disk entries.  The file is written
behind the store (PrefixCache.swift:397-399)."""
import numpy as np
import pytest

from kvutil import Filled, i32, rand_bits, to_dev

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
if not torch.cuda.is_available():  # pragma: no cover - CPU container
    pytest.skip("no HIP device", allow_module_level=True)

import krill_amd  # noqa: E402
from krill_amd import q8file  # noqa: E402
from krill_amd.cache import PrefixCache  # noqa: E402
from krill_amd.pool import prefix_key  # noqa: E402


def _snap(pool, seq, n, layer):
    t, _ = pool.batch_tables([seq], max(1, (n + 63) // 64))
    return {k: v.cpu().numpy() for k, v in pool.gather(layer, i32(t), i32([n]), n).items()}


@pytest.mark.parametrize("mode", ["ref_row", "affine_g64"])
def test_disk_round_trip_restores_identical_cache(mode, tmp_path):
    print(f"\ncase prefix_disk mode={mode}", flush=True)
    H, D, layers, T = 2, 128, 3, 300
    pool = krill_amd.KVPool(layers, H, D, 64, mode, "bf16", free_list_seed=3)
    f = Filled(pool, [T], np.random.default_rng(1), "bf16", layers=tuple(range(layers)))
    seq = f.seqs[0]
    tokens = np.arange(1000, 1000 + T)
    pc = PrefixCache(pool, "model-x", cache_dir=tmp_path, disk_budget_gb=1)
    assert pc.store_quantized(tokens, seq)
    pc.wait_for_disk_writes()
    key = prefix_key("model-x", None, 2, tokens)
    path = tmp_path / f"{key:016x}.q8.safetensors"
    assert path.exists() and pc.disk_count == 1
    file_layers = q8file.load_entry(path)
    assert len(file_layers) == layers
    for layer in range(layers):
        kq, ks, kz, vq, vs, vz = f.expected(layer, 0)
        want = {"keys": kq, "values": vq, "key_scales": ks, "key_zeros": kz, "value_scales": vs,
                "value_zeros": vz}
        for field, _ in q8file.NAMES:
            got = file_layers[layer][field]
            assert got.shape[0] == 1 and got.shape[1:] == want[field].shape, (layer, field, got.shape)
            if got.dtype == np.float16:
                got = got.view(np.uint16)
            np.testing.assert_array_equal(got[0], want[field])

    # memory gone, file kept: a fresh cache object on the same directory
    pool.prefix_clear()
    pc2 = PrefixCache(pool, "model-x", cache_dir=tmp_path, disk_budget_gb=1)
    # the request runs 20 tokens past the entry: the scan reaches it (step 4)
    n, entry = pc2.lookup_quantized(np.concatenate([tokens, np.arange(20)]))
    assert n == T and entry is not None and pc2.memory_count == 1
    restored = pool.seq_fork(entry, T)
    for layer in range(layers):
        a, b = _snap(pool, seq, T, layer), _snap(pool, restored, T, layer)
        for field in a:
            assert np.array_equal(a[field].view(np.uint8), b[field].view(np.uint8)), (layer, field)
        # and the oracle's bytes
        kq, _, kz, vq, vs, _ = f.expected(layer, 0)
        np.testing.assert_array_equal(b["keys"][0], kq)
        np.testing.assert_array_equal(b["values"][0], vq)
        np.testing.assert_array_equal(b["key_zeros"][0].view(np.uint16), kz)
        np.testing.assert_array_equal(b["value_scales"][0].view(np.uint16), vs)

    # attention over the original and the restored sequence: identical
    q = to_dev(rand_bits(np.random.default_rng(2), (2, H * 4, 1, D), "bf16"), "bf16")
    tabs, lens = pool.batch_tables([seq, restored], (T + 63) // 64)
    out = pool.attention(layers - 1, q[:1].expand(2, -1, -1, -1).contiguous(), i32(tabs), i32(lens), T,
                         1 / np.sqrt(D))
    torch.cuda.synchronize()
    assert torch.equal(out[0], out[1])
    pool.close()


def test_disk_entry_of_other_model_or_length_is_a_miss(tmp_path):
    print("\ncase prefix_disk_miss", flush=True)
    pool = krill_amd.KVPool(1, 2, 64, 16, "ref_row", "bf16", free_list_seed=4)
    f = Filled(pool, [40], np.random.default_rng(5), "bf16")
    tokens = np.arange(40)
    pc = PrefixCache(pool, "a", cache_dir=tmp_path, disk_budget_gb=1)
    assert pc.store_quantized(tokens, f.seqs[0])
    pool.prefix_clear()
    assert PrefixCache(pool, "b", cache_dir=tmp_path).lookup_quantized(tokens) == (0, None)
    # shorter request: every scanned length misses (the file holds 40 tokens)
    assert PrefixCache(pool, "a", cache_dir=tmp_path).lookup_quantized(tokens[:39]) == (0, None)
    assert PrefixCache(pool, "a", cache_dir=tmp_path).lookup_quantized(tokens)[0] == 40
    pool.close()
