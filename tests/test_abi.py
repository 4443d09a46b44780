"""The C ABI: the library loads without a GPU, exports every entry point the
header declares, and reports errors as codes plus a message (never aborts)."""
import ctypes
import re

import numpy as np
import pytest

import krill_amd
from krill_amd import KrillError
from krill_amd import _lib as L


def header_functions():
    text = open(L.HEADER_PATH).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(krill_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(L.LIB_PATH)
    names = header_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_bindings_cover_every_declared_symbol():
    assert sorted(L.SIGNATURES) == header_functions()


def test_abi_version_and_empty_error():
    assert L.lib().krill_abi_version() == 1
    L.lib().krill_seq_create(None, None)
    assert "pool" in L.last_error()


def test_pool_create_validates_the_descriptor():
    for kw, code in [(dict(head_dim=96), L.KRILL_E_UNSUPPORTED), (dict(num_blocks=0), L.KRILL_E_INVAL)]:
        args = dict(num_layers=1, num_kv_heads=2, head_dim=128, num_blocks=4)
        args.update(kw)
        with pytest.raises(KrillError) as e:
            krill_amd.KVPool(args["num_layers"], args["num_kv_heads"], args["head_dim"], args["num_blocks"],
                             host_only=True)
        assert e.value.code == code and e.value.message
    with pytest.raises(KrillError) as e:
        krill_amd.KVPool(1, 2, 128, 4, host_only=True, evict_watermark=1.5)
    assert e.value.code == L.KRILL_E_INVAL


def test_kernels_refuse_host_only_pools():
    p = krill_amd.KVPool(2, 2, 128, 8, host_only=True)
    lib = L.lib()
    dummy = ctypes.c_void_p(16)
    rc = lib.krill_quantize_append(p.handle, 0, dummy, dummy, dummy, 1, 1, None)
    assert rc == L.KRILL_E_STATE and "host-only" in L.last_error()
    rc = lib.krill_decode_attention(p.handle, 0, dummy, dummy, dummy, 1, 1, 64, 8, 0.1, dummy, L.DTYPE_F32,
                                    dummy, 1 << 20, None)
    assert rc == L.KRILL_E_STATE
    snap = L.Snapshot(16, 16, 16, 16, 16, 16)
    assert lib.krill_gather(p.handle, 0, dummy, dummy, 1, 1, 1, 0, ctypes.byref(snap), None) == L.KRILL_E_STATE
    assert lib.krill_copy_blocks(p.handle, dummy, 1, None) == L.KRILL_E_STATE


def test_workspace_size_and_path_limits():
    p = krill_amd.KVPool(1, 8, 128, 64, host_only=True)
    ws = p.workspace_size(32, 40, 1, 8192)
    assert ws > 0
    p.set_option(L.OPT_ATTN_PATH, 1)  # VALU only: 9+ rows per KV head are not supported there
    with pytest.raises(KrillError) as e:
        p.workspace_size(4, 8 * 4, 8, 1024)
    assert e.value.code == L.KRILL_E_UNSUPPORTED
    p.set_option(L.OPT_ATTN_PATH, 0)
    assert p.workspace_size(4, 8 * 4, 8, 1024) > 0
    with pytest.raises(KrillError):
        p.workspace_size(4, 30, 1, 1024)  # Hq not a multiple of Hkv
    with pytest.raises(KrillError):
        p.set_option(99, 1)


def test_stats_shape_and_block_bytes():
    p = krill_amd.KVPool(3, 8, 128, 10, "affine_g64", host_only=True)
    st = p.stats()
    # per (layer, block): 8 heads x (K + V bytes + 2 x 64 tokens x 2 groups x 4 bytes)
    assert st["block_bytes"] == 8 * (128 * 128 + 512 * 2)
    assert st["device_bytes"] == 0 and st["num_blocks"] == 10
    q = krill_amd.KVPool(3, 8, 128, 10, "ref_row", host_only=True)
    assert q.stats()["block_bytes"] == 8 * (128 * 128 + 512)


def test_batch_tables_and_block_table():
    p = krill_amd.KVPool(1, 2, 64, 32, host_only=True)
    a, b = p.seq_create(), p.seq_create()
    p.reserve_append(a, 130)
    p.reserve_append(b, 5)
    tables, lens = p.batch_tables([a, b], 4)
    assert lens.tolist() == [130, 5]
    assert tables[0, :3].tolist() == p.block_table(a).tolist() and tables[0, 3] == 0
    assert tables[1, 0] == p.block_table(b)[0]
    with pytest.raises(KrillError) as e:
        p.batch_tables([a], 2)
    assert e.value.code == L.KRILL_E_RANGE
    assert np.all(np.isin(p.block_table(a), np.arange(32)))


def test_cascade_and_window_entry_points_validate_on_host():
    p = krill_amd.KVPool(1, 8, 128, 64, host_only=True)
    lib = L.lib()
    out = ctypes.c_size_t()
    # shared-prefix cascade: a prefix of at least one block; sizes grow with the batch
    assert lib.krill_shared_prefix_workspace_size(p.handle, 4, 40, 0, 100, ctypes.byref(out)) == L.KRILL_E_INVAL
    assert lib.krill_shared_prefix_workspace_size(p.handle, 4, 40, 64, 100, ctypes.byref(out)) == L.KRILL_OK
    small = out.value
    assert lib.krill_shared_prefix_workspace_size(p.handle, 64, 40, 64, 100, ctypes.byref(out)) == L.KRILL_OK
    assert out.value > small
    # windowed attention: window >= 2, workspace holds the per-call table view
    assert lib.krill_window_workspace_size(p.handle, 4, 40, 1, 128, 8192, 1, ctypes.byref(out)) == L.KRILL_E_INVAL
    assert lib.krill_window_workspace_size(p.handle, 4, 40, 1, 128, 8192, 1024, ctypes.byref(out)) == L.KRILL_OK
    assert out.value >= 4 * 128 * 4
    dummy = ctypes.c_void_p(16)
    rc = lib.krill_attention_windowed(p.handle, 0, dummy, 1, dummy, dummy, None, 1024, 1, 1, 64, 8, 0.1, dummy,
                                      L.DTYPE_F32, dummy, 1 << 20, None)
    assert rc == L.KRILL_E_STATE and "host-only" in L.last_error()
    rc = lib.krill_decode_attention_shared_prefix(p.handle, 0, dummy, dummy, 1, dummy, dummy, 1, 1, 1, 8, 0.1,
                                                  dummy, L.DTYPE_F32, dummy, 1 << 20, None)
    assert rc == L.KRILL_E_STATE
    # batch_starts: bad handles are errors, not crashes
    seqs = np.array([12345], np.int32)
    starts = np.zeros(1, np.int32)
    rc = lib.krill_batch_starts(p.handle, seqs.ctypes.data_as(L.PI32), 1, starts.ctypes.data_as(L.PI32))
    assert rc == L.KRILL_E_INVAL
    s = p.seq_create()
    assert p.batch_starts([s]).tolist() == [0]
    with pytest.raises(KrillError):
        p.set_option(L.OPT_WINDOW, -5)
    p.close()
