"""ctypes binding of libkrillhip.so (the C ABI in include/libkrillhip.h).

The library is loaded from this package directory only.  If it is missing the
import of any kernel entry point raises ``KrillLibraryError``: there is no
CPU fallback anywhere in the product path.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# KRILL_LIBRARY names another build in this directory (the diagnostic
# libkrillhip_stamps.so of `make stamps`); a bare file name only.
_LIB_NAME = os.environ.get("KRILL_LIBRARY", "libkrillhip.so")
if os.path.basename(_LIB_NAME) != _LIB_NAME or not _LIB_NAME.endswith(".so"):
    raise ValueError(f"KRILL_LIBRARY must name a .so file in {HERE}")
LIB_PATH = os.path.join(HERE, _LIB_NAME)
HEADER_PATH = os.path.join(os.path.dirname(HERE), "include", "libkrillhip.h")

KRILL_OK = 0
KRILL_E_INVAL = -1
KRILL_E_NOMEM = -2
KRILL_E_RANGE = -3
KRILL_E_HIP = -4
KRILL_E_STATE = -5
KRILL_E_UNSUPPORTED = -6

QUANT_REF_ROW = 0
QUANT_AFFINE_G64 = 1

DTYPE_F16 = 0
DTYPE_BF16 = 1
DTYPE_F32 = 2

POOL_HOST_ONLY = 1

OPT_SPLIT_BLOCKS = 1
OPT_ATTN_PATH = 2
OPT_WINDOW = 3
OPT_PREFIX_SPLIT = 4

_CODE_NAMES = {
    KRILL_E_INVAL: "KRILL_E_INVAL",
    KRILL_E_NOMEM: "KRILL_E_NOMEM",
    KRILL_E_RANGE: "KRILL_E_RANGE",
    KRILL_E_HIP: "KRILL_E_HIP",
    KRILL_E_STATE: "KRILL_E_STATE",
    KRILL_E_UNSUPPORTED: "KRILL_E_UNSUPPORTED",
}


class KrillLibraryError(RuntimeError):
    """libkrillhip.so is not built or cannot be loaded."""


class KrillError(RuntimeError):
    def __init__(self, code: int, message: str):
        self.code = code
        self.message = message
        super().__init__(f"{_CODE_NAMES.get(code, code)}: {message}")


class PoolDesc(ctypes.Structure):
    _fields_ = [
        ("num_layers", ctypes.c_int32),
        ("num_kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_tokens", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("quant_mode", ctypes.c_int32),
        ("in_dtype", ctypes.c_int32),
        ("flags", ctypes.c_uint32),
        ("evict_watermark", ctypes.c_float),
        ("max_prefix_entries", ctypes.c_int32),
        ("min_prefix_len", ctypes.c_int32),
        ("max_entry_bytes", ctypes.c_int64),
        ("free_list_seed", ctypes.c_uint64),
    ]


class PoolStats(ctypes.Structure):
    _fields_ = [
        ("num_blocks", ctypes.c_int32),
        ("blocks_used", ctypes.c_int32),
        ("blocks_free", ctypes.c_int32),
        ("blocks_shared", ctypes.c_int32),
        ("live_seqs", ctypes.c_int32),
        ("prefix_entries", ctypes.c_int32),
        ("appended_tokens", ctypes.c_int64),
        ("cow_copies", ctypes.c_int64),
        ("evicted_entries", ctypes.c_int64),
        ("evicted_blocks", ctypes.c_int64),
        ("pending_copies", ctypes.c_int64),
        ("device_bytes", ctypes.c_int64),
        ("block_bytes", ctypes.c_int64),
    ]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class Snapshot(ctypes.Structure):
    _fields_ = [
        ("keys", ctypes.c_void_p),
        ("values", ctypes.c_void_p),
        ("key_scales", ctypes.c_void_p),
        ("key_zeros", ctypes.c_void_p),
        ("value_scales", ctypes.c_void_p),
        ("value_zeros", ctypes.c_void_p),
    ]


_lib = None

I32 = ctypes.c_int32
I64 = ctypes.c_int64
U64 = ctypes.c_uint64
P = ctypes.c_void_p
PI32 = ctypes.POINTER(ctypes.c_int32)
PI64 = ctypes.POINTER(ctypes.c_int64)
STR = ctypes.c_char_p

# name -> argtypes; every entry point returns int32 unless listed in _RESTYPE.
SIGNATURES = {
    "krill_last_error": [],
    "krill_abi_version": [],
    "krill_diag_wave_stamps": [P, I32],
    "krill_pool_create": [ctypes.POINTER(PoolDesc), P, ctypes.POINTER(P)],
    "krill_pool_destroy": [P],
    "krill_pool_get_stats": [P, ctypes.POINTER(PoolStats)],
    "krill_pool_set_stream": [P, P],
    "krill_pool_refcounts": [P, PI32, I32],
    "krill_pool_set_option": [P, I32, I64],
    "krill_pool_flush": [P, P],
    "krill_seq_create": [P, PI32],
    "krill_seq_fork": [P, I32, I32, PI32],
    "krill_seq_free": [P, I32],
    "krill_seq_reset": [P, I32],
    "krill_seq_length": [P, I32, PI32],
    "krill_seq_memory_bytes": [P, I32, PI64],
    "krill_seq_truncate": [P, I32, I32],
    "krill_seq_reserve_append": [P, I32, I32, PI32],
    "krill_seq_block_table": [P, I32, PI32, I32, PI32],
    "krill_batch_tables": [P, PI32, I32, I32, PI32, PI32],
    "krill_batch_starts": [P, PI32, I32, PI32],
    "krill_prefix_store": [P, I32, STR, STR, PI64, I32, PI32],
    "krill_prefix_lookup": [P, STR, STR, PI64, I32, PI32, PI32],
    "krill_prefix_probe": [P, STR, STR, PI64, I32, PI32],
    "krill_prefix_lookup_longest": [P, STR, STR, PI64, I32, PI32, PI32],
    "krill_prefix_clear": [P],
    "krill_prefix_count": [P, PI32],
    "krill_prefix_key": [STR, STR, I32, PI64, I64, ctypes.POINTER(U64)],
    "krill_quantize_append": [P, I32, P, P, P, I32, I32, P],
    "krill_quantize_append_strided": [P, I32, P, P, I64, I64, I64, P, I32, I32, P],
    "krill_quantize_append_rope": [P, I32, P, P, I64, I64, I64, P, P, P, I32, I32, I32, P],
    "krill_gather": [P, I32, P, P, I32, I32, I32, I32, ctypes.POINTER(Snapshot), P],
    "krill_gather_dequant": [P, I32, P, P, I32, I32, I32, I32, P, P, P],
    "krill_scatter": [P, I32, ctypes.POINTER(Snapshot), I32, I32, P, P, I32, P],
    "krill_copy_blocks": [P, P, I32, P],
    "krill_attention_workspace_size": [P, I32, I32, I32, I32, ctypes.POINTER(ctypes.c_size_t)],
    "krill_decode_attention": [P, I32, P, P, P, I32, I32, I32, I32, ctypes.c_float, P, I32, P, ctypes.c_size_t, P],
    "krill_verify_attention": [P, I32, P, I32, P, P, I32, I32, I32, I32, ctypes.c_float, P, I32, P,
                               ctypes.c_size_t, P],
    "krill_decode_append_attention": [P, I32, P, P, P, I64, I64, P, P, I32, I32, I32, I32, ctypes.c_float, P,
                                      I32, P, ctypes.c_size_t, P],
    "krill_decode_append_attention_noalloc": [P, I32, P, P, P, I64, I64, P, P, I32, I32, I32, I32, ctypes.c_float,
                                              P, I32, P],
    "krill_window_workspace_size": [P, I32, I32, I32, I32, I32, I32, ctypes.POINTER(ctypes.c_size_t)],
    "krill_attention_windowed": [P, I32, P, I32, P, P, P, I32, I32, I32, I32, I32, ctypes.c_float, P, I32, P,
                                 ctypes.c_size_t, P],
    "krill_decode_append_attention_windowed": [P, I32, P, P, P, I64, I64, P, P, P, I32, I32, I32, I32, I32,
                                               ctypes.c_float, P, I32, P, I32, P, ctypes.c_size_t, P],
    "krill_shared_prefix_workspace_size": [P, I32, I32, I32, I32, ctypes.POINTER(ctypes.c_size_t)],
    "krill_decode_attention_shared_prefix": [P, I32, P, P, I32, P, P, I32, I32, I32, I32, ctypes.c_float, P, I32,
                                             P, ctypes.c_size_t, P],
    "krill_decode_append_attention_shared_prefix": [P, I32, P, P, P, I64, I64, P, I32, P, P, I32, I32, I32, I32,
                                                    ctypes.c_float, P, I32, P, ctypes.c_size_t, P],
    "krill_decode_append_attention_rope": [P, I32, P, P, P, I64, I64, P, P, I32, I32, I32, I32, ctypes.c_float, P,
                                           I32, P, I32, P, ctypes.c_size_t, P],
}
_RESTYPE = {"krill_last_error": ctypes.c_char_p}


def lib():
    """Load libkrillhip.so (once).  Raises KrillLibraryError when absent."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise KrillLibraryError(
                f"{LIB_PATH} is not built; run `make -C krill_amd/csrc` or __graft_entry__.build()")
        try:
            L = ctypes.CDLL(LIB_PATH)
        except OSError as e:  # pragma: no cover - environment specific
            raise KrillLibraryError(f"cannot load {LIB_PATH}: {e}") from e
        for name, args in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = _RESTYPE.get(name, ctypes.c_int32)
        _lib = L
    return _lib


def last_error() -> str:
    return lib().krill_last_error().decode(errors="replace")


def check(rc: int) -> int:
    if rc != KRILL_OK:
        raise KrillError(rc, last_error())
    return rc
