"""krill_amd: MI355X (gfx950) int8 paged KV-cache hot path for Krill.

The product is libkrillhip.so (C ABI: include/libkrillhip.h), built from
krill_amd/csrc.  This package is its Python face: ctypes bindings, a pool
wrapper and the reference-shaped cache API used by tests and the benchmark.
"""
from ._lib import KrillError, KrillLibraryError, lib  # noqa: F401
from .cache import (PagedQuantizedKVCache, PrefixCache, QuantizedKVSnapshot, SequenceKV,  # noqa: F401
                    make_quantized_kv_caches)
from .kernels import KrillKernels  # noqa: F401
from .pool import KVPool, prefix_key  # noqa: F401

__all__ = [
    "KrillError", "KrillLibraryError", "lib", "KVPool", "prefix_key", "PagedQuantizedKVCache", "PrefixCache",
    "QuantizedKVSnapshot", "SequenceKV", "make_quantized_kv_caches", "KrillKernels",
]
