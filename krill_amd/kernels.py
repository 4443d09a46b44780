"""KrillKernels: the static kernel entry points the model layer calls.

Mirrors the static-enum registry of Sources/KrillKernels/KernelRegistry.swift
:13-162 (``isAvailable`` / ``status`` plus one static function per kernel)
as the host of the paged int8 KV kernels.  The entry points take what the
model layer holds at a decode or verify step -- the batch's
PagedQuantizedKVCache of one layer, one per sequence -- and turn it into
the library's block tables, lengths and slot mappings, so one launch serves
the whole batch where the reference stacks the per-sequence caches first
(stackCachesLeftPaddedQuantized, BatchedDecode.swift:96-151, then SDPA at
Attention.swift:95-98 / Gemma4Model.swift:516-517).  Every call goes into
libkrillhip; a missing library or device raises instead of falling back.
"""
from __future__ import annotations

import numpy as np

from . import _lib as L
from .cache import PagedQuantizedKVCache


def _torch():
    import torch

    return torch


def _batch(caches):
    """(pool, layer) shared by every cache of a batch."""
    if not caches:
        raise ValueError("empty batch")
    pool, layer = caches[0].s.pool, caches[0].layer
    for c in caches:
        if not isinstance(c, PagedQuantizedKVCache):
            raise TypeError("caches must be PagedQuantizedKVCache")
        if c.s.pool is not pool or c.layer != layer:
            raise ValueError("every cache of a batch must be the same layer of one pool")
    if len({c.s.seq for c in caches}) != len(caches):
        raise ValueError("a sequence appears twice in the batch")
    return pool, layer


def _tables(pool, caches, device, extra: int = 0):
    """Block tables [B, max_blocks] and this layer's lengths (+ `extra`) [B]
    on `device`.  The table width covers every block the sequences hold: a
    layer may be behind its sequence (restored or appended one layer at a
    time), and the tables carry the whole sequence."""
    torch = _torch()
    lens = np.array([c.sequence_length + extra for c in caches], np.int32)
    mb = max(1, int(max((int(c.s.length) + 63) // 64 for c in caches)), int(max((int(n) + 63) // 64 for n in lens)))
    t, _ = pool.batch_tables([c.s.seq for c in caches], mb)
    return (torch.as_tensor(np.ascontiguousarray(t), device=device),
            torch.as_tensor(lens, device=device), int(lens.max()) if lens.size else 0)


class KrillKernels:
    @staticmethod
    def is_available() -> bool:
        """True when libkrillhip loads and a HIP device is visible."""
        try:
            L.lib()
        except L.KrillLibraryError:
            return False
        return bool(_torch().cuda.is_available())

    @staticmethod
    def status() -> str:
        try:
            L.lib()
        except L.KrillLibraryError as e:
            return f"libkrillhip unavailable: {e}"
        torch = _torch()
        if not torch.cuda.is_available():
            return "libkrillhip loaded; no HIP device visible"
        return f"libkrillhip ABI {L.lib().krill_abi_version()} on {torch.cuda.get_device_name(0)}"

    @staticmethod
    def quantize_append(caches, keys, values):
        """update() of every cache of the batch in one launch: keys / values
        [B, Hkv, L, D] in the pool's input dtype, row b appended to caches[b]
        (QuantizedKVCache.swift:49-75 without the dequantized return)."""
        torch = _torch()
        pool, layer = _batch(caches)
        B, L_ = int(keys.shape[0]), int(keys.shape[2])
        if B != len(caches) or tuple(values.shape) != tuple(keys.shape):
            raise ValueError("keys/values must be [len(caches), Hkv, L, D]")
        try:
            slots = np.stack([c.s.slots_for(layer, L_) for c in caches]).astype(np.int32)
            pool.quantize_append(layer, keys.contiguous(), values.contiguous(),
                                 torch.as_tensor(slots, device=keys.device))
        except BaseException:
            # nothing was appended: release what the reservation added
            for c in caches:
                c.s.shrink_to_layers()
            raise
        for c in caches:
            c.s.layer_len[layer] += L_

    @staticmethod
    def paged_decode_attention(queries, caches, scale: float, keys=None, values=None, out_dtype=None):
        """Decode attention of queries [B, Hq, 1, D] over each sequence's
        cache of this layer.  With keys / values ([B, Hkv, 1, D]) the step's
        new token is appended first, in the same launch (the update + SDPA of
        a decode step)."""
        pool, layer = _batch(caches)
        if queries.shape[0] != len(caches) or queries.shape[2] != 1:
            raise ValueError("queries must be [len(caches), Hq, 1, D]")
        if (keys is None) != (values is None):
            raise ValueError("keys and values come together")
        if keys is None:
            tables, lens, max_len = _tables(pool, caches, queries.device)
            return pool.attention(layer, queries, tables, lens, max_len, scale, out_dtype)
        want = (len(caches), pool.num_kv_heads, 1, pool.head_dim)
        if tuple(keys.shape) != want or tuple(values.shape) != want:
            raise ValueError(f"keys/values must be {list(want)}")
        # The caches change only once the launch is accepted: the slots are
        # reserved first (the kernel writes position len - 1 of each table),
        # and released again if the call fails.
        try:
            for c in caches:
                c.s.slots_for(layer, 1)
            tables, lens, max_len = _tables(pool, caches, queries.device, extra=1)
            out = pool.decode_append_attention(layer, queries, keys, values, tables, lens, max_len, scale,
                                               out_dtype)
        except BaseException:
            for c in caches:
                c.s.shrink_to_layers()
            raise
        for c in caches:
            c.s.layer_len[layer] += 1
        return out

    @staticmethod
    def paged_verify_attention(queries, caches, scale: float, out_dtype=None):
        """Speculative-verify / chunked-prefill attention: queries [B, Hq, Lq,
        D] are the last Lq cached positions of each sequence (already
        appended), causal inside that window (BatchedDecode.swift:299-312)."""
        pool, layer = _batch(caches)
        Lq = int(queries.shape[2])
        if queries.shape[0] != len(caches):
            raise ValueError("queries must be [len(caches), Hq, Lq, D]")
        if any(c.sequence_length < Lq for c in caches):
            raise ValueError("every sequence must hold its Lq query positions")
        tables, lens, max_len = _tables(pool, caches, queries.device)
        return pool.attention(layer, queries, tables, lens, max_len, scale, out_dtype)

    @staticmethod
    def stacked_quantized(caches, left_pad: bool = True):
        """stackCachesLeftPaddedQuantized (BatchedDecode.swift:96-151): the
        batch's quantized snapshot [B, Hkv, S_max, ...], shorter sequences
        left-padded with zero bytes."""
        pool, layer = _batch(caches)
        tables, lens, max_len = _tables(pool, caches, "cuda")
        return pool.gather(layer, tables, lens, max(max_len, 1), left_pad=left_pad)

    @staticmethod
    def copy_blocks(pool, src_dst):
        """Whole-block copies in every layer (int32 [n, 2] device pairs)."""
        pool.copy_blocks(src_dst)
