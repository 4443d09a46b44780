"""KrillKernels: static entry points of the paged int8 KV kernels.

Mirrors the static-enum registry of Sources/KrillKernels/KernelRegistry.swift
:13-162 (``isAvailable`` / ``status`` plus one static function per kernel).
Each function is a direct call into libkrillhip; a missing library or device
raises instead of falling back.
"""
from __future__ import annotations

from . import _lib as L
from .pool import KVPool


class KrillKernels:
    @staticmethod
    def is_available() -> bool:
        """True when libkrillhip loads and a HIP device is visible."""
        try:
            L.lib()
        except L.KrillLibraryError:
            return False
        import torch

        return bool(torch.cuda.is_available())

    @staticmethod
    def status() -> str:
        try:
            L.lib()
        except L.KrillLibraryError as e:
            return f"libkrillhip unavailable: {e}"
        import torch

        if not torch.cuda.is_available():
            return "libkrillhip loaded; no HIP device visible"
        return f"libkrillhip ABI {L.lib().krill_abi_version()} on {torch.cuda.get_device_name(0)}"

    @staticmethod
    def quantize_append(pool: KVPool, layer: int, keys, values, slot_mapping):
        pool.quantize_append(layer, keys, values, slot_mapping)

    @staticmethod
    def paged_decode_attention(pool: KVPool, layer: int, queries, block_tables, seq_lens, max_seq_len: int,
                               scale: float, out_dtype=None, workspace=None, out=None):
        if queries.shape[2] != 1:
            raise ValueError("decode attention takes one query row per head ([B, Hq, 1, D])")
        return pool.attention(layer, queries, block_tables, seq_lens, max_seq_len, scale, out_dtype, workspace, out)

    @staticmethod
    def paged_verify_attention(pool: KVPool, layer: int, queries, block_tables, seq_lens, max_seq_len: int,
                               scale: float, out_dtype=None, workspace=None, out=None):
        return pool.attention(layer, queries, block_tables, seq_lens, max_seq_len, scale, out_dtype, workspace, out)

    @staticmethod
    def gather(pool: KVPool, layer: int, block_tables, seq_lens, s_out: int, left_pad: bool = False):
        return pool.gather(layer, block_tables, seq_lens, s_out, left_pad)

    @staticmethod
    def copy_blocks(pool: KVPool, src_dst):
        pool.copy_blocks(src_dst)
