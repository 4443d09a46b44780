"""Python face of one libkrillhip pool: the block manager plus the gfx950
kernels, with PyTorch tensors as device memory and torch's current stream as
the HIP stream.  Thin by design: every call goes straight through the C ABI
(include/libkrillhip.h); nothing here computes KV data on the host.
"""
from __future__ import annotations

import ctypes

import numpy as np

from . import _lib as L

QUANT_MODES = {"ref_row": L.QUANT_REF_ROW, "affine_g64": L.QUANT_AFFINE_G64}


def _torch():
    import torch

    return torch


def _dtype_code(dt) -> int:
    torch = _torch()
    if dt in ("bf16", torch.bfloat16):
        return L.DTYPE_BF16
    if dt in ("f16", torch.float16):
        return L.DTYPE_F16
    if dt in ("f32", torch.float32):
        return L.DTYPE_F32
    raise ValueError(f"unsupported dtype {dt!r}")


def _torch_dtype(code: int):
    torch = _torch()
    return {L.DTYPE_BF16: torch.bfloat16, L.DTYPE_F16: torch.float16, L.DTYPE_F32: torch.float32}[code]


def _i32p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int32))


def _i64p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))


def _enc(s):
    return None if s is None else s.encode()


class KVPool:
    """Paged int8 KV pool: `num_blocks` 64-token blocks for every layer and KV head.

    quant_mode "ref_row" stores the reference's per-(token, head) min/max rows
    (QuantizedKVCache.swift:181-197); "affine_g64" stores affine 8-bit groups
    of 64 with fp16 scale/bias.  in_dtype is the dtype of the K/V/Q tensors
    handed to the kernels (bf16 or f16).  host_only pools run the block
    manager without device memory (kernels are refused).
    """

    def __init__(self, num_layers: int, num_kv_heads: int, head_dim: int, num_blocks: int,
                 quant_mode: str = "affine_g64", in_dtype="bf16", *, host_only: bool = False,
                 stream=None, evict_watermark: float = 0.0, max_prefix_entries: int = 0,
                 min_prefix_len: int = 0, max_entry_bytes: int = -1, free_list_seed: int = 0):
        self.num_layers = num_layers
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.num_blocks = num_blocks
        self.quant_mode = quant_mode
        self.mode = QUANT_MODES[quant_mode]
        self.in_dtype_code = _dtype_code(in_dtype)
        self.groups = head_dim // 64 if self.mode == L.QUANT_AFFINE_G64 else 1
        self.host_only = host_only
        desc = L.PoolDesc(num_layers, num_kv_heads, head_dim, 64, num_blocks, self.mode,
                          self.in_dtype_code, L.POOL_HOST_ONLY if host_only else 0,
                          float(evict_watermark), int(max_prefix_entries), int(min_prefix_len),
                          int(max_entry_bytes), int(free_list_seed))
        self._h = ctypes.c_void_p()
        st = ctypes.c_void_p(stream) if stream else None
        L.check(L.lib().krill_pool_create(ctypes.byref(desc), st, ctypes.byref(self._h)))

    # ------------------------------------------------------------ lifetime
    def close(self):
        if getattr(self, "_h", None) and self._h.value:
            L.check(L.lib().krill_pool_destroy(self._h))
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def handle(self):
        return self._h

    # ------------------------------------------------------------- pool
    def stats(self) -> dict:
        s = L.PoolStats()
        L.check(L.lib().krill_pool_get_stats(self._h, ctypes.byref(s)))
        return s.as_dict()

    def refcounts(self) -> np.ndarray:
        out = np.empty(self.num_blocks, np.int32)
        L.check(L.lib().krill_pool_refcounts(self._h, _i32p(out), self.num_blocks))
        return out

    def set_option(self, option: int, value: int):
        L.check(L.lib().krill_pool_set_option(self._h, option, int(value)))

    def flush(self, stream=None):
        L.check(L.lib().krill_pool_flush(self._h, self._stream(stream)))

    # -------------------------------------------------------- sequences
    def seq_create(self) -> int:
        out = ctypes.c_int32()
        L.check(L.lib().krill_seq_create(self._h, ctypes.byref(out)))
        return out.value

    def seq_fork(self, src: int, n_tokens: int) -> int:
        out = ctypes.c_int32()
        L.check(L.lib().krill_seq_fork(self._h, src, n_tokens, ctypes.byref(out)))
        return out.value

    def seq_free(self, seq: int):
        L.check(L.lib().krill_seq_free(self._h, seq))

    def seq_reset(self, seq: int):
        L.check(L.lib().krill_seq_reset(self._h, seq))

    def seq_length(self, seq: int) -> int:
        out = ctypes.c_int32()
        L.check(L.lib().krill_seq_length(self._h, seq, ctypes.byref(out)))
        return out.value

    def seq_memory_bytes(self, seq: int) -> int:
        out = ctypes.c_int64()
        L.check(L.lib().krill_seq_memory_bytes(self._h, seq, ctypes.byref(out)))
        return out.value

    def seq_truncate(self, seq: int, n: int):
        L.check(L.lib().krill_seq_truncate(self._h, seq, n))

    def reserve_append(self, seq: int, n: int) -> np.ndarray:
        slots = np.empty(max(n, 1), np.int32)
        L.check(L.lib().krill_seq_reserve_append(self._h, seq, n, _i32p(slots)))
        return slots[:n]

    def block_table(self, seq: int) -> np.ndarray:
        n = ctypes.c_int32()
        cap = (self.seq_length(seq) + 63) // 64 + 1
        out = np.empty(max(cap, 1), np.int32)
        L.check(L.lib().krill_seq_block_table(self._h, seq, _i32p(out), cap, ctypes.byref(n)))
        return out[: n.value].copy()

    def batch_tables(self, seqs, max_blocks: int):
        seqs = np.ascontiguousarray(seqs, np.int32)
        B = seqs.size
        tables = np.zeros((max(B, 1), max(max_blocks, 1)), np.int32)
        lens = np.zeros(max(B, 1), np.int32)
        L.check(L.lib().krill_batch_tables(self._h, _i32p(seqs), B, max_blocks, _i32p(tables), _i32p(lens)))
        return tables[:B, :max_blocks], lens[:B]

    def batch_starts(self, seqs) -> np.ndarray:
        """First retained token of each sequence (sliding-window pools)."""
        seqs = np.ascontiguousarray(seqs, np.int32)
        out = np.zeros(max(seqs.size, 1), np.int32)
        L.check(L.lib().krill_batch_starts(self._h, _i32p(seqs), seqs.size, _i32p(out)))
        return out[: seqs.size]

    # ---------------------------------------------------------- prefix
    def prefix_store(self, seq: int, tokens, model_id: str = "", media_hash=None) -> bool:
        t = np.ascontiguousarray(tokens, np.int64)
        stored = ctypes.c_int32()
        tp = _i64p(t) if t.size else None
        L.check(L.lib().krill_prefix_store(self._h, seq, _enc(model_id), _enc(media_hash), tp, t.size,
                                           ctypes.byref(stored)))
        return bool(stored.value)

    def _lookup(self, fn, tokens, model_id, media_hash):
        t = np.ascontiguousarray(tokens, np.int64)
        plen, ent = ctypes.c_int32(), ctypes.c_int32()
        tp = _i64p(t) if t.size else None
        L.check(fn(self._h, _enc(model_id), _enc(media_hash), tp, t.size, ctypes.byref(plen), ctypes.byref(ent)))
        return plen.value, (ent.value if ent.value >= 0 else None)

    def prefix_lookup(self, tokens, model_id: str = "", media_hash=None):
        """Exact-entry scan (PrefixCache.lookupQuantized): (prefix_len, entry_seq)."""
        return self._lookup(L.lib().krill_prefix_lookup, tokens, model_id, media_hash)

    def prefix_probe(self, tokens, model_id: str = "", media_hash=None):
        """Entry sequence keyed by exactly `tokens`, or None (one step of the
        exact scan, PrefixCache.swift:294-298; touched on a hit)."""
        t = np.ascontiguousarray(tokens, np.int64)
        ent = ctypes.c_int32()
        tp = _i64p(t) if t.size else None
        L.check(L.lib().krill_prefix_probe(self._h, _enc(model_id), _enc(media_hash), tp, t.size, ctypes.byref(ent)))
        return ent.value if ent.value >= 0 else None

    def prefix_lookup_longest(self, tokens, model_id: str = "", media_hash=None):
        """Longest common prefix (PrefixCache.lookupLongestPrefixQuantized)."""
        return self._lookup(L.lib().krill_prefix_lookup_longest, tokens, model_id, media_hash)

    def prefix_clear(self):
        L.check(L.lib().krill_prefix_clear(self._h))

    def prefix_count(self) -> int:
        out = ctypes.c_int32()
        L.check(L.lib().krill_prefix_count(self._h, ctypes.byref(out)))
        return out.value

    # ---------------------------------------------------------- kernels
    @staticmethod
    def _stream(stream=None):
        """hipStream_t for a torch stream, a raw handle (int) or None (torch's current stream)."""
        if stream is not None:
            return ctypes.c_void_p(getattr(stream, "cuda_stream", stream))
        torch = _torch()
        if torch.cuda.is_available():
            return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        return None

    def _check_dev(self, name, t, dtype=None, shape=None):
        torch = _torch()
        if not isinstance(t, torch.Tensor) or not t.is_cuda:
            raise ValueError(f"{name} must be a CUDA (HIP) tensor")
        if not t.is_contiguous():
            raise ValueError(f"{name} must be contiguous")
        if dtype is not None and t.dtype != dtype:
            raise ValueError(f"{name} has dtype {t.dtype}, expected {dtype}")
        if shape is not None and tuple(t.shape) != tuple(shape):
            raise ValueError(f"{name} has shape {tuple(t.shape)}, expected {tuple(shape)}")

    @property
    def in_dtype(self):
        return _torch_dtype(self.in_dtype_code)

    def quantize_append(self, layer: int, k, v, slot_mapping, stream=None):
        """k, v: [B, Hkv, L, D] in in_dtype; slot_mapping: int32 [B, L] (device)."""
        torch = _torch()
        B, H, Lq, D = k.shape
        if H != self.num_kv_heads or D != self.head_dim:
            raise ValueError(f"K/V shape {tuple(k.shape)} does not match pool heads/dim")
        self._check_dev("k", k, self.in_dtype)
        self._check_dev("v", v, self.in_dtype, k.shape)
        self._check_dev("slot_mapping", slot_mapping, torch.int32, (B, Lq))
        L.check(L.lib().krill_quantize_append(self._h, layer, k.data_ptr(), v.data_ptr(), slot_mapping.data_ptr(),
                                              B, Lq, self._stream(stream)))

    def quantize_append_rope(self, layer: int, k, v, slot_mapping, positions, cos_sin, stream=None):
        """quantize_append with K rotated first (krill_quantize_append_rope):
        positions int32 [B, L], cos_sin float32 [max_pos, D] (see rope_table)."""
        torch = _torch()
        B, H, Lq, D = k.shape
        if H != self.num_kv_heads or D != self.head_dim:
            raise ValueError(f"K/V shape {tuple(k.shape)} does not match pool heads/dim")
        self._check_dev("k", k, self.in_dtype)
        self._check_dev("v", v, self.in_dtype, k.shape)
        self._check_dev("slot_mapping", slot_mapping, torch.int32, (B, Lq))
        self._check_dev("positions", positions, torch.int32, (B, Lq))
        self._check_dev("cos_sin", cos_sin, torch.float32)
        if cos_sin.dim() != 2 or cos_sin.shape[1] != D:
            raise ValueError(f"cos_sin must be [max_pos, {D}]")
        L.check(L.lib().krill_quantize_append_rope(self._h, layer, k.data_ptr(), v.data_ptr(), H * Lq * D, Lq * D, D,
                                                   slot_mapping.data_ptr(), positions.data_ptr(), cos_sin.data_ptr(),
                                                   cos_sin.shape[0], B, Lq, self._stream(stream)))

    def quantize_append_strided(self, layer: int, k, v, strides, slot_mapping, B: int, Lq: int, stream=None):
        """k, v: device tensors addressed with element strides (b, h, l), d contiguous."""
        torch = _torch()
        self._check_dev("slot_mapping", slot_mapping, torch.int32, (B, Lq))
        sb, sh, sl = (int(s) for s in strides)
        L.check(L.lib().krill_quantize_append_strided(self._h, layer, k.data_ptr(), v.data_ptr(), sb, sh, sl,
                                                      slot_mapping.data_ptr(), B, Lq, self._stream(stream)))

    def _tables(self, tables, lens):
        torch = _torch()
        self._check_dev("block_tables", tables, torch.int32)
        self._check_dev("seq_lens", lens, torch.int32)
        if tables.dim() != 2 or lens.dim() != 1 or tables.shape[0] != lens.shape[0]:
            raise ValueError("block_tables must be [B, max_blocks] and seq_lens [B]")
        return tables.shape[0], tables.shape[1]

    def gather(self, layer: int, tables, lens, S_out: int, left_pad: bool = False, stream=None) -> dict:
        """Paged -> snapshot dict of keys/values u8 [B,H,S,D] and scales/zeros f16 [B,H,S,G]."""
        torch = _torch()
        B, mb = self._tables(tables, lens)
        H, D, G = self.num_kv_heads, self.head_dim, self.groups
        dev = tables.device
        snap = {
            "keys": torch.empty((B, H, S_out, D), dtype=torch.uint8, device=dev),
            "values": torch.empty((B, H, S_out, D), dtype=torch.uint8, device=dev),
            "key_scales": torch.empty((B, H, S_out, G), dtype=torch.float16, device=dev),
            "key_zeros": torch.empty((B, H, S_out, G), dtype=torch.float16, device=dev),
            "value_scales": torch.empty((B, H, S_out, G), dtype=torch.float16, device=dev),
            "value_zeros": torch.empty((B, H, S_out, G), dtype=torch.float16, device=dev),
        }
        s = L.Snapshot(*(snap[n].data_ptr() for n in
                         ("keys", "values", "key_scales", "key_zeros", "value_scales", "value_zeros")))
        L.check(L.lib().krill_gather(self._h, layer, tables.data_ptr(), lens.data_ptr(), B, mb, S_out,
                                     1 if left_pad else 0, ctypes.byref(s), self._stream(stream)))
        return snap

    def gather_dequant(self, layer: int, tables, lens, S_out: int, left_pad: bool = False, stream=None):
        torch = _torch()
        B, mb = self._tables(tables, lens)
        shape = (B, self.num_kv_heads, S_out, self.head_dim)
        k = torch.empty(shape, dtype=torch.float16, device=tables.device)
        v = torch.empty(shape, dtype=torch.float16, device=tables.device)
        L.check(L.lib().krill_gather_dequant(self._h, layer, tables.data_ptr(), lens.data_ptr(), B, mb, S_out,
                                             1 if left_pad else 0, k.data_ptr(), v.data_ptr(),
                                             self._stream(stream)))
        return k, v

    def scatter(self, layer: int, snap: dict, src_start, slot_mapping, stream=None):
        """Copy snapshot rows [src_start[b], +L) into slot_mapping[b] (both int32 device)."""
        torch = _torch()
        B, H, S_in, D = snap["keys"].shape
        G = self.groups
        for n in ("keys", "values"):
            self._check_dev(n, snap[n], torch.uint8, (B, H, S_in, D))
        for n in ("key_scales", "key_zeros", "value_scales", "value_zeros"):
            self._check_dev(n, snap[n], torch.float16, (B, H, S_in, G))
        self._check_dev("src_start", src_start, torch.int32, (B,))
        self._check_dev("slot_mapping", slot_mapping, torch.int32)
        Lq = slot_mapping.shape[1]
        s = L.Snapshot(*(snap[n].data_ptr() for n in
                         ("keys", "values", "key_scales", "key_zeros", "value_scales", "value_zeros")))
        L.check(L.lib().krill_scatter(self._h, layer, ctypes.byref(s), B, S_in, src_start.data_ptr(),
                                      slot_mapping.data_ptr(), Lq, self._stream(stream)))

    def copy_blocks(self, src_dst, stream=None):
        torch = _torch()
        self._check_dev("src_dst", src_dst, torch.int32)
        L.check(L.lib().krill_copy_blocks(self._h, src_dst.data_ptr(), src_dst.numel() // 2, self._stream(stream)))

    def workspace_size(self, B: int, Hq: int, Lq: int, max_seq_len: int) -> int:
        out = ctypes.c_size_t()
        L.check(L.lib().krill_attention_workspace_size(self._h, B, Hq, Lq, max_seq_len, ctypes.byref(out)))
        return out.value

    def shared_prefix_workspace_size(self, B: int, Hq: int, prefix_blocks: int, max_suffix_len: int) -> int:
        out = ctypes.c_size_t()
        L.check(L.lib().krill_shared_prefix_workspace_size(self._h, B, Hq, prefix_blocks, max_suffix_len,
                                                           ctypes.byref(out)))
        return out.value

    def attention(self, layer: int, q, tables, lens, max_seq_len: int, scale: float, out_dtype=None,
                  ws=None, out=None, stream=None):
        """q: [B, Hq, Lq, D] in in_dtype.  Lq == 1 is decode, Lq > 1 verify/chunked prefill."""
        torch = _torch()
        B, Hq, Lq, D = q.shape
        self._check_dev("q", q, self.in_dtype)
        Bt, mb = self._tables(tables, lens)
        if Bt != B or D != self.head_dim:
            raise ValueError("q batch/head_dim does not match the tables/pool")
        out_dtype = torch.float32 if out_dtype is None else out_dtype
        code = _dtype_code(out_dtype)
        if out is None:
            out = torch.empty((B, Hq, Lq, D), dtype=out_dtype, device=q.device)
        else:
            self._check_dev("out", out, out_dtype, (B, Hq, Lq, D))
        need = self.workspace_size(B, Hq, Lq, max_seq_len)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        st = self._stream(stream)
        if Lq == 1:
            L.check(L.lib().krill_decode_attention(self._h, layer, q.data_ptr(), tables.data_ptr(), lens.data_ptr(),
                                                   B, mb, max_seq_len, Hq, float(scale), out.data_ptr(), code,
                                                   ws.data_ptr(), ws.numel(), st))
        else:
            L.check(L.lib().krill_verify_attention(self._h, layer, q.data_ptr(), Lq, tables.data_ptr(),
                                                   lens.data_ptr(), B, mb, max_seq_len, Hq, float(scale),
                                                   out.data_ptr(), code, ws.data_ptr(), ws.numel(), st))
        return out

    def attention_windowed(self, layer: int, q, tables, lens, starts, window: int, max_seq_len: int, scale: float,
                           out_dtype=None, ws=None, out=None, stream=None):
        """Sliding-window attention: row j of sequence b (position p = lens[b] -
        Lq + j) sees keys [max(starts[b], p - window + 1), p]; starts (int32
        [B] device, or None for 0) from batch_starts."""
        torch = _torch()
        B, Hq, Lq, D = q.shape
        self._check_dev("q", q, self.in_dtype)
        Bt, mb = self._tables(tables, lens)
        if Bt != B or D != self.head_dim:
            raise ValueError("q batch/head_dim does not match the tables/pool")
        if starts is not None:
            self._check_dev("starts", starts, torch.int32, (B,))
        out_dtype = torch.float32 if out_dtype is None else out_dtype
        code = _dtype_code(out_dtype)
        if out is None:
            out = torch.empty((B, Hq, Lq, D), dtype=out_dtype, device=q.device)
        else:
            self._check_dev("out", out, out_dtype, (B, Hq, Lq, D))
        need = ctypes.c_size_t()
        L.check(L.lib().krill_window_workspace_size(self._h, B, Hq, Lq, mb, max_seq_len, window, ctypes.byref(need)))
        if ws is None or ws.numel() < need.value:
            ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=q.device)
        L.check(L.lib().krill_attention_windowed(
            self._h, layer, q.data_ptr(), Lq, tables.data_ptr(), lens.data_ptr(),
            starts.data_ptr() if starts is not None else None, window, B, mb, max_seq_len, Hq, float(scale),
            out.data_ptr(), code, ws.data_ptr(), ws.numel(), self._stream(stream)))
        return out

    def decode_append_attention_windowed(self, layer: int, q, k_new, v_new, tables, lens, starts, window: int,
                                         max_seq_len: int, scale: float, cos_sin=None, out_dtype=None, ws=None,
                                         out=None, stream=None):
        """The sliding layers' decode step in one launch: each sequence's newest
        token (k_new / v_new [B, Hkv, 1, D], in_dtype) written at position
        lens[b] - 1, then windowed attention of q [B, Hq, 1, D]; with cos_sin
        (float32 [max_pos, D]) queries and new K rows turn by that position
        first.  Same output and pool bytes as quantize_append(_rope) at the
        reserved slots followed by attention_windowed."""
        torch = _torch()
        B, Hq, Lq, D = q.shape
        if Lq != 1:
            raise ValueError("the windowed decode step takes one query row per sequence")
        self._check_dev("q", q, self.in_dtype)
        Bt, mb = self._tables(tables, lens)
        if Bt != B or D != self.head_dim:
            raise ValueError("q batch/head_dim does not match the tables/pool")
        H = self.num_kv_heads
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            self._check_dev(name, t, self.in_dtype)
            if t.numel() != B * H * D or t.shape[0] != B or t.shape[1] != H:
                raise ValueError(f"{name} has shape {tuple(t.shape)}, expected [{B}, {H}, (1,) {D}]")
        if starts is not None:
            self._check_dev("starts", starts, torch.int32, (B,))
        if cos_sin is not None:
            self._check_dev("cos_sin", cos_sin, torch.float32)
            if cos_sin.dim() != 2 or cos_sin.shape[1] != D:
                raise ValueError(f"cos_sin must be [max_pos, {D}]")
        out_dtype = torch.float32 if out_dtype is None else out_dtype
        code = _dtype_code(out_dtype)
        if out is None:
            out = torch.empty((B, Hq, 1, D), dtype=out_dtype, device=q.device)
        else:
            self._check_dev("out", out, out_dtype, (B, Hq, 1, D))
        need = ctypes.c_size_t()
        L.check(L.lib().krill_window_workspace_size(self._h, B, Hq, 1, mb, max_seq_len, window, ctypes.byref(need)))
        if ws is None or ws.numel() < need.value:
            ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=q.device)
        L.check(L.lib().krill_decode_append_attention_windowed(
            self._h, layer, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), H * D, D, tables.data_ptr(),
            lens.data_ptr(), starts.data_ptr() if starts is not None else None, window, B, mb, max_seq_len, Hq,
            float(scale), cos_sin.data_ptr() if cos_sin is not None else None,
            int(cos_sin.shape[0]) if cos_sin is not None else 0, out.data_ptr(), code, ws.data_ptr(), ws.numel(),
            self._stream(stream)))
        return out

    def attention_shared_prefix(self, layer: int, q, prefix_table, suffix_tables, suffix_lens, max_suffix_len: int,
                                scale: float, out_dtype=None, ws=None, out=None, stream=None, k_new=None,
                                v_new=None):
        """Decode attention of B sequences sharing the blocks prefix_table (int32
        [P] device) before their own suffix blocks (suffix_tables [B, mb],
        suffix_lens [B], tokens after the 64 P prefix tokens).  With k_new /
        v_new ([B, Hkv, 1, D]) the step's new token is appended in the same
        launches at suffix position suffix_lens[b] - 1."""
        torch = _torch()
        B, Hq, Lq, D = q.shape
        if Lq != 1 or D != self.head_dim:
            raise ValueError("q must be [B, Hq, 1, head_dim]")
        self._check_dev("q", q, self.in_dtype)
        self._check_dev("prefix_table", prefix_table, torch.int32)
        Bt, mb = self._tables(suffix_tables, suffix_lens)
        if Bt != B:
            raise ValueError("q batch does not match the suffix tables")
        P = int(prefix_table.numel())
        out_dtype = torch.float32 if out_dtype is None else out_dtype
        code = _dtype_code(out_dtype)
        if out is None:
            out = torch.empty((B, Hq, 1, D), dtype=out_dtype, device=q.device)
        else:
            self._check_dev("out", out, out_dtype, (B, Hq, 1, D))
        need = ctypes.c_size_t()
        L.check(L.lib().krill_shared_prefix_workspace_size(self._h, B, Hq, P, max_suffix_len, ctypes.byref(need)))
        if ws is None or ws.numel() < need.value:
            ws = torch.empty(max(need.value, 1), dtype=torch.uint8, device=q.device)
        if k_new is None:
            L.check(L.lib().krill_decode_attention_shared_prefix(
                self._h, layer, q.data_ptr(), prefix_table.data_ptr(), P, suffix_tables.data_ptr(),
                suffix_lens.data_ptr(), B, mb, max_suffix_len, Hq, float(scale), out.data_ptr(), code, ws.data_ptr(),
                ws.numel(), self._stream(stream)))
            return out
        H = self.num_kv_heads
        self._check_dev("k_new", k_new, self.in_dtype, (B, H, 1, D))
        self._check_dev("v_new", v_new, self.in_dtype, (B, H, 1, D))
        L.check(L.lib().krill_decode_append_attention_shared_prefix(
            self._h, layer, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), H * D, D, prefix_table.data_ptr(), P,
            suffix_tables.data_ptr(), suffix_lens.data_ptr(), B, mb, max_suffix_len, Hq, float(scale),
            out.data_ptr(), code, ws.data_ptr(), ws.numel(), self._stream(stream)))
        return out

    def decode_append_attention_rope(self, layer: int, q, k_new, v_new, tables, lens, max_seq_len: int,
                                     scale: float, cos_sin, out_dtype=None, ws=None, out=None, stream=None):
        """decode_append_attention with the queries and new K rows unrotated:
        both turn by the new token's position lens[b] - 1 (cos_sin: float32
        [max_pos, D], max_pos >= max_seq_len; see rope_table)."""
        return self._decode_append(layer, q, k_new, v_new, tables, lens, max_seq_len, scale, out_dtype, ws, out,
                                   stream, cos_sin)

    def decode_append_attention(self, layer: int, q, k_new, v_new, tables, lens, max_seq_len: int, scale: float,
                                out_dtype=None, ws=None, out=None, stream=None):
        return self._decode_append(layer, q, k_new, v_new, tables, lens, max_seq_len, scale, out_dtype, ws, out,
                                   stream, None)

    def _decode_append(self, layer, q, k_new, v_new, tables, lens, max_seq_len, scale, out_dtype, ws, out, stream,
                       cos_sin):
        """Decode step with the append fused: writes each sequence's newest token
        (k_new, v_new: [B, Hkv, 1, D] or [B, Hkv, D] in in_dtype) at position
        lens[b] - 1, then attends q [B, Hq, 1, D] over the cache.  Same pool bytes
        and output as quantize_append at those slots followed by attention."""
        torch = _torch()
        B, Hq, Lq, D = q.shape
        if Lq != 1:
            raise ValueError("decode_append_attention takes one query row per sequence")
        self._check_dev("q", q, self.in_dtype)
        Bt, mb = self._tables(tables, lens)
        if Bt != B or D != self.head_dim:
            raise ValueError("q batch/head_dim does not match the tables/pool")
        H = self.num_kv_heads
        for name, t in (("k_new", k_new), ("v_new", v_new)):
            self._check_dev(name, t, self.in_dtype)
            if t.numel() != B * H * D or t.shape[0] != B or t.shape[1] != H:
                raise ValueError(f"{name} has shape {tuple(t.shape)}, expected [{B}, {H}, (1,) {D}]")
        out_dtype = torch.float32 if out_dtype is None else out_dtype
        code = _dtype_code(out_dtype)
        if out is None:
            out = torch.empty((B, Hq, 1, D), dtype=out_dtype, device=q.device)
        else:
            self._check_dev("out", out, out_dtype, (B, Hq, 1, D))
        need = self.workspace_size(B, Hq, 1, max_seq_len)
        if ws is None or ws.numel() < need:
            ws = torch.empty(max(need, 1), dtype=torch.uint8, device=q.device)
        if cos_sin is None:
            L.check(L.lib().krill_decode_append_attention(
                self._h, layer, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), H * D, D, tables.data_ptr(),
                lens.data_ptr(), B, mb, max_seq_len, Hq, float(scale), out.data_ptr(), code, ws.data_ptr(),
                ws.numel(), self._stream(stream)))
        else:
            self._check_dev("cos_sin", cos_sin, torch.float32)
            if cos_sin.dim() != 2 or cos_sin.shape[1] != D:
                raise ValueError(f"cos_sin must be [max_pos, {D}]")
            L.check(L.lib().krill_decode_append_attention_rope(
                self._h, layer, q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), H * D, D, tables.data_ptr(),
                lens.data_ptr(), B, mb, max_seq_len, Hq, float(scale), cos_sin.data_ptr(), cos_sin.shape[0],
                out.data_ptr(), code, ws.data_ptr(), ws.numel(), self._stream(stream)))
        return out


def rope_table(max_pos: int, head_dim: int, base: float = 10000.0) -> np.ndarray:
    """float32 [max_pos, head_dim] cos/sin table for krill_quantize_append_rope:
    row p holds cos(p * base^(-2i/D)) for i < D/2, then the sines, computed
    in double precision and rounded once (MLX RoPE angles, traditional = false)."""
    half = head_dim // 2
    inv = base ** (-2.0 * np.arange(half, dtype=np.float64) / head_dim)
    ang = np.arange(max_pos, dtype=np.float64)[:, None] * inv[None, :]
    return np.concatenate([np.cos(ang), np.sin(ang)], axis=1).astype(np.float32)


def prefix_key(model_id: str, media_hash, dtype_tag: int, tokens) -> int:
    """PrefixCache.cacheKey (PrefixCache.swift:511-532) as computed by the library."""
    t = np.ascontiguousarray(tokens, np.int64)
    out = ctypes.c_uint64()
    L.check(L.lib().krill_prefix_key(_enc(model_id), _enc(media_hash), dtype_tag, _i64p(t) if t.size else None,
                                     t.size, ctypes.byref(out)))
    return out.value
