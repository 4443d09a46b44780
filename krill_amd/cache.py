"""Reference-shaped cache API over a KVPool.

Mirrors the Swift surfaces the Krill batcher calls, with the reference's
names and argument meaning:

* ``QuantizedKVSnapshot``      Sources/KrillCache/QuantizedKVCache.swift:150-173
* ``PagedQuantizedKVCache``    QuantizedKVCache (QuantizedKVCache.swift:17-146):
  update / snapshot / reset / sequence_length / memory_size_bytes /
  quantized_snapshot / restore_quantized / truncate
* ``make_quantized_kv_caches`` makeQuantizedKVCaches (QuantizedKVCache.swift:207-210)
* ``PrefixCache``              the int8 half of PrefixCache
  (PrefixCache.swift:161-308, :369-400, :511-551)

The caches of one sequence share one block table, so all layers of a
sequence address the same token positions (each layer has its own bytes at
each position): the sequence reserves positions up to the longest layer,
a layer appends at its own length, truncate / reset apply to the whole
sequence (the engine always does these to every layer together,
InferenceEngine.swift:1402-1417), and restore_quantized replaces one layer's
contents, as the reference's does.
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .pool import KVPool


def _torch():
    import torch

    return torch


@dataclass
class QuantizedKVSnapshot:
    """Six tensors of one layer: u8 keys/values [B,H,S,D], f16 scales/zeros [B,H,S,G]."""

    keys: object
    values: object
    key_scales: object
    key_zeros: object
    value_scales: object
    value_zeros: object

    @property
    def sequence_length(self) -> int:
        return int(self.keys.shape[2])

    @classmethod
    def from_dict(cls, d: dict) -> "QuantizedKVSnapshot":
        return cls(d["keys"], d["values"], d["key_scales"], d["key_zeros"], d["value_scales"], d["value_zeros"])

    def as_dict(self) -> dict:
        return {"keys": self.keys, "values": self.values, "key_scales": self.key_scales,
                "key_zeros": self.key_zeros, "value_scales": self.value_scales, "value_zeros": self.value_zeros}


class SequenceKV:
    """One sequence of a KVPool; the per-layer caches are views of it."""

    def __init__(self, pool: KVPool, seq: int | None = None):
        self.pool = pool
        self.seq = pool.seq_create() if seq is None else seq
        self.layer_len = [0] * pool.num_layers
        if seq is not None:
            n = pool.seq_length(seq)
            self.layer_len = [n] * pool.num_layers

    @property
    def length(self) -> int:
        return self.pool.seq_length(self.seq)

    def slots_for(self, layer: int, n: int, start: int | None = None) -> np.ndarray:
        """Physical slots of positions [start, start + n) (default: the
        layer's length), reserving the positions beyond the sequence's length
        (copy-on-write of a shared tail block included)."""
        start = self.layer_len[layer] if start is None else start
        have = self.length
        if start > have:
            raise RuntimeError(f"layer {layer} writes at {start} while the sequence holds {have}")
        if start + n > have:
            self.pool.reserve_append(self.seq, start + n - have)
        table = self.pool.block_table(self.seq)
        pos = np.arange(start, start + n)
        return (table[pos // 64] * 64 + pos % 64).astype(np.int32)

    def shrink_to_layers(self):
        """Release the positions beyond the longest layer."""
        top = max(self.layer_len) if self.layer_len else 0
        if top < self.length:
            self.pool.seq_truncate(self.seq, top)

    def truncate(self, n: int):
        """QuantizedKVCache.truncate semantics (no-op unless 0 <= n < length)."""
        if 0 <= n < self.length:
            self.pool.seq_truncate(self.seq, n)
            self.layer_len = [min(x, n) for x in self.layer_len]

    def reset(self):
        self.pool.seq_reset(self.seq)
        self.layer_len = [0] * self.pool.num_layers

    def free(self):
        self.pool.seq_free(self.seq)

    def tables(self, device="cuda"):
        torch = _torch()
        n = self.length
        table = self.pool.block_table(self.seq)
        t = torch.as_tensor(table.reshape(1, -1) if table.size else np.zeros((1, 1), np.int32), device=device)
        return t.to(torch.int32), torch.tensor([n], dtype=torch.int32, device=device)


class PagedQuantizedKVCache:
    """One layer of one sequence (QuantizedKVCache.swift:17-146)."""

    def __init__(self, seqkv: SequenceKV, layer: int):
        self.s = seqkv
        self.layer = layer

    @property
    def sequence_length(self) -> int:
        return self.s.layer_len[self.layer]

    @property
    def memory_size_bytes(self) -> int:
        """memorySizeBytes (QuantizedKVCache.swift:33-42) for this layer."""
        n = self.sequence_length
        p = self.s.pool
        return 2 * n * p.num_kv_heads * p.head_dim + 4 * n * p.num_kv_heads * p.groups * 2

    def append(self, keys, values):
        """Quantize + append [1, Hkv, L, D] without dequantizing the cache."""
        torch = _torch()
        L = int(keys.shape[2])
        slots = self.s.slots_for(self.layer, L)
        sm = torch.as_tensor(slots.reshape(1, L), device=keys.device)
        self.s.pool.quantize_append(self.layer, keys.contiguous(), values.contiguous(), sm)
        self.s.layer_len[self.layer] += L

    def update(self, keys, values):
        """update(keys:values:) (QuantizedKVCache.swift:49-75): append, then
        return the whole cache dequantized to fp16 [1, Hkv, T, D]."""
        self.append(keys, values)
        return self.snapshot()

    def snapshot(self):
        """snapshot() (QuantizedKVCache.swift:82-89): dequantized fp16 K/V or None."""
        n = self.sequence_length
        if n == 0:
            return None
        tables, lens = self._tables(n)
        return self.s.pool.gather_dequant(self.layer, tables, lens, n)

    def quantized_snapshot(self):
        """quantizedSnapshot() (QuantizedKVCache.swift:106-115)."""
        n = self.sequence_length
        if n == 0:
            return None
        tables, lens = self._tables(n)
        return QuantizedKVSnapshot.from_dict(self.s.pool.gather(self.layer, tables, lens, n))

    def restore_quantized(self, snap: QuantizedKVSnapshot):
        """restoreQuantized(_:) (QuantizedKVCache.swift:122-129): this layer's
        contents become the snapshot's S tokens; the other layers keep
        theirs.  The bytes are copied into the pool, so later appends or
        truncates never change the snapshot.  Positions the sequence already
        holds are overwritten in place, which a block shared with another
        sequence or a prefix entry must not be: restoring into those raises
        (restore into a fresh cache instead, as the prefix replay does)."""
        torch = _torch()
        s, p = self.s, self.s.pool
        S = snap.sequence_length
        in_place = min(S, s.length)
        if in_place > 0:
            held = s.pool.block_table(s.seq)[: (in_place + 63) // 64]
            if (p.refcounts()[held] > 1).any():
                raise RuntimeError("restore_quantized would overwrite blocks shared with another sequence "
                                   "or a prefix entry; restore into a fresh cache")
        if S > 0:
            slots = s.slots_for(self.layer, S, start=0)
            dev = snap.keys.device
            p.scatter(self.layer, snap.as_dict(), torch.zeros(1, dtype=torch.int32, device=dev),
                      torch.as_tensor(slots.reshape(1, S), device=dev))
        s.layer_len[self.layer] = S
        s.shrink_to_layers()

    def truncate(self, n: int):
        self.s.truncate(n)

    def reset(self):
        self.s.reset()

    def _tables(self, n: int):
        torch = _torch()
        table = self.s.pool.block_table(self.s.seq)
        dev = "cuda"
        return (torch.as_tensor(table.reshape(1, -1), device=dev).to(torch.int32),
                torch.tensor([n], dtype=torch.int32, device=dev))


def make_quantized_kv_caches(pool: KVPool, seq: int | None = None):
    """makeQuantizedKVCaches(numLayers:) (QuantizedKVCache.swift:207-210)."""
    s = SequenceKV(pool, seq)
    return [PagedQuantizedKVCache(s, layer) for layer in range(pool.num_layers)]


class PrefixCache:
    """int8 prefix entries of one pool (PrefixCache.swift int8 API).

    Memory tier: the library's entries, frozen forks of a sequence: storing
    shares its blocks (refcounted, no copy) and a hit forks a new sequence
    from the entry.  Disk tier (``cache_dir`` set): every stored entry is also
    written as ``<key>.q8.safetensors`` (krill_amd.q8file; the bytes are
    copied to the host at store time and the file is written behind, on the
    process's background writer, unless ``write_behind`` is False), and a lookup that
    misses in memory at a length tries the file of that length before the
    next shorter one (PrefixCache.swift:273-308); a file hit is restored into
    fresh blocks and becomes a memory entry again.  The reference always has
    a disk tier (default ~/.krill/cache); here it is off unless a directory
    is given.  A restored entry keeps its tokens (the lookup knows them), so
    unlike the reference's disk-hydrated entries it can also serve
    longest-prefix hits."""

    def __init__(self, pool: KVPool, model_id: str = "", cache_dir=None, disk_budget_gb=None,
                 max_entry_gb=None, min_prefix_len: int = 8, write_behind: bool = True):
        from .q8file import DiskTier, _env_gb

        self.pool = pool
        self.model_id = model_id
        self.min_prefix_len = min_prefix_len  # the pool's min_prefix_len (PrefixCache minPrefixLength)
        self.disk = DiskTier(cache_dir, disk_budget_gb) if cache_dir is not None else None
        gb = max_entry_gb if max_entry_gb is not None else _env_gb("KRILL_PREFIX_CACHE_MAX_ENTRY_GB")
        gb = 4.0 if gb is None else gb
        self.max_entry_bytes = -1 if gb <= 0 else int(gb * 1_000_000_000)
        self.write_behind = write_behind

    @staticmethod
    def common_prefix_length(a, b) -> int:
        """PrefixCache.commonPrefixLength (PrefixCache.swift:266-271)."""
        n = min(len(a), len(b))
        i = 0
        while i < n and a[i] == b[i]:
            i += 1
        return i

    def _key(self, tokens, media_hash) -> int:
        from .pool import prefix_key

        return prefix_key(self.model_id, media_hash, 2, tokens)  # KVDtype.int8 = 2

    def _entry_bytes(self, n: int) -> int:
        p = self.pool
        return p.num_layers * p.num_kv_heads * n * (2 * p.head_dim + 8 * p.groups)

    def store_quantized(self, tokens, seq: int, media_hash=None) -> bool:
        """storeQuantized (PrefixCache.swift:369-400): memory entry, then the file."""
        if len(tokens) < self.min_prefix_len:
            return False
        if 0 < self.max_entry_bytes < self._entry_bytes(len(tokens)):
            return False
        stored = self.pool.prefix_store(seq, tokens, self.model_id, media_hash)
        if stored and self.disk is not None and self.disk.enabled:
            # the bytes come to the host now (the entry's blocks may be
            # evicted and reused later); the file write goes behind
            self.disk.write(self._key(tokens, media_hash), self._layers_of(seq, len(tokens)),
                            background=self.write_behind)
        return stored

    def wait_for_disk_writes(self):
        """Until every queued file write has finished (waitForDiskWrites,
        PrefixCache.swift:760-766)."""
        from .q8file import wait_for_disk_writes

        wait_for_disk_writes()

    def lookup_quantized(self, tokens, media_hash=None):
        """(prefix_len, entry_seq) of an exact entry, or (0, None)."""
        if self.disk is None or not self.disk.enabled:
            return self.pool.prefix_lookup(tokens, self.model_id, media_hash)
        # scan (PrefixCache.swift:273-308): at each length the memory entry
        # (one exact probe), then that length's file, then the next length
        tokens = np.ascontiguousarray(tokens, np.int64)
        step = max(1, self.min_prefix_len // 2)
        n = len(tokens)
        while n >= self.min_prefix_len:
            entry = self.pool.prefix_probe(tokens[:n], self.model_id, media_hash)
            if entry is not None:
                return n, entry
            layers = self.disk.load(self._key(tokens[:n], media_hash))
            if layers is not None and self._restore(tokens[:n], layers, media_hash):
                entry = self.pool.prefix_probe(tokens[:n], self.model_id, media_hash)
                if entry is not None:
                    return n, entry
            n -= step
        return 0, None

    def lookup_longest_prefix_quantized(self, tokens, media_hash=None):
        return self.pool.prefix_lookup_longest(tokens, self.model_id, media_hash)

    @property
    def memory_count(self) -> int:
        return self.pool.prefix_count()

    @property
    def disk_count(self) -> int:
        if self.disk is None:
            return 0
        self.wait_for_disk_writes()
        return self.disk.count

    def clear(self):
        self.pool.prefix_clear()
        if self.disk is not None:
            self.disk.clear()

    # ------------------------------------------------------------ files
    def _layers_of(self, seq: int, n: int) -> list:
        """The first n tokens of seq, every layer, as host snapshot arrays."""
        s = SequenceKV(self.pool, seq)
        tables, lens = s.tables()
        lens.fill_(n)
        out = []
        for layer in range(self.pool.num_layers):
            snap = self.pool.gather(layer, tables, lens, n)
            out.append({k: v.cpu().numpy() for k, v in snap.items()})
        return out

    def _restore(self, tokens, layers, media_hash) -> bool:
        """A file's layers into fresh blocks, stored as a memory entry."""
        torch = _torch()
        p = self.pool
        n = len(tokens)
        want = {"keys": (1, p.num_kv_heads, n, p.head_dim), "key_scales": (1, p.num_kv_heads, n, p.groups)}
        if len(layers) != p.num_layers:
            return False
        for snap in layers:
            for f, shape in (("keys", want["keys"]), ("values", want["keys"]), ("key_scales", want["key_scales"]),
                             ("key_zeros", want["key_scales"]), ("value_scales", want["key_scales"]),
                             ("value_zeros", want["key_scales"])):
                if tuple(snap[f].shape) != shape:
                    return False
        seq = p.seq_create()
        try:
            slots = p.reserve_append(seq, n)
            sm = torch.as_tensor(slots.reshape(1, n), device="cuda")
            zero = torch.zeros(1, dtype=torch.int32, device="cuda")
            for layer, snap in enumerate(layers):
                d = {k: torch.from_numpy(np.ascontiguousarray(v)).to("cuda") for k, v in snap.items()}
                p.scatter(layer, d, zero, sm)
            return p.prefix_store(seq, tokens, self.model_id, media_hash)
        finally:
            p.seq_free(seq)
