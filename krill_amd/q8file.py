"""On-disk int8 prefix entries: ``<key>.q8.safetensors`` and the disk tier of
the prefix cache.

File layout (PrefixCache.swift:553-598 load, :600-627 write): one safetensors
file per entry, per layer i the six arrays of a QuantizedKVSnapshot
(QuantizedKVCache.swift:150-173) under ``layer_{i}_qk`` (keys, u8
[1,Hkv,T,D]), ``layer_{i}_qv`` (values, u8), ``layer_{i}_ks`` / ``_kz`` (key
scales / zeros, f16 [1,Hkv,T,G]) and ``layer_{i}_vs`` / ``_vz`` (value
scales / zeros).  G = 1 in the reference's row mode, so row-mode pools read
and write the reference's files; affine pools store their G = D/64 groups
under the same names.  File name: the 16-hex-digit FNV-1a v3 entry key
(PrefixCache.swift:511-532) plus ``.q8.safetensors`` (:499).

Writes can go behind (PrefixCache.swift:20-21, :397-399): one background
writer thread shared by every disk tier of the process, like the
reference's serial disk queue; the caller hands over host arrays, so the
write never touches the pool.  A load of a file whose write is still queued
waits for the queue first, and the queue drains at interpreter exit.

Disk budget (PrefixCache.swift:98-113, :600-695): a running byte counter,
seeded by one directory scan on the first write; a write that takes it over
the budget evicts the oldest files by modification time down to 90 % of the
budget; a load refreshes the file's modification time.  Budget 0 disables
the disk tier, a negative budget disables eviction.
"""
from __future__ import annotations

import atexit
import os
import queue
import threading
from pathlib import Path

import numpy as np

SUFFIX = ".q8.safetensors"
NAMES = (("keys", "qk"), ("values", "qv"), ("key_scales", "ks"), ("key_zeros", "kz"),
         ("value_scales", "vs"), ("value_zeros", "vz"))


def entry_arrays(layers) -> dict:
    """layers: per layer a dict of the six snapshot arrays (numpy) -> file arrays."""
    out = {}
    for i, snap in enumerate(layers):
        for field, tag in NAMES:
            out[f"layer_{i}_{tag}"] = np.ascontiguousarray(snap[field])
    return out


def layers_of(arrays: dict) -> list:
    """File arrays -> per-layer snapshot dicts, layers 0, 1, .. while all six
    arrays of a layer are present (PrefixCache.swift:581-595)."""
    layers = []
    i = 0
    while all(f"layer_{i}_{tag}" in arrays for _, tag in NAMES):
        layers.append({field: arrays[f"layer_{i}_{tag}"] for field, tag in NAMES})
        i += 1
    return layers


def save_entry(path, layers, metadata=None):
    from safetensors.numpy import save_file

    save_file(entry_arrays(layers), str(path), metadata=metadata)


def load_entry(path) -> list:
    from safetensors.numpy import load_file

    return layers_of(load_file(str(path)))


def entry_bytes(layers) -> int:
    """int8KVBytes (PrefixCache.swift:708-716): the six arrays' bytes over all layers."""
    return int(sum(np.asarray(snap[f]).nbytes for snap in layers for f, _ in NAMES))


def _env_gb(name: str):
    v = os.environ.get(name)
    if v is None:
        return None
    try:
        return float(v)
    except ValueError:
        return None


class _WriteQueue:
    """The process's background writer: jobs run one at a time, in order."""

    def __init__(self):
        self._q = queue.Queue()
        self._lock = threading.Lock()
        self._pending = {}  # path -> queued writes
        self._thread = None
        self.errors = 0  # jobs that raised (a write-behind failure is not reported to the caller)

    def submit(self, path: Path, job):
        with self._lock:
            self._pending[path] = self._pending.get(path, 0) + 1
            if self._thread is None:
                self._thread = threading.Thread(target=self._run, name="krill-disk-writer", daemon=True)
                self._thread.start()
        self._q.put((path, job))

    def _run(self):
        while True:
            path, job = self._q.get()
            try:
                job()
            except Exception:
                self.errors += 1
            finally:
                with self._lock:
                    n = self._pending.pop(path, 1) - 1
                    if n > 0:
                        self._pending[path] = n
                self._q.task_done()

    def pending(self, path: Path) -> bool:
        with self._lock:
            return path in self._pending

    def wait(self):
        """Until every write queued so far has finished (waitForDiskWrites)."""
        self._q.join()


_WRITER = _WriteQueue()
atexit.register(_WRITER.wait)


def wait_for_disk_writes():
    _WRITER.wait()


class DiskTier:
    """The prefix cache's disk tier over one directory."""

    def __init__(self, cache_dir, disk_budget_gb=None):
        self.dir = Path(cache_dir)
        gb = disk_budget_gb if disk_budget_gb is not None else _env_gb("KRILL_PREFIX_CACHE_GB")
        gb = 2.0 if gb is None else gb
        self.budget = -1 if gb < 0 else int(gb * 1_000_000_000)
        self._lock = threading.Lock()
        self._bytes = 0
        self._seeded = False
        self.dir.mkdir(parents=True, exist_ok=True)

    @property
    def enabled(self) -> bool:
        return self.budget != 0

    def path(self, key: int) -> Path:
        return self.dir / f"{key:016x}{SUFFIX}"

    def _scan_bytes(self) -> int:
        return sum(p.stat().st_size for p in self.dir.iterdir() if p.name.endswith(".safetensors"))

    def write(self, key: int, layers, background: bool = False) -> bool:
        """Write the entry's file (host arrays `layers`), now or on the
        background writer; True when a write was done or queued."""
        if not self.enabled:
            return False
        if background:
            _WRITER.submit(self.path(key), lambda: self._write_now(key, layers))
            return True
        return self._write_now(key, layers)

    def _write_now(self, key: int, layers) -> bool:
        p = self.path(key)
        prior = p.stat().st_size if p.exists() else 0
        save_entry(p, layers, metadata={"format": "mlx"})
        new = p.stat().st_size
        with self._lock:
            if not self._seeded:
                self._bytes = self._scan_bytes()  # includes the file just written
                self._seeded = True
            else:
                self._bytes += new - prior
            over = self.budget > 0 and self._bytes > self.budget
        if over:
            self.evict_to_low_water()
        return True

    def load(self, key: int):
        """The entry's layers, or None (no file, unreadable, no complete layer)."""
        if not self.enabled:
            return None
        p = self.path(key)
        if _WRITER.pending(p):
            _WRITER.wait()
        if not p.exists():
            return None
        try:
            layers = load_entry(p)
        except Exception:
            return None
        try:
            os.utime(p, None)  # a hit is a use: the LRU keeps it
        except OSError:
            pass
        return layers or None

    def evict_to_low_water(self):
        """Oldest files first until the directory holds <= 90 % of the budget."""
        if self.budget <= 0:
            return
        low = self.budget - self.budget // 10
        files = []
        total = 0
        for p in self.dir.iterdir():
            if not p.name.endswith(".safetensors"):
                continue
            st = p.stat()
            files.append((st.st_mtime, st.st_size, p))
            total += st.st_size
        if total > self.budget:
            files.sort(key=lambda f: f[0])
            for _, size, p in files:
                if total <= low:
                    break
                try:
                    p.unlink()
                    total -= size
                except OSError:
                    pass
        with self._lock:
            self._bytes = total
            self._seeded = True

    def clear(self):
        _WRITER.wait()  # no queued write lands after the clear
        for p in list(self.dir.iterdir()):
            if p.is_file():
                p.unlink()
        with self._lock:
            self._bytes = 0
            self._seeded = True

    @property
    def count(self) -> int:
        return sum(1 for p in self.dir.iterdir() if p.name.endswith(".safetensors"))
