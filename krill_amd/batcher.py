"""Epoch-free continuous batching over a KVPool.

The reference batcher (Sources/KrillEngine/ContinuousBatcher.swift) runs in
epochs: at each boundary it drops finished rows, prefills newcomers
(``prefillAndAdmit``), stacks every active row's cache left-padded into one
batch (``stackCachesLeftPaddedAny``, :303-335 -> BatchedDecode.swift:96-151,
an O(total context) copy), decodes until the active set changes (:366-466),
then scatters the grown stack back into each row's cache (``scatterBack``,
:733-802, another O(total context) copy).

With paged KV the rows' caches are already where the attention reads them:
the batch is a list of block tables.  A row may join or leave at any step;
joining costs the newcomer's own prefill, leaving frees its blocks, and the
rows already running are not copied.  ``Scheduler`` keeps the admission
order of the reference (pending requests in arrival order, at most
``max_rows`` active, a finished or cancelled row leaves before the next step,
:277-301); ``ContinuousBatcher`` drives the pool:

* admission: a sequence per newcomer, its prompt appended in chunks
  (``prefill_chunk`` tokens; per layer ``quantize_append`` then causal
  attention of the chunk's rows, the chunked prefill of
  InferenceEngine.swift:3122-3149);
* decode step: one slot per active row, the batch's block tables, per layer
  one ``decode_append_attention`` (append of the new token fused with the
  attention over every row's cache);
* retirement: ``seq_free`` (refcounted blocks return to the pool).

The model is the caller's: ``model.prefill(req, start, n, layer)`` and
``model.decode(reqs, positions, layer)`` return the bf16/fp16 projections
(q [B, Hq, L, D], k and v [B, Hkv, L, D], on the device), and
``model.consume(reqs, layer, positions, out)`` receives the attention output
rows.
"""
from __future__ import annotations

from collections import deque
from dataclasses import dataclass, field

import numpy as np

from .pool import KVPool


def _torch():
    import torch

    return torch


@dataclass
class Request:
    """One generation request: prompt length and tokens to generate."""

    rid: int
    prompt_len: int
    max_new_tokens: int
    cancelled: bool = False


@dataclass
class Row:
    """An active request and its sequence in the pool."""

    req: Request
    seq: int = -1
    generated: int = 0
    finished: bool = False
    length: int = 0  # tokens in the cache


class Scheduler:
    """Active set and pending queue (ContinuousBatcher.swift:277-301 without
    the epoch): ``plan_step`` retires finished / cancelled rows and admits
    pending requests in arrival order up to ``max_rows``."""

    def __init__(self, max_rows: int):
        if max_rows < 1:
            raise ValueError("max_rows must be >= 1")
        self.max_rows = max_rows
        self.pending: deque = deque()
        self.rows: list = []

    def submit(self, req: Request):
        if req.prompt_len < 1 or req.max_new_tokens < 0:
            raise ValueError("a request needs a prompt and max_new_tokens >= 0")
        self.pending.append(req)

    def cancel(self, rid: int):
        for r in self.pending:
            if r.rid == rid:
                r.cancelled = True
        for row in self.rows:
            if row.req.rid == rid:
                row.req.cancelled = True

    def plan_step(self):
        """(retired rows, admitted rows) for the next step; the active set
        keeps its order, newcomers join at the end."""
        retired = [r for r in self.rows if r.finished or r.req.cancelled]
        self.rows = [r for r in self.rows if not (r.finished or r.req.cancelled)]
        admitted = []
        while self.pending and len(self.rows) < self.max_rows:
            req = self.pending.popleft()
            if req.cancelled:
                continue
            row = Row(req)
            self.rows.append(row)
            admitted.append(row)
        return retired, admitted

    @property
    def idle(self) -> bool:
        return not self.rows and not self.pending


class ContinuousBatcher:
    def __init__(self, pool: KVPool, model, max_rows: int, query_heads: int, scale: float,
                 prefill_chunk: int = 256, max_context: int = 1 << 17, out_dtype=None, stream=None):
        torch = _torch()
        self.pool, self.model = pool, model
        self.sched = Scheduler(max_rows)
        self.Hq, self.scale, self.stream = query_heads, float(scale), stream
        self.prefill_chunk = prefill_chunk
        self.max_blocks = (max_context + 63) // 64
        self.out_dtype = torch.bfloat16 if out_dtype is None else out_dtype
        self.layers = pool.num_layers
        self._ws = None
        self._dev = torch.device("cuda", torch.cuda.current_device())
        self.steps = 0
        self.admitted = 0
        self.retired = 0

    # --------------------------------------------------------------- API
    def submit(self, req: Request):
        self.sched.submit(req)

    def cancel(self, rid: int):
        self.sched.cancel(rid)

    @property
    def rows(self):
        return self.sched.rows

    @property
    def idle(self) -> bool:
        return self.sched.idle

    def step(self) -> int:
        """Retire, admit (prefill), then one decode step of every active row
        that still has tokens to generate.  Returns the rows decoded.  With a
        `stream` (a torch stream) the whole step -- the model's inputs, the
        table uploads, the workspace and the kernels -- runs on it."""
        if self.stream is None:
            return self._step()
        torch = _torch()
        with torch.cuda.stream(self.stream):
            return self._step()

    def _step(self) -> int:
        retired, admitted = self.sched.plan_step()
        for row in retired:
            self.pool.seq_free(row.seq)
            row.seq = -1
            self.retired += 1
        for row in admitted:
            row.seq = self.pool.seq_create()
            self._prefill(row)
            self.admitted += 1
        live = [r for r in self.rows if r.generated < r.req.max_new_tokens]
        for r in self.rows:
            if r.generated >= r.req.max_new_tokens:
                r.finished = True
        if live:
            self._decode(live)
        self.steps += 1
        return len(live)

    def run(self, max_steps: int = 1 << 30):
        n = 0
        while not self.idle and n < max_steps:
            self.step()
            n += 1
        return n

    # ------------------------------------------------------------ internals
    def _workspace(self, B: int, Lq: int, max_len: int):
        torch = _torch()
        need = self.pool.workspace_size(B, self.Hq, Lq, max_len)
        if self._ws is None or self._ws.numel() < need:
            self._ws = torch.empty(max(need, 1 << 20), dtype=torch.uint8, device=self._dev)
        return self._ws

    def _tables(self, rows):
        torch = _torch()
        mb = max(1, max((r.length + 63) // 64 for r in rows))
        if mb > self.max_blocks:
            raise ValueError(f"a row exceeds max_context ({self.max_blocks * 64} tokens)")
        t, n = self.pool.batch_tables([r.seq for r in rows], mb)
        return (torch.from_numpy(np.ascontiguousarray(t)).to(self._dev, non_blocking=False),
                torch.from_numpy(np.ascontiguousarray(n)).to(self._dev, non_blocking=False), int(n.max()))

    def _prefill(self, row: Row):
        torch = _torch()
        T, C = row.req.prompt_len, self.prefill_chunk
        for start in range(0, T, C):
            n = min(C, T - start)
            slots = self.pool.reserve_append(row.seq, n)
            row.length = start + n
            slots_d = torch.from_numpy(slots.reshape(1, n).copy()).to(self._dev)
            tables, lens, mx = self._tables([row])
            for layer in range(self.layers):
                q, k, v = self.model.prefill(row.req, start, n, layer)
                self.pool.quantize_append(layer, k, v, slots_d, stream=self.stream)
                out = self.pool.attention(layer, q, tables, lens, mx, self.scale, self.out_dtype,
                                          ws=self._workspace(1, n, mx), stream=self.stream)
                self.model.consume([row.req], layer, np.arange(start, start + n), out)

    def _decode(self, rows):
        for r in rows:
            self.pool.reserve_append(r.seq, 1)
            r.length += 1
        tables, lens, mx = self._tables(rows)
        reqs = [r.req for r in rows]
        positions = np.array([r.length - 1 for r in rows], np.int64)
        ws = self._workspace(len(rows), 1, mx)
        for layer in range(self.layers):
            q, k, v = self.model.decode(reqs, positions, layer)
            out = self.pool.decode_append_attention(layer, q, k, v, tables, lens, mx, self.scale, self.out_dtype,
                                                    ws=ws, stream=self.stream)
            self.model.consume(reqs, layer, positions, out)
        for r in rows:
            r.generated += 1
            if r.generated >= r.req.max_new_tokens:
                r.finished = True
