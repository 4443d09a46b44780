"""Block manager through the C ABI on a host-only pool (no GPU needed).

Known-answer cases re-express the reference's cache tests at the level of
token positions: the paged cache must hold, position by position, what the
reference's contiguous cache holds after the same updates, truncates and
restores (KVCacheTests.swift, SpeculativeDecodingTests.swift:99-158,
QuantizedPrefixCacheTests.swift, PrefixCacheTests.swift).  A simulated
device (slot -> token id, block copies applied for every copy-on-write)
checks the paging itself."""
import threading

import numpy as np
import pytest

import krill_amd
from krill_amd import KrillError
from krill_amd import _lib as L


def host_pool(blocks=64, **kw):
    return krill_amd.KVPool(2, 2, 128, blocks, "affine_g64", "bf16", host_only=True, **kw)


class Sim:
    """Logical content per sequence and a simulated device memory.  Block
    copies are applied whenever a reservation replaced a shared tail block."""

    def __init__(self, pool):
        self.pool = pool
        self.mem = {}      # slot -> token id
        self.content = {}  # seq -> list of token ids
        self.next_tok = 1

    def create(self):
        s = self.pool.seq_create()
        self.content[s] = []
        return s

    def append(self, s, n):
        before = self.pool.block_table(s)
        length = len(self.content[s])
        slots = self.pool.reserve_append(s, n)
        after = self.pool.block_table(s)
        if length % 64 and before[length // 64] != after[length // 64]:
            src, dst = before[length // 64], after[length // 64]   # copy-on-write
            for t in range(64):
                if src * 64 + t in self.mem:
                    self.mem[dst * 64 + t] = self.mem[src * 64 + t]
        rc = self.pool.refcounts()
        for sl in slots:
            assert rc[sl // 64] == 1, "a slot handed out for writing lives in a shared block"
        toks = list(range(self.next_tok, self.next_tok + n))
        self.next_tok += n
        for sl, t in zip(slots, toks):
            self.mem[int(sl)] = t
        self.content[s] += toks
        return slots

    def fork(self, s, n):
        f = self.pool.seq_fork(s, n)
        self.content[f] = self.content[s][:n]
        return f

    def truncate(self, s, n):
        self.pool.seq_truncate(s, n)
        if 0 <= n < len(self.content[s]):
            self.content[s] = self.content[s][:n]

    def free(self, s):
        self.pool.seq_free(s)
        del self.content[s]

    def read(self, s):
        table = self.pool.block_table(s)
        n = self.pool.seq_length(s)
        return [self.mem.get(int(table[p // 64]) * 64 + p % 64) for p in range(n)]

    def check(self, entries=()):
        for s, c in self.content.items():
            assert self.pool.seq_length(s) == len(c)
            assert len(self.pool.block_table(s)) == (len(c) + 63) // 64
            assert self.read(s) == c
        # refcount = number of tables (live + prefix entries) holding the block
        want = np.zeros(self.pool.num_blocks, np.int32)
        for s in list(self.content) + list(entries):
            for b in self.pool.block_table(s):
                want[b] += 1
        np.testing.assert_array_equal(self.pool.refcounts(), want)
        st = self.pool.stats()
        assert st["blocks_used"] == int((want > 0).sum())
        assert st["blocks_free"] == self.pool.num_blocks - st["blocks_used"]


# ------------------------------------------------------- known answers

def test_update_concatenates_along_sequence_axis():
    """KVCacheTests.swift:54-89: 1 row then 2 rows -> positions 0,1,2 in order."""
    p = host_pool()
    sim = Sim(p)
    s = sim.create()
    sim.append(s, 1)
    sim.append(s, 2)
    assert sim.read(s) == [1, 2, 3] and p.seq_length(s) == 3
    sim.check()


def test_truncate_slices_and_beyond_length_is_noop():
    """KVCacheTests.swift:134-179 and QuantizedKVCache.truncate (:135-145)."""
    p = host_pool()
    sim = Sim(p)
    s = sim.create()
    sim.append(s, 4)
    sim.truncate(s, 3)
    assert sim.read(s) == [1, 2, 3]
    sim.truncate(s, 6)   # beyond length: no-op
    sim.truncate(s, -1)  # negative: no-op for the quantized cache
    assert sim.read(s) == [1, 2, 3]
    sim.check()


def test_truncate_then_update_overwrites_stale_rows():
    """KVCacheTests.swift:239-275: append 10, truncate 6, append 2 equals a
    fresh cache fed the final sequence; the stale slots are reused."""
    p = host_pool()
    sim = Sim(p)
    s = sim.create()
    first = sim.append(s, 10)
    sim.truncate(s, 6)
    again = sim.append(s, 2)
    np.testing.assert_array_equal(again, first[6:8])
    assert sim.read(s) == [1, 2, 3, 4, 5, 6, 11, 12]
    sim.check()


def test_speculative_rollback_vectors():
    """SpeculativeDecodingTests.swift:99-158: keep prev + accepted; full accept
    keeps all k verify rows plus the bonus row."""
    p = host_pool()
    sim = Sim(p)
    s = sim.create()
    sim.append(s, 10)
    prev = p.seq_length(s)
    sim.append(s, 4)
    assert p.seq_length(s) == 14
    sim.truncate(s, prev + 2)
    assert sim.read(s) == list(range(1, 11)) + [11, 12]
    t = sim.create()
    sim.append(t, 10)
    sim.append(t, 4)
    sim.append(t, 1)
    assert p.seq_length(t) == 15 and sim.read(t)[-5:] == [25, 26, 27, 28, 29]
    sim.check()


def test_growth_across_many_blocks():
    """KVCacheTests.swift:306-331: 300 appends of 2 rows survive intact."""
    p = host_pool(blocks=16)
    sim = Sim(p)
    s = sim.create()
    for _ in range(300):
        sim.append(s, 2)
    assert p.seq_length(s) == 600 and sim.read(s) == list(range(1, 601))
    sim.check()


def test_reset_and_memory_bytes():
    p = host_pool()
    s = p.seq_create()
    p.reserve_append(s, 100)
    # memorySizeBytes (QuantizedKVCache.swift:33-42) with G = 2 groups
    assert p.seq_memory_bytes(s) == 2 * 100 * 2 * 128 + 4 * 100 * 2 * 2 * 2
    p.seq_reset(s)
    assert p.seq_length(s) == 0 and p.stats()["blocks_used"] == 0


def test_fork_shares_blocks_and_cow_protects_the_sharer():
    p = host_pool()
    sim = Sim(p)
    a = sim.create()
    sim.append(a, 100)
    f = sim.fork(a, 70)
    assert p.block_table(f).tolist() == p.block_table(a).tolist()
    assert p.refcounts()[p.block_table(a)].tolist() == [2, 2]
    sim.append(f, 5)            # tail block 1 is shared -> copied
    assert p.stats()["cow_copies"] == 1
    assert p.block_table(f)[0] == p.block_table(a)[0] and p.block_table(f)[1] != p.block_table(a)[1]
    sim.append(a, 3)            # a's tail is no longer shared: written in place
    assert p.stats()["cow_copies"] == 1
    sim.check()
    g = sim.fork(a, 64)          # fork at a block boundary: the next token opens a new block
    sim.append(g, 1)
    assert p.stats()["cow_copies"] == 1
    sim.check()


def test_pool_exhaustion_is_an_error_that_changes_nothing():
    p = host_pool(blocks=4)
    s = p.seq_create()
    p.reserve_append(s, 200)
    with pytest.raises(KrillError) as e:
        p.reserve_append(s, 100)
    assert e.value.code == L.KRILL_E_NOMEM
    assert p.seq_length(s) == 200 and p.stats()["blocks_used"] == 4
    p.reserve_append(s, 56)  # exactly fills the pool
    assert p.seq_length(s) == 256


def test_frozen_entries_reject_mutation_and_bad_handles():
    p = host_pool()
    s = p.seq_create()
    p.reserve_append(s, 20)
    assert p.prefix_store(s, list(range(20)), "m")
    _, e = p.prefix_lookup(list(range(20)), "m")
    for fn in (lambda: p.reserve_append(e, 1), lambda: p.seq_truncate(e, 3), lambda: p.seq_free(e)):
        with pytest.raises(KrillError) as err:
            fn()
        assert err.value.code == L.KRILL_E_STATE
    for fn in (lambda: p.seq_length(999), lambda: p.seq_free(-1)):
        with pytest.raises(KrillError) as err:
            fn()
        assert err.value.code == L.KRILL_E_INVAL
    with pytest.raises(KrillError) as err:
        p.seq_fork(s, 21)
    assert err.value.code == L.KRILL_E_RANGE


# ---------------------------------------------------------------- prefix

def test_prefix_store_and_full_hit():
    """QuantizedPrefixCacheTests.swift:25-53, :142-171: a full hit restores
    the stored sequence; truncate(count - 1) and re-forward returns to count."""
    p = host_pool(min_prefix_len=4, max_prefix_entries=4)
    sim = Sim(p)
    s = sim.create()
    sim.append(s, 6)
    assert p.prefix_store(s, list(range(6)), "m-int8")
    plen, e = p.prefix_lookup(list(range(6)), "m-int8")
    assert plen == 6 and e is not None
    r = p.seq_fork(e, 5)           # restore + truncate(to: 5)
    sim.content[r] = sim.content[s][:5]
    sim.append(r, 1)               # re-feed the last token
    assert p.seq_length(r) == 6
    sim.check(entries=[e])
    # the entry is unchanged by the restored sequence's write
    assert sim.read(e) == [1, 2, 3, 4, 5, 6]


def test_lookup_longest_prefix_vectors():
    """QuantizedPrefixCacheTests.swift:92-121 (LCP 5, below-min miss)."""
    p = host_pool(min_prefix_len=4)
    s = p.seq_create()
    p.reserve_append(s, 8)
    stored = [10, 11, 12, 13, 14, 15, 16, 17]
    assert p.prefix_store(s, stored, "m-int8")
    assert p.prefix_lookup_longest([10, 11, 12, 13, 14, 99, 99], "m-int8")[0] == 5
    assert p.prefix_lookup_longest([10, 11, 0, 0, 0, 0], "m-int8") == (0, None)
    assert p.prefix_lookup_longest([10, 11, 12, 13, 14, 99, 99], "other") == (0, None)
    assert p.prefix_lookup_longest([10, 11, 12, 13, 14, 99, 99], "m-int8", "img") == (0, None)


def test_longest_match_wins():
    """PrefixCacheTests.swift:321-343."""
    p = host_pool(min_prefix_len=4)
    short = list(range(6)) + [50]
    long = list(range(9)) + [60]
    a, b = p.seq_create(), p.seq_create()
    p.reserve_append(a, len(short))
    p.reserve_append(b, len(long))
    p.prefix_store(a, short, "m")
    p.prefix_store(b, long, "m")
    plen, e = p.prefix_lookup_longest(list(range(9)) + [99, 99], "m")
    assert plen == 9 and p.seq_length(e) == len(long)


def test_exact_scan_steps_down_by_half_min_length():
    """scan (PrefixCache.swift:273-308): checkLen = n, n - min/2, ..."""
    p = host_pool(min_prefix_len=8)
    s = p.seq_create()
    p.reserve_append(s, 16)
    p.prefix_store(s, list(range(12)), "m")
    assert p.prefix_lookup(list(range(16)), "m")[0] == 12      # 16 -> 12 hits
    assert p.prefix_lookup(list(range(15)), "m") == (0, None)   # 15, 11: no entry of that length
    assert p.prefix_lookup(list(range(7)), "m") == (0, None)    # below minPrefixLength


def test_store_guards_and_lru_capacity():
    p = host_pool(min_prefix_len=4, max_prefix_entries=3, max_entry_bytes=2 * (2 * 10 * 2 * 128 + 4 * 10 * 2 * 2 * 2))
    s = p.seq_create()
    p.reserve_append(s, 40)
    assert not p.prefix_store(s, [1, 2, 3], "m")            # below minPrefixLength
    assert not p.prefix_store(s, list(range(11)), "m")      # over the per-entry byte cap
    for i in range(5):
        assert p.prefix_store(s, [100 + i] + list(range(5)), "m")
    assert p.prefix_count() == 3                            # LRU capacity
    assert p.prefix_lookup([100] + list(range(5)), "m") == (0, None)   # oldest evicted
    assert p.prefix_lookup([104] + list(range(5)), "m")[0] == 6


def test_watermark_eviction_frees_unreferenced_blocks():
    """At 90% occupancy the oldest entries whose blocks no live sequence holds
    are evicted; entries shared with live sequences survive."""
    p = host_pool(blocks=20, max_prefix_entries=16, min_prefix_len=4)
    live = p.seq_create()
    p.reserve_append(live, 128)                       # 2 blocks, stays live
    p.prefix_store(live, list(range(128)), "m")       # entry shares live's blocks
    olds = []
    for i in range(4):
        s = p.seq_create()
        p.reserve_append(s, 192)                      # 3 blocks each
        p.prefix_store(s, [1000 * (i + 1)] + list(range(191)), "m")
        p.seq_free(s)                                 # only the entry holds them now
        olds.append([1000 * (i + 1)] + list(range(191)))
    assert p.stats()["blocks_used"] == 14 and p.prefix_count() == 5
    big = p.seq_create()
    p.reserve_append(big, 5 * 64)                     # 14 + 5 > 18 (90% of 20)
    st = p.stats()
    assert st["blocks_used"] <= 18 and st["evicted_entries"] >= 1
    assert p.prefix_lookup(olds[0], "m") == (0, None)  # least recently stored went first
    assert p.prefix_lookup(list(range(128)), "m")[0] == 128  # shared with a live seq: kept
    p.reserve_append(big, 64 * 5)                     # needs the rest: evicts what it must
    assert p.prefix_lookup(list(range(128)), "m")[0] == 128
    with pytest.raises(KrillError):
        p.reserve_append(big, 64 * 10)


def test_prefix_key_matches_oracle(oracle):
    toks = [5, -3, 1 << 40]
    assert krill_amd.prefix_key("model", "media", 2, toks) == oracle.prefix_key("model", "media", 2, toks)
    assert krill_amd.prefix_key("model", None, 2, []) == oracle.prefix_key("model", None, 2, [])


# ----------------------------------------------------------- randomized

def test_model_based_random_operations():
    hypothesis = pytest.importorskip("hypothesis")
    st = hypothesis.strategies

    @hypothesis.settings(max_examples=60, deadline=None)
    @hypothesis.given(st.lists(st.tuples(st.integers(0, 6), st.integers(0, 10**6)), min_size=5, max_size=60))
    def run(ops):
        p = host_pool(blocks=48, min_prefix_len=4, max_prefix_entries=4, evict_watermark=0.9)
        sim = Sim(p)
        entries = {}
        for op, arg in ops:
            seqs = sorted(sim.content)
            if op == 0 or not seqs:
                sim.create()
            elif op == 1:
                s = seqs[arg % len(seqs)]
                try:
                    sim.append(s, 1 + arg % 90)
                except KrillError as e:
                    assert e.code == L.KRILL_E_NOMEM
            elif op == 2:
                s = seqs[arg % len(seqs)]
                sim.truncate(s, arg % (len(sim.content[s]) + 2) - 1)
            elif op == 3:
                s = seqs[arg % len(seqs)]
                sim.fork(s, arg % (len(sim.content[s]) + 1))
            elif op == 4:
                sim.free(seqs[arg % len(seqs)])
            elif op == 5:
                s = seqs[arg % len(seqs)]
                if not sim.content[s]:
                    continue
                toks = [arg] + sim.content[s][1:]
                if p.prefix_store(s, toks, "m"):
                    entries[tuple(toks)] = list(sim.content[s])
            else:
                keys = list(entries)
                if keys:
                    toks = list(keys[arg % len(keys)])
                    plen, e = p.prefix_lookup(toks, "m")
                    if e is not None:
                        # an entry that survives still holds exactly what was stored
                        got = sim.read(e)
                        assert got == entries[tuple(toks)][:plen]
            # entries evicted or alive: recount
            live_entries = []
            for toks in list(entries):
                plen, e = p.prefix_lookup(list(toks), "m")
                if e is None:
                    del entries[toks]
                else:
                    live_entries.append(e)
            sim.check(entries=live_entries)
        p.close()

    run()


def test_concurrent_hammer_keeps_capacity_invariant():
    """PrefixCacheTests.swift:354-380: 8 threads x 200 iterations."""
    p = host_pool(blocks=4096, min_prefix_len=4, max_prefix_entries=4)
    errors = []

    def worker(t):
        try:
            for i in range(200):
                s = p.seq_create()
                p.reserve_append(s, 6)
                toks = list(range(t * 1000 + i, t * 1000 + i + 6))
                p.prefix_store(s, toks, f"m{i % 3}")
                p.prefix_lookup(toks, f"m{i % 3}")
                p.prefix_lookup(list(range(6)), f"m{i % 3}")
                p.seq_free(s)
                if i % 50 == 0:
                    p.prefix_clear()
        except Exception as e:  # pragma: no cover - reported below
            errors.append(e)

    threads = [threading.Thread(target=worker, args=(t,)) for t in range(8)]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors
    assert p.prefix_count() <= 4
    st = p.stats()
    assert st["live_seqs"] == 0
    p.prefix_clear()
    assert p.stats()["blocks_used"] == 0


# ---- sliding window (pool option): RotatingKVCache retention in paged form

def _window_pool(window, blocks=64):
    p = host_pool(blocks)
    p.set_option(L.OPT_WINDOW, window)
    return p


def test_window_retains_last_window_tokens_reference_vectors(oracle):
    # RotatingKVCacheTests.swift:115-131 (window 4, ten single appends)
    p = _window_pool(4)
    s = p.seq_create()
    for t in range(10):
        p.reserve_append(s, 1)
        start = int(p.batch_starts([s])[0])
        assert p.seq_length(s) == t + 1 and (t + 1) - start == min(t + 1, 4)
        assert (t + 1, start) == oracle.rotating_retained_start([("append", 1)] * (t + 1), 4)
    p.close()


def test_window_truncate_bounds_reference_vectors():
    # RotatingKVCacheTests.swift:133-161: retained 6..9 after ten appends
    p = _window_pool(4)
    s = p.seq_create()
    for _ in range(10):
        p.reserve_append(s, 1)
    assert int(p.batch_starts([s])[0]) == 6
    with pytest.raises(KrillError) as e:
        p.seq_truncate(s, 5)  # position 5 was rotated out
    assert e.value.code == L.KRILL_E_RANGE and p.seq_length(s) == 10
    p.seq_truncate(s, 8)
    assert p.seq_length(s) == 8
    p.reserve_append(s, 1)  # retained 6, 7 and the new token
    assert p.seq_length(s) == 9 and int(p.batch_starts([s])[0]) == 6
    p.close()


def test_window_frees_blocks_and_matches_the_rotating_model(oracle):
    W = 150
    p = _window_pool(W, blocks=40)
    s = p.seq_create()
    rng = np.random.default_rng(5)
    ops = []
    for _ in range(40):
        if rng.random() < 0.15 and ops:
            total, start = oracle.rotating_retained_start(ops, W)
            n = int(rng.integers(start, total + 1))
            ops.append(("truncate", n))
            p.seq_truncate(s, n)
        else:
            L_ = int(rng.integers(1, 90))
            ops.append(("append", L_))
            p.reserve_append(s, L_)
        total, start = oracle.rotating_retained_start(ops, W)
        assert p.seq_length(s) == total and int(p.batch_starts([s])[0]) == start
        table = p.block_table(s)
        # blocks wholly below the first retained token are dropped (-1), the rest held
        assert all(b == -1 for b in table[: start // 64]) and all(b >= 0 for b in table[start // 64:])
        assert p.stats()["blocks_used"] == len(table) - start // 64
    # 40 appends of up to 89 tokens in a 40-block pool: only the window stays
    assert p.seq_length(s) > 40 * 64 // 4
    p.seq_free(s)
    assert p.stats()["blocks_used"] == 0
    p.close()


def test_window_guards():
    p = _window_pool(100)
    with pytest.raises(KrillError):
        p.set_option(L.OPT_WINDOW, 1)
    s = p.seq_create()
    p.reserve_append(s, 300)
    p.reserve_append(s, 1)  # trims: first retained token 201
    assert int(p.batch_starts([s])[0]) == 201
    with pytest.raises(KrillError) as e:
        p.seq_fork(s, 150)  # below the window
    assert e.value.code == L.KRILL_E_RANGE
    f = p.seq_fork(s, 250)
    assert int(p.batch_starts([f])[0]) == 201
    with pytest.raises(KrillError) as e:
        p.prefix_store(s, np.arange(301))  # a prefix entry needs every token
    assert e.value.code == L.KRILL_E_UNSUPPORTED
    with pytest.raises(KrillError):
        p.set_option(L.OPT_WINDOW, 0)  # tokens already dropped
    p.close()


# ---- regressions: entries as store sources, failed appends, the exact probe

def _refcount_invariant(p, seqs):
    """Every block's refcount equals the number of table entries naming it
    over the given live sequences and the prefix entries."""
    rc = p.refcounts()
    want = np.zeros_like(rc)
    for s in seqs:
        for b in p.block_table(s):
            if b >= 0:
                want[b] += 1
    return rc, want


def test_store_from_an_entry_with_the_same_key_keeps_its_blocks():
    p = host_pool(min_prefix_len=8)
    s = p.seq_create()
    p.reserve_append(s, 100)
    toks = list(range(100))
    assert p.prefix_store(s, toks, "m")
    _, e = p.prefix_lookup(toks, "m")
    table = p.block_table(e).copy()
    # the source is the entry that the key match replaces
    assert p.prefix_store(e, toks, "m")
    plen, e2 = p.prefix_lookup(toks, "m")
    assert plen == 100 and p.prefix_count() == 1
    assert np.array_equal(p.block_table(e2), table)
    rc = p.refcounts()
    assert all(rc[b] == 2 for b in table)   # the live sequence and the new entry
    p.seq_free(s)
    assert all(p.refcounts()[b] == 1 for b in table)
    p.prefix_clear()
    assert p.stats()["blocks_used"] == 0
    p.close()


def test_store_from_an_entry_that_capacity_eviction_drops():
    p = host_pool(min_prefix_len=8, max_prefix_entries=1)
    s = p.seq_create()
    p.reserve_append(s, 200)
    toks = list(range(200))
    assert p.prefix_store(s, toks, "m")
    _, e = p.prefix_lookup(toks, "m")
    p.seq_free(s)                       # the entry holds the only references
    assert p.prefix_store(e, toks[:100], "m")   # at capacity: the source is evicted
    assert p.prefix_count() == 1
    plen, e2 = p.prefix_lookup(toks[:100], "m")
    assert plen == 100 and p.seq_length(e2) == 100
    assert p.stats()["blocks_used"] == 2          # the 100-token entry's two blocks
    assert all(p.refcounts()[b] == 1 for b in p.block_table(e2))
    p.prefix_clear()
    assert p.stats()["blocks_used"] == 0
    p.close()


def test_failed_append_on_a_window_pool_changes_nothing():
    p = _window_pool(100, blocks=4)
    s = p.seq_create()
    p.reserve_append(s, 200)                 # 4 blocks, nothing trimmed yet
    other_table = p.block_table(s).copy()
    q = p.seq_fork(s, 200)                   # shares every block: the trim frees none
    with pytest.raises(KrillError) as e:
        p.reserve_append(s, 100)             # would trim to 101 and need a 5th block
    assert e.value.code == L.KRILL_E_NOMEM
    assert p.seq_length(s) == 200 and int(p.batch_starts([s])[0]) == 0
    assert np.array_equal(p.block_table(s), other_table)
    assert p.stats()["blocks_used"] == 4
    assert all(p.refcounts()[b] == 2 for b in other_table)
    p.seq_free(q)
    p.reserve_append(s, 100)                 # now the trimmed blocks make room
    assert int(p.batch_starts([s])[0]) == 101 and p.seq_length(s) == 300
    p.close()


def test_failed_append_rolls_back_a_trim_that_freed_blocks():
    # the trim frees a block (its only reference) and the append still
    # needs more blocks than the pool then has
    p = _window_pool(70, blocks=4)
    s = p.seq_create()
    p.reserve_append(s, 150)                       # blocks 0..2, tail block 2 partly filled
    f = p.seq_fork(s, 150)                         # shares all three
    p.seq_free(f)
    before = p.block_table(s).copy()
    used = p.stats()["blocks_used"]
    with pytest.raises(KrillError):
        p.reserve_append(s, 300)                   # needs 4 more blocks after the trim frees 1
    assert np.array_equal(p.block_table(s), before)
    assert p.stats()["blocks_used"] == used and int(p.batch_starts([s])[0]) == 0
    assert all(p.refcounts()[b] == 1 for b in before)
    p.close()


def test_fork_below_the_window_leaks_no_sequence_id():
    p = _window_pool(100)
    s = p.seq_create()
    p.reserve_append(s, 300)
    p.reserve_append(s, 1)
    spare = p.seq_create()
    p.seq_free(spare)                     # its id is the next one handed out
    with pytest.raises(KrillError):
        p.seq_fork(s, 150)
    assert p.seq_create() == spare
    p.close()


def test_exact_probe_hits_one_length_and_touches_only_on_a_hit():
    p = host_pool(min_prefix_len=8, max_prefix_entries=2)
    s = p.seq_create()
    p.reserve_append(s, 64)
    a, b = list(range(40)), list(range(100, 140))
    assert p.prefix_store(s, a, "m") and p.prefix_store(s, b, "m")
    assert p.prefix_probe(a[:39], "m") is None        # one length only, no scan
    assert p.prefix_probe(a, "other") is None
    assert p.prefix_probe(a[:7], "m") is None         # below minPrefixLength
    assert p.prefix_probe(a, "m") is not None         # hit: a becomes most recent
    p.prefix_store(s, list(range(200, 240)), "m")     # evicts the least recent: b
    assert p.prefix_probe(b, "m") is None and p.prefix_probe(a, "m") is not None
    p.close()


def test_disk_scan_probes_each_length_once(tmp_path):
    from krill_amd.cache import PrefixCache

    p = host_pool(min_prefix_len=8)
    cache = PrefixCache(p, "m", cache_dir=tmp_path, min_prefix_len=8)
    calls = []
    real = p.prefix_probe
    p.prefix_probe = lambda t, *a: calls.append(len(t)) or real(t, *a)
    toks = np.arange(2048)
    assert cache.lookup_quantized(toks) == (0, None)
    assert calls == list(range(2048, 7, -4))
    s = p.seq_create()
    p.reserve_append(s, 16)
    assert p.prefix_store(s, toks[:12], "m")
    calls.clear()
    assert cache.lookup_quantized(toks[:16])[0] == 12
    assert calls == [16, 12]
    p.close()


def test_cache_layers_share_positions_and_restore_replaces_one_layer():
    """The reference-shaped cache's host bookkeeping (no device work): layers
    append at their own lengths, the sequence holds positions up to the
    longest layer, truncate applies to all layers, a restore of a shorter
    layer releases the positions no layer holds any more."""
    from krill_amd.cache import make_quantized_kv_caches

    p = host_pool()
    c0, c1 = make_quantized_kv_caches(p)
    s0 = c0.s.slots_for(0, 70)
    c0.s.layer_len[0] += 70
    assert p.seq_length(c0.s.seq) == 70
    s1 = c1.s.slots_for(1, 70)  # the positions layer 0 reserved
    c1.s.layer_len[1] += 70
    np.testing.assert_array_equal(s0, s1)
    assert p.seq_length(c0.s.seq) == 70
    c1.s.slots_for(1, 10)  # layer 1 runs ahead
    c1.s.layer_len[1] += 10
    assert p.seq_length(c0.s.seq) == 80 and c0.sequence_length == 70
    c0.truncate(75)  # applies to the sequence: layer 1 drops to 75, layer 0 keeps 70
    assert (c0.sequence_length, c1.sequence_length, p.seq_length(c0.s.seq)) == (70, 75, 75)
    with pytest.raises(RuntimeError):
        c0.s.slots_for(0, 1, start=76)  # beyond the sequence
    c1.s.layer_len[1] = 70  # as a restore of a 70-token snapshot leaves it
    c1.s.shrink_to_layers()
    assert p.seq_length(c0.s.seq) == 70
    p.close()


def test_krill_kernels_validate_the_batch_on_the_host():
    from krill_amd import KrillKernels
    from krill_amd.cache import make_quantized_kv_caches

    p = host_pool()
    a = make_quantized_kv_caches(p)
    b = make_quantized_kv_caches(p)
    q = np.zeros((2, 4, 1, 128), np.float32)
    with pytest.raises(ValueError, match="empty"):
        KrillKernels.paged_decode_attention(q, [], 0.1)
    with pytest.raises(ValueError, match="same layer"):
        KrillKernels.paged_decode_attention(q, [a[0], b[1]], 0.1)
    with pytest.raises(ValueError, match="twice"):
        KrillKernels.paged_decode_attention(q, [a[0], a[0]], 0.1)
    with pytest.raises(ValueError, match="queries"):
        KrillKernels.paged_decode_attention(q[:1], [a[0], b[0]], 0.1)
    with pytest.raises(ValueError, match="together"):
        KrillKernels.paged_decode_attention(q, [a[0], b[0]], 0.1, keys=q)
    with pytest.raises(TypeError):
        KrillKernels.paged_decode_attention(q, [a[0], object()], 0.1)
    assert isinstance(KrillKernels.status(), str)
    p.close()


def test_krill_kernels_change_no_state_when_the_call_fails():
    """A decode step whose launch is refused leaves every cache as it was:
    no layer length advances and no reserved position stays behind (here the
    call fails because the tensors are not on a HIP device)."""
    import torch

    from krill_amd import KrillKernels
    from krill_amd.cache import make_quantized_kv_caches

    p = host_pool()
    a = make_quantized_kv_caches(p)
    b = make_quantized_kv_caches(p)
    for c in (a[0], b[0], a[1], b[1]):
        c.s.slots_for(c.layer, 70)
        c.s.layer_len[c.layer] += 70
    q = torch.zeros((2, 4, 1, 128), dtype=torch.bfloat16)
    kv = torch.zeros((2, 2, 1, 128), dtype=torch.bfloat16)
    before = [(p.seq_length(c.s.seq), list(c.s.layer_len)) for c in (a[0], b[0])]
    with pytest.raises(Exception):
        KrillKernels.paged_decode_attention(q, [a[0], b[0]], 0.1, keys=kv, values=kv)
    assert [(p.seq_length(c.s.seq), list(c.s.layer_len)) for c in (a[0], b[0])] == before
    with pytest.raises(ValueError, match="keys/values"):
        KrillKernels.paged_decode_attention(q, [a[0], b[0]], 0.1, keys=kv[:, :1], values=kv[:, :1])
    assert [(p.seq_length(c.s.seq), list(c.s.layer_len)) for c in (a[0], b[0])] == before
    with pytest.raises(Exception):
        KrillKernels.quantize_append([a[0], b[0]], torch.zeros((2, 2, 3, 128), dtype=torch.bfloat16),
                                     torch.zeros((2, 2, 3, 128), dtype=torch.bfloat16))
    assert [(p.seq_length(c.s.seq), list(c.s.layer_len)) for c in (a[0], b[0])] == before
    p.close()


def test_krill_kernels_tables_cover_a_layer_behind_its_sequence():
    """The table width follows the blocks each sequence holds, not the layer's
    length: layer 1 two blocks behind layer 0 still gets whole tables."""
    from krill_amd.cache import make_quantized_kv_caches
    from krill_amd.kernels import _tables

    torch = pytest.importorskip("torch")
    p = host_pool()
    c0, c1 = make_quantized_kv_caches(p)
    c0.s.slots_for(0, 200)
    c0.s.layer_len[0] += 200
    c1.s.layer_len[1] = 60  # as a restore of a 60-token snapshot into layer 1 leaves it
    t, lens, mx = _tables(p, [c1], "cpu")
    assert t.shape == (1, 4) and int(lens[0]) == 60 and mx == 60
    np.testing.assert_array_equal(t.numpy()[0], p.block_table(c0.s.seq))
    t, lens, mx = _tables(p, [c1], "cpu", extra=1)
    assert t.shape == (1, 4) and int(lens[0]) == 61
    p.close()
