"""The host pool manager (block pool, block tables, sharing, COW, eviction, compaction) on
a host-only pool: no GPU.  Block copies the pool issues are applied to the oracle's
simulated pool, so every check is on the logical keys and values each sequence reads."""
import ctypes

import numpy as np
import pytest

import oracle
from oracle.pool_ref import KvPoolRef, SeqRef, after_run, attention_plan

B = 16


def layout(dtype="f16", G=2, D=32):
    from qubivex_amd import KvLayout

    return KvLayout(dtype, G, D, B)


def host_pool(n_blocks, n_layers=1, **kw):
    from qubivex_amd import KvPool

    return KvPool(None, layout(**kw), n_blocks, n_layers)


class Data:
    """Logical content of a host-only pool: the oracle's SimPool plus the copy batches."""

    def __init__(self, pool):
        L = pool.layout
        self.pool = pool
        self.sim = oracle.SimPool(pool.n_blocks, L.kv_heads, L.head_dim, L.block, oracle.F16)
        self.r = np.random.default_rng(99)

    def sync_copies(self, batches=None):
        for src, dst in (self.pool.take_batches() if batches is None else batches):
            assert not set(src.tolist()) & set(dst.tolist()), "a batch reads what it writes"
            assert len(set(dst.tolist())) == dst.size, "a batch writes a block twice"
            w = 2 * self.sim.B * self.sim.kv_out
            blocks = self.sim.words.reshape(-1, w)
            blocks[dst] = blocks[src].copy()  # all reads of the batch, then all writes

    def append(self, seqs, counts, layer):
        slots = self.pool.plan_append(seqs, counts, layer)
        self.sync_copies()
        kv = self.sim.kv_out
        k = self.r.standard_normal((slots.size, kv)).astype(np.float32)
        v = self.r.standard_normal((slots.size, kv)).astype(np.float32)
        self.sim.store(k, v, slots)
        return slots

    def read(self, seq, layer=0):
        blocks, table_at, pos = self.pool.tables([seq], layer)
        return self.sim.gather(blocks, table_at, 0, int(pos[0]) + 1)


def test_free_list_hands_out_block_zero_first():
    """discrete.rs:446-449: (0..blocks).rev(), so pop() yields 0, 1, 2, ..."""
    p = host_pool(10)
    s = p.create()
    p.plan_append([s], [3 * B], 0)
    assert p.tables([s], 0)[0].tolist() == [0, 1, 2]
    p.release(s)
    s2 = p.create()
    p.plan_append([s2], [1], 0)
    # released blocks go back on top in table order: the last pushed (2) comes first
    assert p.tables([s2], 0)[0].tolist() == [2]


def test_tables_follow_attention_plan_restated():
    """Random decode schedule: the C++ pool's tables equal those of the restated
    attention_plan (crates/qubivex-runtime/src/discrete.rs:951-1009), releases included."""
    r = np.random.default_rng(1)
    n_blocks, n_layers = 6000, 3
    p = host_pool(n_blocks, n_layers)
    ref = KvPoolRef(n_blocks, B)
    live = {}  # c++ handle -> SeqRef
    for step in range(200):
        if len(live) < 6 and r.random() < 0.3:
            live[p.create()] = SeqRef()
        if live and r.random() < 0.05:
            h = list(live)[int(r.integers(len(live)))]
            p.release(h)
            live.pop(h).mirror.release()
        if not live:
            continue
        handles = sorted(live)
        grow = {h: int(r.integers(1, 40)) for h in handles}
        for layer in range(n_layers):
            seqs = [live[h] for h in handles]
            for h in handles:
                live[h].pos = p.length(h, 0) + grow[h] - 1 if layer == 0 else live[h].pos
            for q in seqs:
                q.host_k = q.host_v = [np.zeros(0)] * 0
            plan = attention_plan(ref, seqs, 0, 0, layer)
            assert plan is not None
            after_run(ref, seqs, layer, plan)
            p.plan_append(handles, [live[h].pos + 1 - p.length(h, layer) for h in handles], layer)
            blocks, table_at, pos = p.tables(handles, layer)
            assert blocks.tolist() == plan["blocks"]
            assert table_at.tolist() == plan["table_at"]
            assert pos.tolist() == plan["pos"]
        # every layer's tables in one call: the per-layer tables, layer after layer
        ab, at, ap = p.tables_layers(handles, 0, n_layers)
        off = 0
        for layer in range(n_layers):
            b1, t1, p1 = p.tables(handles, layer)
            k = len(handles)
            assert ab[off:off + b1.size].tolist() == b1.tolist()
            assert (at[layer * k:(layer + 1) * k] - off).tolist() == t1.tolist()
            assert ap[layer * k:(layer + 1) * k].tolist() == p1.tolist()
            off += b1.size
        assert ab.size == off
    assert p.stats()["free"] == len(ref.free)


def test_plan_attention_equals_restated_attention_plan():
    """Host-authoritative decode passes with prompts, decode steps, clears (epoch changes)
    and releases: blocks, table_at, pos and sync_to equal the restated attention_plan
    (crates/qubivex-runtime/src/discrete.rs:951-1009) pass for pass."""
    r = np.random.default_rng(11)
    n_blocks, n_layers = 5000, 2
    p = host_pool(n_blocks, n_layers)
    ref = KvPoolRef(n_blocks, B)
    live = {}  # handle -> [SeqRef, host positions held]
    for step in range(150):
        if len(live) < 5 and r.random() < 0.3:
            h = p.create()
            live[h] = [SeqRef(epoch=int(r.integers(0, 3))), int(r.integers(0, 100))]
        if live and r.random() < 0.05:  # a cache dropped: its mirror gives its blocks back
            h = list(live)[int(r.integers(len(live)))]
            p.release(h)
            q = live.pop(h)[0]
            if q.mirror is not None:
                q.mirror.release()  # the reference's Mirror drop
        if live and r.random() < 0.08:  # clear and refill: a new epoch
            h = list(live)[int(r.integers(len(live)))]
            live[h][0].epoch += 1
            live[h][1] = int(r.integers(0, 40))
        if not live:
            continue
        handles = sorted(live)
        for h in handles:  # this pass's token sits at the host's next position
            live[h][0].pos = live[h][1]
        for layer in range(n_layers):
            seqs = [live[h][0] for h in handles]
            for q in seqs:
                q.host_k = q.host_v = []
            want = attention_plan(ref, seqs, 0, 0, layer)
            assert want is not None
            after_run(ref, seqs, layer, want)
            got = p.plan_attention(handles, [live[h][0].pos for h in handles],
                                   [live[h][0].epoch for h in handles], layer)
            assert got["blocks"].tolist() == want["blocks"], (step, layer)
            assert got["table_at"].tolist() == want["table_at"]
            assert got["pos"].tolist() == want["pos"]
            assert got["sync_to"].tolist() == want["sync_to"], (step, layer)
        for h in handles:
            live[h][1] += 1  # the pass's token is now in the host cache
    assert p.stats()["free"] == len(ref.free)


def test_plan_attention_declines_the_layer_a_short_pool_cannot_hold():
    """crates/qubivex-runtime/tests/discrete.rs:735-760: a pool one block short of every
    layer declines that layer each step (`full`), and gives every block back on drop; the
    prompt's rows are copied in once per layer."""
    from qubivex_amd import OutOfDeviceMemory

    L, prompt, steps = 4, 5, 8  # every position stays inside one block per layer
    p = host_pool(L - 1, L)
    s = p.create()
    ran = 0
    for step in range(steps):
        pos = prompt + step
        for layer in range(L):
            try:
                p.plan_attention([s], [pos], [0], layer)
                ran += 1
            except OutOfDeviceMemory:
                assert layer == L - 1
    st = p.stats()
    assert (ran, st["full"]) == (steps * (L - 1), steps)
    assert st["synced_rows"] == prompt * (L - 1)  # the prompt, once per layer that ran
    assert st["allocated"] == 0  # a host-only pool holds no device memory (KvPoolStats)
    p.release(s)
    assert p.stats()["free"] == p.stats()["blocks"]


def test_plan_attention_epoch_restart_copies_the_new_rows_in():
    p = host_pool(32, 1)
    s = p.create()
    first = p.plan_attention([s], [40], [0], 0)
    assert first["sync_to"].size == 40 and p.stats()["free"] == 29
    again = p.plan_attention([s], [41], [0], 0)
    assert again["sync_to"].size == 0  # nothing new on the host side
    restarted = p.plan_attention([s], [5], [1], 0)  # the cache was cleared and refilled
    assert restarted["sync_to"].size == 5 and p.stats()["free"] == 31
    # the released blocks went back in table order, so the last one comes out first
    assert first["blocks"].tolist() == [0, 1, 2] and restarted["blocks"].tolist() == [2]


def test_every_block_returns_on_release():
    p = host_pool(64, 2)
    seqs = [p.create() for _ in range(4)]
    for layer in range(2):
        p.plan_append(seqs, [17, 40, 1, 100], layer)
    assert p.stats()["free"] == 64 - 2 * (2 + 3 + 1 + 7)
    for s in seqs:
        p.release(s)
    st = p.stats()
    assert st["free"] == st["blocks"] == 64
    assert st["synced_rows"] == 2 * (17 + 40 + 1 + 100)


def test_a_dry_pool_declines_and_changes_nothing():
    """A pool one block short: the call fails with OutOfDeviceMemory, counts `full`, and
    leaves every table as it was (discrete.rs:882-891)."""
    from qubivex_amd import OutOfDeviceMemory

    p = host_pool(5)
    a, b = p.create(), p.create()
    p.plan_append([a], [3 * B], 0)
    before = (p.tables([a], 0)[0].tolist(), p.stats()["free"])
    with pytest.raises(OutOfDeviceMemory):
        p.plan_append([a, b], [1, 2 * B], 0)  # needs 1 + 2, has 2
    assert p.stats()["full"] == 1
    assert (p.tables([a], 0)[0].tolist(), p.stats()["free"]) == before
    assert p.length(b, 0) == 0


def test_a_dry_pool_reports_requested_used_and_capacity():
    """QVKV_E_OOM carries ComputeError::OutOfDeviceMemory's fields
    (crates/qubivex-compute/src/lib.rs:64-75): the blocks asked for, the blocks in use and
    the pool, in bytes; a later failure of another kind clears them."""
    from qubivex_amd import OutOfDeviceMemory, ShapeError, _lib

    p = host_pool(5)
    bb = p.layout.block_bytes
    a, b = p.create(), p.create()
    p.plan_append([a], [3 * B], 0)
    with pytest.raises(OutOfDeviceMemory) as ei:
        p.plan_append([a, b], [1, 2 * B], 0)  # 3 blocks asked, 3 of 5 in use
    assert (ei.value.requested, ei.value.used, ei.value.capacity) == (3 * bb, 3 * bb, 5 * bb)
    with pytest.raises(ShapeError):
        p.plan_append([a], [1], 7)  # no such layer
    r, u, c = (ctypes.c_uint64(9) for _ in range(3))
    _lib.lib.qvkv_last_oom(ctypes.byref(r), ctypes.byref(u), ctypes.byref(c))
    assert (r.value, u.value, c.value) == (0, 0, 0)


def test_device_pools_order_their_copies_after_the_callers_stream(monkeypatch):
    """The binding hands the pool manager torch's current stream (or the one given), which
    the library's copy-on-write and compaction copies wait for; host-only pools pass none.
    (The device side, an event recorded on that stream and waited for by the copy, is
    exercised on the GPU by the copy-on-write configuration test.)"""
    from qubivex_amd import kv

    p = host_pool(64, 2)
    seen = []
    real = {n: getattr(kv.lib, n) for n in ("qvkv_pool_plan_append", "qvkv_pool_plan_attention",
                                            "qvkv_pool_compact")}

    def spy(name):
        def f(*args):
            seen.append((name, args[-1]))
            return real[name](*args)
        return f

    for n in real:
        monkeypatch.setattr(kv.lib, n, spy(n))
    s = p.create()
    p.plan_append([s], [5], 0)
    p.compact()
    assert [a for _, a in seen] == [None, None]
    seen.clear()
    fake = ctypes.c_void_p(0xABC0)
    monkeypatch.setattr(kv, "_stream", lambda stream: fake if stream is None else stream)
    p.dev = "a device"  # the Python side only: the C pool stays host-only
    p.plan_append([s], [5], 0)
    p.plan_attention([s], [12], [0], 1)
    p.compact()
    mine = ctypes.c_void_p(0xDEF0)
    p.plan_append([s], [1], 0, stream=mine)
    assert [a.value for _, a in seen] == [0xABC0, 0xABC0, 0xABC0, 0xDEF0]
    p.dev = None


def test_fork_shares_blocks_and_copies_on_write():
    p = host_pool(64, 2)
    data = Data(p)
    parent = p.create()
    P = 2 * B + 7  # the last block partially filled
    for layer in range(2):
        data.append([parent], [P], layer)
    want = [data.read(parent, layer) for layer in range(2)]
    kids = [p.fork(parent, P) for _ in range(3)]
    pblocks = p.tables([parent], 0)[0]
    assert all(p.refcount(int(b)) == 4 for b in pblocks)
    assert p.stats()["shared_blocks"] == 2 * 3
    free_before = p.stats()["free"]
    # every child writes its own next tokens: each copies the shared partial block first
    for i, kid in enumerate(kids):
        data.append([kid], [3 + i], 0)
    st = p.stats()
    assert st["cow_copies"] == 3 and st["free"] == free_before - 3
    assert p.refcount(int(pblocks[-1])) == 1  # only the parent still holds it
    for i, kid in enumerate(kids):
        k, v = data.read(kid, 0)
        assert np.array_equal(k[:, :P], want[0][0]) and np.array_equal(v[:, :P], want[0][1])
        kb = p.tables([kid], 0)[0]
        assert kb[:2].tolist() == pblocks[:2].tolist() and kb[2] != pblocks[2]
    # the parent's reads never changed
    k, v = data.read(parent, 0)
    assert np.array_equal(k, want[0][0]) and np.array_equal(v, want[0][1])
    # the parent writes into its partial block on layer 1, still shared by 3 children
    data.append([parent], [2], 1)
    assert p.stats()["cow_copies"] == 4
    for kid in kids:
        k, _ = data.read(kid, 1)
        assert np.array_equal(k, want[1][0])
    # a block-aligned fork never copies
    q = p.fork(parent, 2 * B)
    data.append([q], [5], 0)
    assert p.stats()["cow_copies"] == 4
    for s in kids + [parent, q]:
        p.release(s)
    assert p.stats()["free"] == 64


def test_fork_of_the_same_block_by_two_writers_in_one_plan():
    """Two children in one plan both copy; the parent, last holder, would not."""
    p = host_pool(32)
    data = Data(p)
    parent = p.create()
    data.append([parent], [B + 5], 0)
    a, b = p.fork(parent, B + 5), p.fork(parent, B + 5)
    data.append([a, b, parent], [1, 1, 1], 0)
    assert p.stats()["cow_copies"] == 2
    want = data.read(parent, 0)[0][:, :B + 5]
    for s in (a, b):
        assert np.array_equal(data.read(s, 0)[0][:, :B + 5], want)


def test_lru_eviction_releases_the_oldest_first():
    p = host_pool(128)
    seqs = [p.create() for _ in range(5)]
    for s in seqs:
        p.plan_append([s], [2 * B], 0)
    p.touch(seqs[0])  # now the newest
    released = p.evict_lru(5)  # 2 blocks each: three sequences
    assert released == [seqs[1], seqs[2], seqs[3]]
    assert p.stats()["evicted_blocks"] == 6
    # a block shared with a survivor is not freed by the eviction of one holder
    kid = p.fork(seqs[4], B)
    p.touch(kid)
    free = p.stats()["free"]
    assert p.evict_lru(1) == [seqs[4]]
    assert p.stats()["free"] == free + 1  # its second block only; the first is the kid's


@pytest.mark.parametrize("mode", ["permute", "fill"])
@pytest.mark.parametrize("seed", [0, 1, 7, 12345])
def test_compaction_moves_live_blocks_to_the_front(seed, mode):
    r = np.random.default_rng(seed + 3)
    p = host_pool(300, 2)
    data = Data(p)
    seqs = [p.create() for _ in range(12)]
    for layer in range(2):
        for s in seqs:
            data.append([s], [int(r.integers(1, 120))], layer)
    kids = [p.fork(seqs[i], min(p.length(seqs[i], 0), p.length(seqs[i], 1)) // 2 + 1)
            for i in range(3)]
    for k in kids:
        data.append([k], [int(r.integers(1, 30))], 0)
        data.append([k], [1], 1)
    for s in seqs[::3]:
        p.release(s)
    live = [s for s in seqs if s not in seqs[::3]] + kids
    before = {(s, l): data.read(s, l) for s in live for l in range(2)}
    refs_before = sorted(p.refcount(b) for b in range(300) if p.refcount(b))
    K = len(refs_before)
    above = sum(1 for b in range(K, 300) if p.refcount(b))
    stay = {b: p.refcount(b) for b in range(K) if p.refcount(b)}
    moved = p.compact(seed, mode=mode)
    if mode == "fill":
        # the fewest moves (only blocks past the live count), one launch, nothing below K moved
        batches = p.take_batches()
        assert moved == above and len(batches) == 1 and len(batches[0][0]) == above
        assert all(int(x) >= K for x in batches[0][0]) and all(int(x) < K for x in batches[0][1])
        assert all(p.refcount(b) == r for b, r in stay.items())
        data.sync_copies(batches)
    data.sync_copies()
    assert sorted(p.refcount(b) for b in range(K)) == refs_before
    assert all(p.refcount(b) == 0 for b in range(K, 300))
    assert p.stats()["moved_blocks"] == moved and moved > 0
    for (s, l), (k, v) in before.items():
        k2, v2 = data.read(s, l)
        assert np.array_equal(k, k2) and np.array_equal(v, v2), (s, l)
        assert p.tables([s], l)[0].max() < K
    # the next block handed out is the first free one after the live ones
    n = p.create()
    p.plan_append([n], [1], 0)
    assert p.tables([n], 0)[0].tolist() == [K]


def test_compaction_of_a_full_pool_with_cycles_needs_a_spare():
    from qubivex_amd import OutOfDeviceMemory

    p = host_pool(8)
    s = p.create()
    p.plan_append([s], [8 * B], 0)
    with pytest.raises(OutOfDeviceMemory):
        p.compact(seed=5)  # a permutation of a full pool has cycles and no spare
    assert p.compact(seed=0) == 0  # ascending order: nothing to move


def test_plan_over_layers_equals_per_layer_plans_in_one_batch():
    """qvkv_pool_plan_append_layers gives the slots and copy-on-write pairs of one
    plan_append per layer (layer-major), with every layer's copies in one batch; on a dry
    pool it fails with nothing changed."""
    from qubivex_amd import OutOfDeviceMemory

    NL = 3
    a, b = host_pool(200, NL), host_pool(200, NL)
    for p in (a, b):
        par = p.create()
        for l in range(NL):
            p.plan_append([par], [2 * B + 5], l)  # a shared partial last block per layer
        kids = [p.fork(par, 2 * B + 5) for _ in range(3)]
        p.take_batches()
    kids = [1, 2, 3]
    counts = [4, 20, 1]
    per_layer = np.concatenate([a.plan_append(kids, counts, l) for l in range(NL)])
    batches_a = a.take_batches()
    together = b.plan_append_layers(kids, counts, 0, NL)
    batches_b = b.take_batches()
    assert np.array_equal(per_layer, together)
    assert len(batches_a) == NL and len(batches_b) == 1
    assert np.array_equal(np.concatenate([s for s, _ in batches_a]), batches_b[0][0])
    assert np.array_equal(np.concatenate([d for _, d in batches_a]), batches_b[0][1])
    for l in range(NL):
        assert [x.tolist() for x in a.tables(kids, l)] == [x.tolist() for x in b.tables(kids, l)]
    # dry: the last layer cannot grow, so no layer changes
    before = [b.tables(kids, l)[0].tolist() for l in range(NL)], b.stats()["free"]
    with pytest.raises(OutOfDeviceMemory):
        b.plan_append_layers(kids, [B * 60] * 3, 0, NL)
    assert ([b.tables(kids, l)[0].tolist() for l in range(NL)], b.stats()["free"]) == before


def test_zero_counts_and_empty_plans_change_nothing():
    """Plans over no sequences, or with zero new positions, take no block and issue no
    copy; a fork of zero positions shares nothing."""
    p = host_pool(16, 2)
    s = p.create()
    assert p.plan_append([], [], 0).size == 0
    assert p.plan_append([s], [0], 1).size == 0
    assert p.plan_append_layers([s], [0], 0, 2).size == 0
    assert p.stats()["free"] == 16 and p.take_batches() == []
    p.plan_append([s], [B + 3], 0)
    kid = p.fork(s, 0)
    assert p.length(kid, 0) == 0 and p.stats()["shared_blocks"] == 0
    assert p.compact(mode="fill") == 0 and p.compact() == 0  # live blocks are 0 and 1 already
