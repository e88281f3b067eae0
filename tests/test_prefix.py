"""The reference's ten PrefixCache tests (crates/qubivex-kv-cache/src/lib.rs:225-378),
run against the library's index (qvkv_prefix_*) and the oracle's restatement; plus the
paged form of a hit (fork + shared blocks) on a host-only pool."""
import numpy as np
import pytest

from oracle.pool_ref import MIN_REUSE, PrefixCacheRef


def cxx(budget):
    from qubivex_amd import PrefixCache

    return PrefixCache(budget)


class RefAdapter:
    def __init__(self, budget):
        self.c = PrefixCacheRef(budget)

    def lookup(self, scope, prompt):
        return self.c.lookup(scope, list(prompt))

    def insert(self, scope, tokens, cost, value):
        return self.c.insert(scope, list(tokens), cost, value)

    def evict_oldest(self):
        return self.c.evict_oldest()

    def clear(self):
        self.c.clear()

    def cost(self):
        return self.c.stats["cost"]

    def stats(self):
        return dict(self.c.stats)


IMPLS = [pytest.param(cxx, id="libqvkv"), pytest.param(RefAdapter, id="restated")]


def run(start, n):
    return list(range(start, start + n))


N = MIN_REUSE * 2


@pytest.mark.parametrize("make", IMPLS)
def test_the_longest_shared_prefix_wins(make):
    c = make(100)
    long = run(0, N)
    short = long[:N - 4] + [9999]
    assert c.insert(None, short, 1, "short")
    assert c.insert(None, long, 1, "long")
    assert c.lookup(None, long + [7, 8]) == ("long", N)
    other = long[:N - 8] + [1, 2, 3]
    assert c.lookup(None, other)[1] == N - 8


@pytest.mark.parametrize("make", IMPLS)
def test_the_last_token_always_runs(make):
    c = make(100)
    t = run(0, N)
    c.insert(None, t, 1, ())
    assert c.lookup(None, t)[1] == N - 1
    assert c.lookup(None, t[:N - 3])[1] == N - 4
    assert c.lookup(None, []) is None


@pytest.mark.parametrize("make", IMPLS)
def test_short_matches_are_not_worth_a_copy(make):
    c = make(100)
    assert not c.insert(None, run(0, MIN_REUSE - 1), 1, ())
    assert c.stats()["entries"] == 0
    c.insert(None, run(0, N), 1, ())
    assert c.lookup(None, run(0, MIN_REUSE - 1) + [9999, 9998]) is None
    assert c.lookup(None, run(0, MIN_REUSE) + [9999])[1] == MIN_REUSE


@pytest.mark.parametrize("make", IMPLS)
def test_scopes_never_see_each_other(make):
    c = make(100)
    t = run(0, N)
    c.insert("a", t, 1, "a")
    assert c.lookup("b", t) is None
    assert c.lookup(None, t) is None
    assert c.insert("b", t, 1, "b")
    assert c.insert(None, t, 1, "none")
    assert c.stats()["entries"] == 3
    assert c.lookup("b", t)[0] == "b"
    assert c.lookup(None, t)[0] == "none"


@pytest.mark.parametrize("make", IMPLS)
def test_the_budget_holds_and_the_least_recently_used_goes_first(make):
    c = make(3)
    a, b, d = run(0, N), run(1000, N), run(2000, N)
    c.insert(None, a, 1, "a")
    c.insert(None, b, 1, "b")
    c.insert(None, run(3000, N), 1, "c")
    assert c.lookup(None, a) is not None  # touching a leaves b the oldest
    c.insert(None, d, 1, "d")
    assert c.cost() == 3
    assert c.lookup(None, b) is None
    assert c.lookup(None, a) is not None
    assert c.lookup(None, d) is not None
    assert c.insert(None, run(4000, N), 3, "e")
    assert c.stats()["entries"] == 1
    assert c.stats()["evicted"] == 4


@pytest.mark.parametrize("make", IMPLS)
def test_a_value_over_budget_is_refused_and_evicts_nothing(make):
    c = make(3)
    a = run(0, N)
    c.insert(None, a, 3, ())
    assert not c.insert(None, run(1000, N), 4, ())
    assert c.lookup(None, a) is not None
    assert c.stats()["evicted"] == 0


@pytest.mark.parametrize("make", IMPLS)
def test_a_conversation_holds_one_entry(make):
    c = make(10)
    long = run(0, N + 10)
    assert c.insert(None, long[:N], 2, 1)
    assert c.insert(None, long, 3, 2)
    s = c.stats()
    assert (s["entries"], c.cost(), s["evicted"]) == (1, 3, 0)
    assert not c.insert(None, long[:N], 2, 3)
    assert c.lookup(None, long)[0] == 2
    branch = long[:N] + [9999]
    assert c.insert(None, branch, 2, 4)
    assert c.stats()["entries"] == 2


@pytest.mark.parametrize("make", IMPLS)
def test_a_replaced_value_makes_room_before_anything_older_is_evicted(make):
    c = make(4)
    old, turn = run(1000, N), run(0, N + 4)
    c.insert(None, old, 2, ())
    c.insert(None, turn[:N], 2, ())
    assert c.insert(None, turn, 2, ())
    assert c.lookup(None, old) is not None


@pytest.mark.parametrize("make", IMPLS)
def test_a_hit_outlives_its_eviction(make):
    c = make(10)
    t = run(0, N)
    c.insert(None, t, 1, [1, 2, 3])
    hit = c.lookup(None, t)
    c.clear()
    assert c.cost() == 0
    assert hit[0] == [1, 2, 3]


@pytest.mark.parametrize("make", IMPLS)
def test_counters_add_up(make):
    c = make(10)
    t = run(0, N)
    assert c.lookup(None, t) is None
    c.insert(None, t, 2, ())
    assert c.lookup(None, t) is not None
    s = c.stats()
    assert (s["lookups"], s["hits"], s["tokens_reused"], s["inserted"]) == (2, 1, N - 1, 1)
    c.clear()
    assert c.stats()["evicted"] == 1
    assert not c.evict_oldest()


def test_dropped_values_are_handed_back():
    c = cxx(4)
    c.insert(None, run(0, N), 2, "x")
    c.insert(None, run(0, N + 1), 2, "y")  # replaces x
    c.insert(None, run(500, N), 2, "z")
    c.insert(None, run(900, N), 2, "w")  # evicts y (oldest)
    assert c.take_dropped() == ["x", "y"]
    c.clear()
    assert sorted(c.take_dropped()) == ["w", "z"]


def test_a_hit_is_a_fork_that_shares_blocks():
    """Paged prefix reuse: retain a finished sequence in the index; a later prompt's hit
    forks it, sharing every full block; the index's eviction releases the retained
    sequence but the fork keeps its blocks (the hit outlives its eviction)."""
    from qubivex_amd import KvLayout, KvPool

    B = 16
    pool = KvPool(None, KvLayout("f16", 2, 32, B), 64, 1)
    c = cxx(100)
    done = pool.create()
    tokens = run(0, 100)
    pool.plan_append([done], [100], 0)
    assert c.insert(None, tokens, (100 + B - 1) // B, done)
    hit = c.lookup(None, tokens[:80] + [7, 7, 7])
    assert hit is not None and hit[1] == 80
    seq = pool.fork(hit[0], hit[1])
    shared = pool.tables([seq], 0)[0]
    assert shared.tolist() == pool.tables([done], 0)[0][:5].tolist()
    assert all(pool.refcount(int(b)) == 2 for b in shared)
    c.clear()
    for v in c.take_dropped():
        pool.release(v)
    assert all(pool.refcount(int(b)) == 1 for b in shared)
    assert pool.stats()["free"] == 64 - 5
    pool.release(seq)
    assert pool.stats()["free"] == 64
