"""The page pool against tessera-kv's own tests (engine/ir/kv/src/pool_test.rs),
transcribed, plus the reference's randomized call sequence with its digest check
and the consistency invariant after every call."""
import pytest

from tessera_amd.kv import Pool, PoolError

T = 0


def err(fn, *a):
    with pytest.raises(PoolError) as e:
        fn(*a)
    return e.value


def test_admission_counts_worst():
    pool = Pool(4, 2)
    a = pool.reserve(T, 1, 6)
    e = err(pool.reserve, T, 1, 4)
    assert (e.name(), e.value) == ("NoRoom", 2)
    s = pool.stats()
    assert (s.size, s.active, s.worst) == (8, 2, 6)
    pool.retain(a)
    s = pool.stats()
    assert (s.live_runs, s.kept_runs, s.active) == (0, 1, 0)
    pool.release(a)
    pool.reserve(T, 1, 8)


def test_shared_writes_copy():
    pool = Pool(8, 2)
    a = pool.reserve(T, 3, 6)
    b = pool.fork(a, 3, 6)
    first, last = pool.pages(a)
    copies = pool.grow(b, 4)
    to = copies[0][1]
    assert copies == [(last, to, 1)]
    assert pool.pages(b) == [first, to]
    assert pool.grow(a, 4) == []


def test_retained_rows_fork():
    pool = Pool(4, 2)
    a = pool.reserve(T, 3, 8)
    pool.grow(a, 8)
    pool.truncate(a, 3)
    pool.retain(a)
    b = pool.fork(a, 3, 4)
    assert pool.pages(b) == pool.pages(a)
    pool.release(b)
    pool.reserve(T, 8, 8)
    assert err(pool.pages, a).name() == "Unknown"


def test_full_pool_adopts():
    pool = Pool(2, 4)
    a = pool.reserve(T, 3, 4)
    pool.reserve(T, 3, 4)
    pool.retain(a)
    e = err(pool.fork, a, 2, 4)
    assert (e.name(), e.value) == ("NoRoom", 1)
    page = pool.pages(a)
    b = pool.adopt(a, 2, 4)
    assert err(pool.adopt, b, 2, 4).name() == "Live"
    assert (pool.pages(b), pool.rows(b)) == (page, 2)
    assert err(pool.rows, a).name() == "Unknown"
    pool.grow(b, 4)


def test_lowest_free_page_first():
    pool = Pool(8, 16)
    a = pool.reserve(T, 40, 96)
    # Room is checked against every live run's worst case: 6 promised + 3 > 8 refuses.
    e = err(pool.reserve, T, 16, 48)
    assert (e.name(), e.value) == ("NoRoom", 3)
    assert pool.pages(a) == [0, 1, 2]
    b = pool.reserve(T, 16, 16)
    assert pool.pages(b) == [3]
    pool.release(a)
    pool.grow(b, 16)
    c = pool.reserve(T, 33, 48)
    assert pool.pages(c) == [0, 1, 2]
    e = err(pool.grow, c, 49)
    assert (e.name(), e.value, e.value2) == ("PastWorst", 49, 48)


def test_random_calls():
    """pool_test.rs random_calls: 1000 seeded calls on small pools; a refused call
    leaves the digest unchanged, and the pool stays consistent."""
    M = (1 << 64) - 1
    for pages in [4, 6, 8, 12]:
        for seed in range(1, 5):
            pool = Pool(pages, 4)
            runs = []
            for _ in range(1000):
                seed = (seed * 6364136223846793005 + 1) & M
                pick = seed >> 33
                run = runs[pick // 8 % max(len(runs), 1)] if runs else None
                before = pool.digest()
                op = pick % 7
                try:
                    if op == 1 and run is not None:
                        runs.append(pool.fork(run, pick % 9, 16))
                    elif op == 2 and run is not None:
                        pool.grow(run, pick % 17)
                    elif op == 3 and run is not None:
                        pool.truncate(run, pick % 9)
                    elif op == 4 and run is not None:
                        pool.retain(run)
                    elif op == 5 and run is not None:
                        pool.release(run)
                        runs = [o for o in runs if o != run]
                    elif op == 6 and run is not None:
                        n = pool.adopt(run, pick % 9, 16)
                        runs = [o for o in runs if o != run] + [n]
                    else:
                        runs.append(pool.reserve(T, pick % 9, 8 + pick % 9))
                except PoolError:
                    assert pool.digest() == before
                assert pool.consistent()


def test_copy_pages_refuses_overlap_on_the_host():
    """Two copies where one's target is the other's source (or target) are refused
    before anything reaches a device."""
    import pytest
    torch = pytest.importorskip("torch")
    from tessera_amd import kv
    K = torch.zeros((8 * 16, 4), dtype=torch.int32)
    with pytest.raises(ValueError, match="overlap"):
        kv.copy_pages([K], [(1, 2, 4), (2, 3, 4)], page=16, pages=8)
    with pytest.raises(ValueError, match="overlap"):
        kv.copy_pages([K], [(1, 3, 4), (2, 3, 4)], page=16, pages=8)
