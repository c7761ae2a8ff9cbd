"""Block metadata: the free stack / refcounts of PagedBlockPool and BlockTable.

The reference's own tests are replayed against both the product host
metadata (libglacier_paged.so, host-only entry points) and the oracle's
restatement, and the two are then required to produce bit-identical tables
under long seeded admit/evict churn.
"""
import numpy as np
import pytest

import glacier_oracle as orc
import glacier_paged as gp
import workloads


class ProductImpl:
    name = "product"

    @staticmethod
    def alloc(n, bs=16):
        return gp.BlockAllocator(n, bs)

    @staticmethod
    def table(a):
        return gp.BlockTable(a)

    Range = gp.InvalidArgument


class OracleImpl:
    name = "oracle"

    @staticmethod
    def alloc(n, bs=16):
        return orc.Alloc(n, bs)

    @staticmethod
    def table(a):
        return orc.BTab(a)

    Range = orc.ArgumentOutOfRange


IMPLS = [ProductImpl, OracleImpl]


@pytest.fixture(params=IMPLS, ids=lambda c: c.name)
def impl(request):
    return request.param


def test_allocates_and_recycles(impl):
    """PagedAttentionTests.cs:10-34."""
    pool = impl.alloc(64)
    assert pool.free_blocks_count == 64
    got = []
    for _ in range(10):
        ok, b = pool.try_allocate_block()
        assert ok
        got.append(b)
    assert pool.free_blocks_count == 54
    for b in got:
        pool.release_block(b)
    assert pool.free_blocks_count == 64


def test_first_pop_is_block_zero_lifo(impl):
    """Constructor pushes total-1..0 (PagedBlockPool.cs:116-120): pops come out 0, 1, 2 ..."""
    pool = impl.alloc(8)
    assert [pool.try_allocate_block()[1] for _ in range(3)] == [0, 1, 2]
    pool.release_block(1)
    assert pool.try_allocate_block()[1] == 1  # last freed is next allocated


def test_block_table_expands_across_boundaries(impl):
    """PagedAttentionTests.cs:36-79: 35 tokens -> 3 blocks, offsets t % 16, 13 free."""
    pool = impl.alloc(16)
    t = impl.table(pool)
    for i in range(35):
        ok, b, off = t.append_token()
        assert ok and b >= 0 and off == i % 16
    assert t.token_count == 35
    span = t.as_span()
    assert len(span) == 3
    assert pool.free_blocks_count == 13
    assert list(span) == [0, 1, 2]
    t.release_all()
    assert t.token_count == 0 and len(t.as_span()) == 0
    assert pool.free_blocks_count == 16


def test_double_free_and_exhaustion(impl):
    """PhaseCServeRemediationTests.cs:69-111."""
    pool = impl.alloc(8)
    _, b0 = pool.try_allocate_block()
    _, b1 = pool.try_allocate_block()
    assert b0 != b1 and pool.free_blocks_count == 6
    pool.release_block(b0)
    assert pool.free_blocks_count == 7
    pool.release_block(b0)
    assert pool.free_blocks_count == 7
    for c in range(8):
        if c != b1:
            pool.release_block(c)
    assert pool.free_blocks_count == 7
    seen = {b1}
    for _ in range(7):
        ok, n = pool.try_allocate_block()
        assert ok and n not in seen
        seen.add(n)
    ok, n = pool.try_allocate_block()
    assert not ok and n == -1


def test_refcounts(impl):
    """PrefixHashKvCacheTests.cs:53-84."""
    pool = impl.alloc(8)
    _, b = pool.try_allocate_block()
    assert pool.get_ref_count(b) == 1
    assert pool.retain_block(b) == 2
    assert pool.retain_block(b) == 3
    assert pool.release_block(b) == 2
    assert pool.release_block(b) == 1
    assert pool.free_blocks_count == 7
    assert pool.release_block(b) == 0
    assert pool.free_blocks_count == 8


def test_out_of_range_ids(impl):
    """PrefixHashKvCacheAdversarialTests.cs:352-366."""
    pool = impl.alloc(4)
    assert pool.release_block(-1) == 0
    assert pool.release_block(100) == 0
    assert pool.get_ref_count(-1) == 0
    assert pool.get_ref_count(100) == 0
    with pytest.raises(impl.Range):
        pool.retain_block(-1)
    with pytest.raises(impl.Range):
        pool.retain_block(100)


def test_double_release_idempotent(impl):
    """PrefixHashKvCacheAdversarialTests.cs:325-350."""
    pool = impl.alloc(4)
    _, b = pool.try_allocate_block()
    assert pool.release_block(b) == 0
    assert pool.free_blocks_count == 4
    assert pool.release_block(b) == 0
    assert pool.free_blocks_count == 4
    for _ in range(4):
        assert pool.try_allocate_block()[0]
    assert pool.free_blocks_count == 0


def test_cow_fork_under_oom_leaves_state(impl):
    """PrefixHashKvCacheAdversarialTests.cs:109-141."""
    pool = impl.alloc(1)
    _, b0 = pool.try_allocate_block()
    pool.retain_block(b0)
    ta = impl.table(pool)
    ta.attach_prefix_blocks([b0], 4)
    tb = impl.table(pool)
    tb.attach_prefix_blocks([b0], 4)
    ok, b, off = ta.append_token()
    assert (ok, b, off) == (False, -1, -1)
    assert ta.token_count == 4 and list(ta.as_span()) == [b0]
    assert pool.get_ref_count(b0) == 2
    ta.release_all()
    assert pool.get_ref_count(b0) == 1
    tb.release_all()
    assert pool.get_ref_count(b0) == 0 and pool.free_blocks_count == 1


def test_cow_fork_swaps_block(impl):
    """PrefixHashKvCacheTests.cs:134-181 (metadata half; the page copy is a GPU test)."""
    pool = impl.alloc(16)
    ta = impl.table(pool)
    for _ in range(10):
        assert ta.append_token()[0]
    shared = ta.as_span()[0]
    pool.retain_block(shared)
    tb = impl.table(pool)
    tb.attach_prefix_blocks([shared], 10)
    assert pool.get_ref_count(shared) == 2
    ok, forked, off = ta.append_token()
    assert ok and off == 10 and forked != shared
    assert pool.get_ref_count(shared) == 1 and pool.get_ref_count(forked) == 1
    ta.release_all()
    tb.release_all()
    assert pool.free_blocks_count == 16


def test_attach_prefix(impl):
    """PrefixHashKvCacheTests.cs:183-200."""
    pool = impl.alloc(16)
    _, b0 = pool.try_allocate_block()
    _, b1 = pool.try_allocate_block()
    t = impl.table(pool)
    t.attach_prefix_blocks([b0, b1], 32)
    assert t.token_count == 32 and list(t.as_span()) == [b0, b1]
    t.release_all()
    assert pool.free_blocks_count == 16


def test_concurrent_sequences_no_leak(impl):
    """ContinuousBatchingLoadChallengeTests.cs:390-439: 10 sequences x 64 tokens -> 4 blocks each."""
    pool = impl.alloc(64)
    tabs = [impl.table(pool) for _ in range(10)]
    for _ in range(64):
        for t in tabs:
            assert t.append_token()[0]
    assert all(len(t.as_span()) == 4 for t in tabs)
    assert pool.free_blocks_count == 24
    for t in tabs:
        t.release_all()
    assert pool.free_blocks_count == 64


def test_product_matches_oracle_under_churn():
    """Bit-identical tables from the product and the oracle on seeded admit/evict/COW churn."""
    rng_ops = np.random.default_rng(1234)
    ops = rng_ops.integers(0, 100, size=4000)
    lens = rng_ops.integers(1, 90, size=4000)
    picks = rng_ops.integers(0, 1 << 30, size=4000)

    def run(impl):
        pool = impl.alloc(300)
        live = []
        log = []
        for op, n, pick in zip(ops, lens, picks):
            if op < 45 or not live:
                t = impl.table(pool)
                got = t.append_tokens(int(n))
                log.append(("admit", got))
                live.append(t)
            elif op < 75:
                t = live[pick % len(live)]
                log.append(("append",) + t.append_token())
            elif op < 90:
                t = live.pop(pick % len(live))
                t.release_all()
                log.append(("evict",))
            else:  # share the first page of one sequence with a new one (prefix attach)
                src = live[pick % len(live)]
                span = src.as_span()
                if len(span):
                    pool.retain_block(int(span[0]))
                    t = impl.table(pool)
                    t.attach_prefix_blocks([int(span[0])], min(src.token_count, 16) // 2 + 1)
                    live.append(t)
                    log.append(("share", int(span[0])))
        state = [(t.token_count, tuple(t.as_span())) for t in live]
        return log, state, pool.free_blocks_count

    assert run(ProductImpl) == run(OracleImpl)


def test_llama8b_tables_product_equals_oracle():
    """The fragmented 2000-step tables of the llama8b_decode step, bit-exact across implementations."""
    prod = workloads.llama8b_decode(steps=600, make_alloc=ProductImpl.alloc, make_table=ProductImpl.table)
    ref = workloads.llama8b_decode(steps=600, make_alloc=OracleImpl.alloc, make_table=OracleImpl.table)
    assert np.array_equal(prod.bt_offsets, ref.bt_offsets)
    assert np.array_equal(prod.bt_ids, ref.bt_ids)
    assert np.array_equal(prod.token_counts, ref.token_counts)
    assert prod.num_rows == 256
    # Fragmented: pages of a row are not a contiguous run.
    runs = [np.all(np.diff(prod.table(b)) == 1) for b in range(prod.num_rows) if len(prod.table(b)) > 1]
    assert not all(runs)


def test_append_token_on_an_empty_partial_table_raises():
    """AttachPrefixBlocks accepts any token count (BlockTable.cs:31-39); the next
    AppendToken inside a page then reads _physicalBlockIds[^1] and throws when the
    table holds no page (:60).  The product raises InvalidArgument and leaves the
    table and the pool unchanged, where it once read past an empty vector."""
    a = gp.BlockAllocator(8, 16)
    t = gp.BlockTable(a)
    t.attach_prefix_blocks([], 5)
    with pytest.raises(gp.InvalidArgument):
        t.append_token()
    assert t.token_count == 5 and t.block_count == 0 and a.free_blocks_count == 8
    assert t.append_tokens(3) == 0
    # At a page boundary an empty table simply allocates, as in the reference.
    t2 = gp.BlockTable(a)
    t2.attach_prefix_blocks([], 16)
    ok, b, off = t2.append_token()
    assert ok and b == 0 and off == 0 and t2.token_count == 17


def test_append_token_null_arguments_are_errors_not_exhaustion():
    """A NULL output pointer is an invalid argument (-1 with GSP_E_INVALID_ARG), never the 0 that
    means the pool is exhausted; the table and the pool stay unchanged."""
    import ctypes

    a = gp.BlockAllocator(4, 16)
    t = gp.BlockTable(a)
    lib = gp.load()
    b = ctypes.c_int32()
    assert lib.gsp_block_table_append_token(t._h, None, ctypes.byref(b)) == -1
    assert lib.gsp_block_table_append_token(t._h, ctypes.byref(b), None) == -1
    assert lib.gsp_block_table_append_token(None, ctypes.byref(b), ctypes.byref(b)) == -1
    assert t.token_count == 0 and t.block_count == 0 and a.free_blocks_count == 4
    assert t.append_token()[0]
