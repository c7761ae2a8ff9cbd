"""The prefix cache: PagedBlockPool.ComputePrefixHash (PagedBlockPool.cs:168-172)
and TryFindPrefixBlock / BindPrefixBlock (:194-234) with the hash bookkeeping of
TryAllocateBlock (:178-189) and ReleaseBlock (:251-279).

The hash is pinned by golden vectors written with the `xxhash` module (the
reference implementation of the published XXH3 algorithm) over every XXH3
length path, seeds and chains.  The map semantics run the reference's own
tests against the product and the oracle, then a seeded churn of allocate /
retain / release / bind / find ops in which both must agree step by step.
"""
import numpy as np
import pytest

import glacier_oracle as orc
import glacier_paged as gp
import make_golden

V = make_golden.load_xxh3_vectors()


def vec(i):
    return V["tokens"][V["offsets"][i]:V["offsets"][i + 1]]


def test_prefix_hash_matches_xxh3_vectors():
    for i in range(len(V["seeds"])):
        got = gp.prefix_hash(int(V["seeds"][i]), vec(i))
        assert got == int(V["expected"][i]), (i, len(vec(i)), int(V["seeds"][i]))


def test_prefix_chain_matches():
    """ContinuousBatchEngine.cs:223-263: each full block's hash seeds the next one."""
    first = int(V["chain_first"][0])
    parent = 0
    for b in range(6):
        assert int(V["seeds"][first + b]) == parent
        parent = gp.prefix_hash(parent, vec(first + b))
        assert parent == int(V["expected"][first + b])


def test_reference_hash_properties():
    """PrefixHashKvCacheTests.cs:11-51 and PrefixHashKvCacheAdversarialTests.cs:143-177."""
    blk = make_golden.REFERENCE_TOKEN_BLOCKS
    a = gp.prefix_hash(0, blk[0])
    assert a != 0 and a == gp.prefix_hash(0, list(blk[0]))
    h0a, h0b = gp.prefix_hash(0, blk[1]), gp.prefix_hash(0, blk[2])
    assert h0a != h0b
    assert gp.prefix_hash(h0a, blk[3]) != gp.prefix_hash(h0b, blk[3])
    assert gp.prefix_hash(0, blk[1]) != gp.prefix_hash(0, blk[4])
    base = np.arange(1, 17, dtype=np.int32)
    assert len({gp.prefix_hash(0, np.roll(base, -s)) for s in range(16)}) == 16
    assert gp.prefix_hash(h0a, blk[5]) != gp.prefix_hash(h0b, blk[5])


def test_prefix_hash_rejects_bad_span():
    lib = gp.load()
    assert lib.gsp_prefix_hash(0, None, -1) == 0
    assert b"invalid" in lib.gsp_last_error()


class Product:
    name = "product"
    alloc = staticmethod(lambda n: gp.BlockAllocator(n, 16))
    Error = gp.InvalidArgument


class Oracle:
    name = "oracle"
    alloc = staticmethod(lambda n: orc.Alloc(n, 16))
    Error = orc.ArgumentOutOfRange


@pytest.fixture(params=[Product, Oracle], ids=lambda c: c.name)
def impl(request):
    return request.param


def test_bind_and_find_registers_and_recycles(impl):
    """PrefixHashKvCacheTests.cs:106-131."""
    pool = impl.alloc(16)
    h = gp.prefix_hash(0, list(range(1, 17)))
    ok, b = pool.try_allocate_block()
    pool.bind_prefix_block(h, b)
    found, fb = pool.try_find_prefix_block(h)
    assert found and fb == b and pool.get_ref_count(b) == 2
    pool.release_block(b)
    assert pool.get_ref_count(b) == 1
    pool.release_block(b)
    assert pool.get_ref_count(b) == 0
    assert pool.try_find_prefix_block(h) == (False, -1)
    assert pool.free_blocks_count == 16


def test_overwrite_then_release_keeps_second_block(impl):
    """PrefixHashKvCacheAdversarialTests.cs:13-41."""
    pool = impl.alloc(16)
    h = 0xABCD1234EF567890
    _, a = pool.try_allocate_block()
    _, b = pool.try_allocate_block()
    pool.bind_prefix_block(h, a)
    pool.bind_prefix_block(h, b)
    pool.release_block(a)
    assert pool.try_find_prefix_block(h) == (True, b)
    pool.release_block(b)
    pool.release_block(b)
    assert pool.try_find_prefix_block(h) == (False, -1)


def test_multi_block_overwrite_eviction_isolation(impl):
    """PrefixHashKvCacheAdversarialTests.cs:268-309."""
    n = 8
    pool = impl.alloc(n)
    h = 0x1122334455667788
    blocks = []
    for _ in range(n):
        ok, b = pool.try_allocate_block()
        assert ok
        pool.bind_prefix_block(h, b)
        blocks.append(b)
    last = blocks[-1]
    assert pool.try_find_prefix_block(h) == (True, last)
    pool.release_block(last)
    for b in blocks[:-1]:
        pool.release_block(b)
    assert pool.try_find_prefix_block(h) == (True, last)
    pool.release_block(last)
    pool.release_block(last)
    assert pool.try_find_prefix_block(h) == (False, -1)
    assert pool.free_blocks_count == n


def test_recycled_block_never_returns_stale_prefix(impl):
    """PrefixHashKvCacheAdversarialTests.cs:209-262, sequentially: a freed block
    reused under another hash is not found under the old one."""
    pool = impl.alloc(1)
    ha, hb = 0xA0A0A0A0A0A0A0A0, 0xB0B0B0B0B0B0B0B0
    _, b = pool.try_allocate_block()
    pool.bind_prefix_block(ha, b)
    pool.release_block(b)
    _, b2 = pool.try_allocate_block()
    assert b2 == b
    pool.bind_prefix_block(hb, b2)
    assert pool.try_find_prefix_block(ha) == (False, -1)
    assert pool.try_find_prefix_block(hb) == (True, b2)
    assert pool.get_ref_count(b2) == 2


def test_bind_rejects_what_the_reference_throws_on(impl):
    pool = impl.alloc(4)
    with pytest.raises(impl.Error):
        pool.bind_prefix_block(0x1234, 4)
    with pytest.raises(impl.Error):
        pool.bind_prefix_block(0x1234, -1)
    with pytest.raises(impl.Error):
        pool.bind_prefix_block(0, 1)
    assert pool.try_find_prefix_block(0) == (False, -1)


def test_product_matches_oracle_under_prefix_churn():
    rng = np.random.default_rng(0xCAC4E)
    total = 24
    p, o = gp.BlockAllocator(total, 16), orc.Alloc(total, 16)
    hashes = [int(x) for x in rng.integers(1, 2**63, size=12, dtype=np.int64)]
    live = []
    for step in range(6000):
        r = rng.random()
        if r < 0.25:
            a, b = p.try_allocate_block(), o.try_allocate_block()
            assert a == b
            if a[0]:
                live.append(a[1])
        elif r < 0.45 and live:
            bid = live.pop(int(rng.integers(len(live))))
            assert p.release_block(bid) == o.release_block(bid)
        elif r < 0.55 and live:
            bid = live[int(rng.integers(len(live)))]
            assert p.retain_block(bid) == o.retain_block(bid)
            live.append(bid)
        elif r < 0.75:
            bid = int(rng.integers(total))
            h = hashes[int(rng.integers(len(hashes)))]
            p.bind_prefix_block(h, bid)
            o.bind_prefix_block(h, bid)
        else:
            h = hashes[int(rng.integers(len(hashes)))]
            a, b = p.try_find_prefix_block(h), o.try_find_prefix_block(h)
            assert a == b, step
            if a[0]:
                live.append(a[1])
        if step % 500 == 0:
            assert [p.get_ref_count(i) for i in range(total)] == [o.get_ref_count(i) for i in range(total)]
            assert p.free_blocks_count == o.free_blocks_count


def test_prefix_hash_chain_matches_block_by_block():
    first = int(V["chain_first"][0])
    prompt = np.concatenate([vec(first + b) for b in range(6)])
    chain = gp.prefix_hash_chain(0, prompt)
    assert [int(x) for x in chain] == [int(V["expected"][first + b]) for b in range(6)]
    # A partial last block is not hashed (only full blocks enter the cache).
    assert len(gp.prefix_hash_chain(0, prompt[:-3])) == 5
    lib = gp.load()
    assert lib.gsp_prefix_hash_chain(0, None, 1, 16, None) == gp.GSP_E_INVALID_ARG
