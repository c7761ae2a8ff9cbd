"""The host block metadata under concurrency.

The reference's pool is shared between threads: HTTP admission looks up cached
prefixes (ContinuousBatchEngine.cs:229-251) while the engine loop allocates and
releases, and its adversarial tests drive it from 16 to 32 threads
(PrefixHashKvCacheAdversarialTests.cs:43-107, 209-265, 439-467).

- tests/native/host_meta_stress.cpp ports those tests over the C ABI with real
  threads, built from the library's host sources plain, with ThreadSanitizer and
  with AddressSanitizer + UndefinedBehaviorSanitizer; each build must pass with no
  sanitizer report.
- The same protocols run through the shipped library from Python threads (ctypes
  releases the GIL during each call).
"""
import subprocess
import threading
from pathlib import Path

import pytest

import glacier_paged as gp

NATIVE = Path(__file__).resolve().parent / "native"


@pytest.fixture(scope="module")
def native_builds():
    subprocess.run(["make", "-C", str(NATIVE), "-j3"], check=True, capture_output=True, text=True)
    return NATIVE / "_build"


@pytest.mark.parametrize("variant", ["host_meta_stress", "host_meta_stress_tsan", "host_meta_stress_asan"])
def test_native_concurrency_under_sanitizers(native_builds, variant):
    res = subprocess.run([str(native_builds / variant)], capture_output=True, text=True, timeout=600)
    report = res.stdout + res.stderr
    assert res.returncode == 0, report
    assert "all cases passed" in res.stdout
    for marker in ("WARNING: ThreadSanitizer", "ERROR: AddressSanitizer", "runtime error:"):
        assert marker not in report, report


def _run(n, fn):
    errs = []

    def wrap(i):
        try:
            fn(i)
        except Exception as e:  # pragma: no cover - reported below
            errs.append(e)

    ts = [threading.Thread(target=wrap, args=(i,)) for i in range(n)]
    for t in ts:
        t.start()
    for t in ts:
        t.join()
    assert not errs, errs


def test_shipped_library_concurrent_cow_forks():
    """16 tables sharing one 8-token page append concurrently: each ends on its own page."""
    a = gp.BlockAllocator(64)
    ok, shared = a.try_allocate_block()
    assert ok
    for _ in range(15):
        a.retain_block(shared)
    tables = [gp.BlockTable(a) for _ in range(16)]
    for t in tables:
        t.attach_prefix_blocks([shared], 8)
    got = [None] * 16
    barrier = threading.Barrier(16)

    def one(i):
        barrier.wait()
        got[i] = tables[i].append_token()

    _run(16, one)
    ids = [g[1] for g in got]
    assert all(g[0] and g[2] == 8 for g in got)
    assert len(set(ids)) == 16 and all(a.get_ref_count(b) == 1 for b in ids)
    for t in tables:
        t.release_all()
    assert a.free_blocks_count == 64


def test_shipped_library_aba_and_churn():
    a = gp.BlockAllocator(4)
    hash_a, hash_b = 0xAAAAAAAAAAAAAAAA, 0xBBBBBBBBBBBBBBBB
    bad = []

    def aba(w):
        for i in range(w, 4000, 8):
            if i % 2 == 0:
                ok, b = a.try_allocate_block()
                if ok:
                    a.bind_prefix_block(hash_a, b)
                    a.release_block(b)
                    ok, r = a.try_allocate_block()
                    if ok:
                        a.bind_prefix_block(hash_b, r)
                        a.release_block(r)
            else:
                ok, f = a.try_find_prefix_block(hash_a)
                if ok:
                    if a.get_ref_count(f) <= 0:
                        bad.append(f)
                    a.release_block(f)

    _run(8, aba)
    assert not bad
    assert a.free_blocks_count == 4 and all(a.get_ref_count(b) >= 0 for b in range(4))
    c = gp.BlockAllocator(64)

    def churn(w):
        for i in range(w, 4000, 32):
            h = 0xAA000000 + i % 16
            ok, b = c.try_allocate_block()
            if ok:
                c.bind_prefix_block(h, b)
                ok, f = c.try_find_prefix_block(h)
                if ok:
                    assert 0 <= f < 64
                    c.release_block(f)
                c.release_block(b)

    _run(32, churn)
    assert c.free_blocks_count == 64 and all(c.get_ref_count(b) >= 0 for b in range(64))
