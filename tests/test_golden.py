"""The committed golden fixtures against the oracle and the product's host metadata.

tests/golden/make_golden.py computes the fixtures with numpy and plain Python
only: float64 dense attention over K/V gathered from the pool layout, and a
restated LIFO free stack / BlockTable driven by a seeded op log.  Matching
them pins the oracle's ComputeAttention restatement
(PagedAttentionKernel.cs:17-372) and both block-metadata implementations
(PagedBlockPool.cs:112-121,178-299,332-342; BlockTable.cs:31-116) to data
that neither of them produced.
"""
import numpy as np
import pytest

import glacier_oracle as orc
import glacier_paged as gp
import make_golden

CASES = make_golden.load_attention_cases()
TABLES = make_golden.load_block_tables()


def test_fixtures_regenerate_identically(tmp_path):
    """The committed files are exactly what the committed script writes."""
    make_golden.write(tmp_path)
    for name in ("attention_cases.npz", "block_tables.npz", "xxh3_vectors.npz"):
        with np.load(make_golden.HERE / name) as a, np.load(tmp_path / name) as b:
            assert sorted(a.files) == sorted(b.files)
            for key in a.files:
                assert a[key].dtype == b[key].dtype, key
                assert np.array_equal(a[key], b[key], equal_nan=a[key].dtype.kind == "f"), key


def test_kat_headdim128_closed_form():
    """PagedAttentionTests.cs:111-179, with the value its symmetry argument leaves open."""
    exp = CASES["kat_headdim128"]["expected"][0]
    assert np.allclose(exp[:2], 24.532020609, rtol=1e-6)
    assert np.allclose(exp[2:], 49.064041217, rtol=1e-6)


@pytest.mark.parametrize("name", sorted(CASES))
@pytest.mark.parametrize("isa", [orc.ISA_SCALAR, orc.ISA_AVX2, orc.ISA_AVX512])
def test_oracle_matches_golden(name, isa):
    if isa > orc.host_isa():
        pytest.skip("ISA not available on this host")
    c = CASES[name]
    n_heads, _, d, _, _, layer, max_seq_len, _ = (int(x) for x in c["meta"])
    pool = orc.HostPool(c["k"].astype(np.float32), c["v"].astype(np.float32))
    out = np.full(c["expected"].shape, np.nan, np.float32)
    orc.attention_step(pool, layer, c["positions"], c["token_counts"], c["bt_offsets"], c["bt_ids"], c["q"],
                       n_heads, float(c["scale"][0]), max_seq_len, q_lens=c["q_lens"], out=out, n_threads=2,
                       isa=isa)
    exp = c["expected"]
    untouched = np.isnan(exp)
    assert np.array_equal(np.isnan(out), untouched)
    err = np.abs(out[~untouched].astype(np.float64) - exp[~untouched])
    assert err.max() <= 2e-5 * (1.0 + np.abs(exp[~untouched]).max()), err.max()


class _Adapt:
    """Gives a product or oracle BlockTable the interface the fixture's replay drives."""

    def __init__(self, table):
        self.t = table

    def append(self):
        return self.t.append_token()[0]

    def attach(self, ids, tokens):
        self.t.attach_prefix_blocks(np.asarray(ids, np.int32), tokens)

    def release_all(self):
        self.t.release_all()

    @property
    def ids(self):
        return self.t.as_span().tolist()

    @property
    def tokens(self):
        return self.t.token_count


IMPLS = {
    "product": (lambda n: gp.BlockAllocator(n, 16), gp.BlockTable),
    "oracle": (lambda n: orc.Alloc(n, 16), orc.BTab),
    "fixture_restatement": (make_golden.Pool, make_golden.Table),
}


@pytest.mark.parametrize("impl", sorted(IMPLS))
def test_block_tables_replay_matches_fixture(impl):
    make_alloc, make_table = IMPLS[impl]
    total = int(TABLES["total_blocks"][0])
    if impl == "fixture_restatement":
        sim = make_golden.Sim(total)
        ref_count = lambda b: sim.pool.ref[b]
        free = lambda: len(sim.pool.stack)
    else:
        sim = make_golden.Sim(total, make_pool=make_alloc, make_table=lambda a: _Adapt(make_table(a)),
                              retain=lambda a, b: a.retain_block(b))
        ref_count = lambda b: sim.pool.get_ref_count(b)
        free = lambda: sim.pool.free_blocks_count
    for op in TABLES["ops"]:
        sim.apply(*(int(x) for x in op))
    assert [t.tokens for t in sim.live] == TABLES["token_counts"].tolist()
    ids = [b for t in sim.live for b in t.ids]
    assert ids == TABLES["bt_ids"].tolist()
    counts = np.diff(TABLES["bt_offsets"])
    assert [len(t.ids) for t in sim.live] == counts.tolist()
    assert [ref_count(b) for b in range(total)] == TABLES["ref_counts"].tolist()
    assert free() == int(TABLES["free_count"][0])


def test_block_table_fixture_exercises_sharing_and_exhaustion():
    """The log covers copy-on-write forks of shared partial pages and a pool that runs dry."""
    seen = {"forks": 0, "dry": 0}

    class Pool(make_golden.Pool):
        def try_allocate(self):
            b = super().try_allocate()
            seen["dry"] += b < 0
            return b

    class Table(make_golden.Table):
        def append(self):
            fork = self.tokens % 16 != 0 and self.pool.ref[self.ids[-1]] > 1
            ok = super().append()
            seen["forks"] += ok and fork
            return ok

    sim = make_golden.Sim(int(TABLES["total_blocks"][0]), make_pool=Pool, make_table=Table)
    for op in TABLES["ops"]:
        sim.apply(*(int(x) for x in op))
    assert seen["forks"] >= 5 and seen["dry"] >= 5, seen
    assert (TABLES["ref_counts"] > 1).any()
