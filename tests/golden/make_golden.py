"""Writes the committed golden fixtures of the paged-attention step.

Run from the repository root:  python tests/golden/make_golden.py

Everything here is computed with numpy and plain Python only.  Nothing
imports the oracle or the product.  The fixtures are therefore an independent
check on both.

attention_cases.npz
    Small paged steps with the expected outputs computed in float64 by dense
    softmax attention over K/V gathered token by token from the pool layout
    [block][layer][kv head][16][d] (PagedBlockPool.cs:77-83,128-131,140-143).
    Query i of a row attends to min(TokenCount, pos + i + 1) tokens
    (PagedAttentionKernel.cs:41, PagedTransformerRunner.cs:425-474).  GQA
    head h reads KV head h // (nH / nKV) (PagedAttentionKernel.cs:44,50-51).
    The scale multiplies the dot product (PagedAttentionKernel.cs:64).  A row
    whose query attends to no token has its expected output set to NaN: the
    kernel must leave it untouched (PagedAttentionKernel.cs:41-42).
    Case "kat_headdim128" is the reference's ComputeAttention_HeadDim128 test
    (PagedAttentionTests.cs:111-179).  Its closed-form value is checked here
    before it is written.

xxh3_vectors.npz
    PagedBlockPool.ComputePrefixHash (PagedBlockPool.cs:168-172) is the 64-bit
    XXH3 hash of a block's token ids (little-endian int32 bytes), seeded with
    the parent block's hash.  The expected values come from the `xxhash`
    module (the reference implementation of the published XXH3 algorithm):
    every length path of XXH3 (0 to 4000 bytes), seeds 0, chained parents and
    random 64-bit seeds, and the token blocks of the reference's own tests
    (PrefixHashKvCacheTests.cs:11-51, PrefixHashKvCacheAdversarialTests.cs:143-177).

block_tables.npz
    A seeded admit / grow / share / evict log replayed on a plain-Python
    restatement of the LIFO free stack with refcounts (PagedBlockPool.cs:
    112-121,178-189,240-299) and of BlockTable (BlockTable.cs:31-116,
    copy-on-write fork included, PagedBlockPool.cs:332-342).  The fixture
    holds the final tables, their CSR packing (the concatenated AsSpan() of
    every live table, BlockTable.cs:103) and the final refcounts.
"""
from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
BS = 16
SEED = 0x676F6C64656E  # fixed; recorded in every case

# --------------------------------------------------------------------------
# attention cases


def gather_reference(k, v, ids, layer, total, q_head, n_heads, scale):
    """float64 softmax(q K^T * scale) V of one query token over `total` tokens."""
    n_kv = k.shape[2]
    group = n_heads // n_kv
    t = np.arange(total)
    blk = np.asarray(ids, dtype=np.int64)[t // BS]
    slot = t % BS
    out = np.empty((n_heads, v.shape[4]), np.float64)
    for h in range(n_heads):
        kk = k[blk, layer, h // group, slot, :].astype(np.float64)
        vv = v[blk, layer, h // group, slot, :].astype(np.float64)
        s = (kk @ q_head[h].astype(np.float64)) * scale
        p = np.exp(s - s.max())
        out[h] = (p / p.sum()) @ vv
    return out


def expected_outputs(case):
    """[total_q][nH][d] float64 (stored rounded to float32); NaN rows attend to nothing."""
    k, v = case["k"].astype(np.float32), case["v"].astype(np.float32)
    n_heads, layer = int(case["meta"][0]), int(case["meta"][5])
    d = k.shape[4]
    q = case["q"]
    out = np.full((q.shape[0], n_heads, d), np.nan)
    qi = 0
    for b in range(len(case["positions"])):
        ids = case["bt_ids"][case["bt_offsets"][b]:case["bt_offsets"][b + 1]]
        for i in range(int(case["q_lens"][b])):
            total = min(int(case["token_counts"][b]), int(case["positions"][b]) + i + 1)
            if total > 0:
                out[qi] = gather_reference(k, v, ids, layer, total, q[qi], n_heads, float(case["scale"][0]))
            qi += 1
    return out


def paged_case(rng, *, n_heads, n_kv, d, kv_f16, rows, layers=1, layer=0, spare=2, max_seq_len=128):
    """rows: list of (token_count, pos, q_len).  Pages are a Fisher-Yates
    permutation of the pool sliced per row in logical order; spare blocks
    stay zero, as a freshly created pool is (PagedBlockPool.cs:87-95)."""
    pages = [-(-tc // BS) for tc, _, _ in rows]
    blocks = sum(pages) + spare
    perm = rng.permutation(blocks).astype(np.int32)
    offsets = np.zeros(len(rows) + 1, np.int32)
    offsets[1:] = np.cumsum(pages)
    ids = perm[:offsets[-1]]
    shape = (blocks, layers, n_kv, BS, d)
    k = np.zeros(shape, np.float32)
    v = np.zeros(shape, np.float32)
    for b in range(len(rows)):
        for j, blk in enumerate(ids[offsets[b]:offsets[b + 1]]):
            valid = min(BS, rows[b][0] - BS * j)
            k[blk, :, :, :valid] = rng.standard_normal((layers, n_kv, valid, d), dtype=np.float32)
            v[blk, :, :, :valid] = rng.standard_normal((layers, n_kv, valid, d), dtype=np.float32)
    if kv_f16:
        k, v = k.astype(np.float16), v.astype(np.float16)
    total_q = sum(r[2] for r in rows)
    q = rng.standard_normal((total_q, n_heads, d), dtype=np.float32)
    case = {
        "k": k, "v": v, "q": q,
        "positions": np.array([r[1] for r in rows], np.int32),
        "token_counts": np.array([r[0] for r in rows], np.int32),
        "q_lens": np.array([r[2] for r in rows], np.int32),
        "bt_offsets": offsets, "bt_ids": ids,
        "scale": np.array([1.0 / math.sqrt(d)], np.float64),
        # n_heads, n_kv, head_dim, kv_f16, layers, layer, max_seq_len, total_blocks
        "meta": np.array([n_heads, n_kv, d, int(kv_f16), layers, layer, max_seq_len, blocks], np.int32),
    }
    case["expected"] = expected_outputs(case).astype(np.float32)
    return case


def kat_headdim128():
    """PagedAttentionTests.cs:111-179: 32 tokens, 4 heads over 2 KV heads,
    k = 0.01f * (t + 1), v = (t + 1) on KV head 0 and 2 (t + 1) on KV head 1,
    q = 1, scale 1 / sqrt(128), pos 31, pages taken from a fresh pool (ids 0, 1)."""
    d, total, n_heads, n_kv = 128, 32, 4, 2
    k = np.zeros((8, 1, n_kv, BS, d), np.float32)
    v = np.zeros_like(k)
    for t in range(total):
        kt = np.float32(np.float32(0.01) * np.float32(t + 1))
        k[t // BS, 0, :, t % BS, :] = kt
        v[t // BS, 0, 0, t % BS, :] = np.float32(t + 1)
        v[t // BS, 0, 1, t % BS, :] = np.float32(2 * (t + 1))
    case = {
        "k": k, "v": v, "q": np.ones((1, n_heads, d), np.float32),
        "positions": np.array([total - 1], np.int32), "token_counts": np.array([total], np.int32),
        "q_lens": np.array([1], np.int32), "bt_offsets": np.array([0, 2], np.int32),
        "bt_ids": np.array([0, 1], np.int32),
        "scale": np.array([np.float32(1.0) / np.float32(math.sqrt(d))], np.float64),
        "meta": np.array([n_heads, n_kv, d, 0, 1, 0, total, 8], np.int32),
    }
    case["expected"] = expected_outputs(case)
    # Closed form: s_t = 128 * 0.01 (t + 1) / sqrt(128) = 0.01 sqrt(128) (t + 1),
    # out = sum_t softmax(s)_t (t + 1) on heads 0-1 and twice that on heads 2-3.
    c = 0.01 * math.sqrt(128.0)
    w = np.exp(c * np.arange(1, total + 1))
    closed = float((w * np.arange(1, total + 1)).sum() / w.sum())
    assert abs(closed - 24.532020609) < 1e-8, closed
    exp = case["expected"][0]
    assert np.allclose(exp[:2], closed, rtol=1e-6) and np.allclose(exp[2:], 2 * closed, rtol=1e-6)
    case["expected"] = case["expected"].astype(np.float32)
    return case


def attention_cases():
    rng = np.random.default_rng(SEED)
    cases = {"kat_headdim128": kat_headdim128()}
    # (token_count, pos, q_len) per row
    cases["d64_g7_f32_two_layers"] = paged_case(
        rng, n_heads=14, n_kv=2, d=64, kv_f16=False, layers=2, layer=1,
        rows=[(1, 0, 1), (17, 16, 1), (40, 39, 1), (0, 0, 1), (33, 12, 1)])
    cases["d128_g7_f32_mixed"] = paged_case(
        rng, n_heads=7, n_kv=1, d=128, kv_f16=False,
        rows=[(18, 17, 1), (20, 3, 17), (10, 30, 1), (16, 15, 1)])
    cases["d128_g4_f16_mixed"] = paged_case(
        rng, n_heads=8, n_kv=2, d=128, kv_f16=True,
        rows=[(20, 19, 1), (17, 0, 17), (5, 4, 1)])
    cases["d128_g8_f16_decode"] = paged_case(
        rng, n_heads=16, n_kv=2, d=128, kv_f16=True,
        rows=[(40, 39, 1), (3, 2, 1)])
    cases["d64_g1_f32_prefill"] = paged_case(
        rng, n_heads=2, n_kv=2, d=64, kv_f16=False,
        rows=[(24, 23, 1), (32, 16, 16), (7, 0, 7)])
    cases["d64_g16_f32_mixed"] = paged_case(
        rng, n_heads=16, n_kv=1, d=64, kv_f16=False,
        rows=[(21, 20, 1), (16, 0, 16)])
    return cases


# --------------------------------------------------------------------------
# block tables


class Pool:
    """LIFO free stack with refcounts (PagedBlockPool.cs:112-121,178-189,240-299)."""

    def __init__(self, total):
        self.stack = list(range(total - 1, -1, -1))  # pushes total-1 .. 0; the first pop is 0
        self.ref = [0] * total
        self.alloc = [0] * total

    def try_allocate(self):
        if not self.stack:
            return -1
        b = self.stack.pop()
        self.alloc[b], self.ref[b] = 1, 1
        return b

    def retain(self, b):
        self.ref[b] += 1

    def release(self, b):
        if not 0 <= b < len(self.ref):
            return
        self.ref[b] -= 1
        if self.ref[b] < 0:
            self.ref[b] = 0
            return
        if self.ref[b] == 0 and self.alloc[b] == 1:
            self.alloc[b] = 0
            self.stack.append(b)


class Table:
    """BlockTable.cs:13-117 over Pool, metadata only."""

    def __init__(self, pool):
        self.pool, self.ids, self.tokens = pool, [], 0

    def attach(self, ids, tokens):
        self.ids += list(ids)
        self.tokens = tokens

    def append(self):
        if self.tokens % BS == 0:
            b = self.pool.try_allocate()
            if b < 0:
                return False
            self.ids.append(b)
        elif self.pool.ref[self.ids[-1]] > 1:
            forked = self.pool.try_allocate()
            if forked < 0:
                return False
            self.pool.release(self.ids[-1])
            self.ids[-1] = forked
        self.tokens += 1
        return True

    def release_all(self):
        for b in self.ids:
            self.pool.release(b)
        self.ids, self.tokens = [], 0


OP_ADMIT, OP_EVICT, OP_GROW, OP_SHARE = 0, 1, 2, 3


class Sim:
    """Applies an op log, one op at a time.  Each op is (kind, a, b, c):
    ADMIT a tokens (a table that cannot take all of them is released and dropped);
    EVICT live[a]; GROW live[a] by b tokens (stops at the first failed append);
    SHARE the first b tokens of live[a] (its pages retained, then attached) and
    append c tokens to the new table (stops at the first failed append)."""

    def __init__(self, total_blocks, make_pool=Pool, make_table=Table, retain=None):
        self.pool = make_pool(total_blocks)
        self.make_table = make_table
        self.retain = retain or (lambda pool, blk: pool.retain(blk))
        self.live = []

    def apply(self, kind, a, b, c):
        if kind == OP_ADMIT:
            t = self.make_table(self.pool)
            if all(t.append() for _ in range(a)):
                self.live.append(t)
            else:
                t.release_all()
        elif kind == OP_EVICT:
            self.live.pop(a).release_all()
        elif kind == OP_GROW:
            for _ in range(b):
                if not self.live[a].append():
                    break
        elif kind == OP_SHARE:
            src = self.live[a]
            shared = list(src.ids[:-(-b // BS)])
            for blk in shared:
                self.retain(self.pool, blk)
            t = self.make_table(self.pool)
            t.attach(shared, b)
            for _ in range(c):
                if not t.append():
                    break
            self.live.append(t)


def block_table_log(total_blocks=96, n_ops=400):
    """A seeded op log whose ops are valid against the live set they see."""
    rng = np.random.default_rng(SEED + 1)
    sim = Sim(total_blocks)
    ops = []
    for _ in range(n_ops):
        tokens = [t.tokens for t in sim.live]
        r = rng.random()
        if not tokens or r < 0.35:
            op = (OP_ADMIT, int(rng.integers(1, 80)), 0, 0)
        elif r < 0.55:
            op = (OP_EVICT, int(rng.integers(len(tokens))), 0, 0)
        elif r < 0.85:
            op = (OP_GROW, int(rng.integers(len(tokens))), int(rng.integers(1, 40)), 0)
        else:
            i = int(rng.integers(len(tokens)))
            if tokens[i] == 0:
                op = (OP_GROW, i, 1, 0)
            else:
                op = (OP_SHARE, i, int(rng.integers(1, tokens[i] + 1)), int(rng.integers(0, 24)))
        ops.append(op)
        sim.apply(*op)
    live = sim.live
    counts = np.array([len(t.ids) for t in live], np.int32)
    offsets = np.zeros(len(live) + 1, np.int32)
    offsets[1:] = np.cumsum(counts)
    return {
        "total_blocks": np.array([total_blocks], np.int32),
        "ops": np.array(ops, np.int32),
        "token_counts": np.array([t.tokens for t in live], np.int32),
        "bt_offsets": offsets,
        "bt_ids": np.array([b for t in live for b in t.ids], np.int32),
        "ref_counts": np.array(sim.pool.ref, np.int32),
        "free_count": np.array([len(sim.pool.stack)], np.int32),
    }


# --------------------------------------------------------------------------
# XXH3 prefix hashes

REFERENCE_TOKEN_BLOCKS = [
    [101, 2054, 2003, 1037, 3231, 102] + [0] * 10,                 # PrefixHashKvCacheTests.cs:14
    list(range(1, 17)),                                             # :27, :44
    list(range(1, 16)) + [99],                                      # :28
    list(range(100, 116)),                                          # :30
    list(range(16, 0, -1)),                                         # :45
    [10, 20, 30, 40, 50, 60, 70, 80, 90, 100, 110, 120, 130, 140, 150, 160],  # Adversarial :167
]


def xxh3_vectors():
    import xxhash  # only this generator needs it

    rng = np.random.default_rng(SEED + 2)
    token_sets, seeds = [], []
    for n in list(range(0, 71)) + [100, 300, 1000]:  # 0 .. 280 bytes, then the long path
        toks = rng.integers(-2**31, 2**31, size=n, dtype=np.int64).astype(np.int32)
        for seed in (0, int(rng.integers(0, 2**63, dtype=np.int64)) * 2 + 1, 2**64 - 1):
            token_sets.append(toks)
            seeds.append(seed)
    # A Merkle chain over a prompt's full blocks, as ContinuousBatchEngine.cs:223-263 walks it.
    prompt = rng.integers(0, 150000, size=16 * 6, dtype=np.int64).astype(np.int32)
    parent = 0
    for b in range(6):
        token_sets.append(prompt[16 * b:16 * (b + 1)])
        seeds.append(parent)
        parent = xxhash.xxh3_64_intdigest(prompt[16 * b:16 * (b + 1)].astype("<i4").tobytes(), seed=parent)
    for blk in REFERENCE_TOKEN_BLOCKS:
        token_sets.append(np.array(blk, np.int32))
        seeds.append(0)
    offsets = np.zeros(len(token_sets) + 1, np.int64)
    offsets[1:] = np.cumsum([len(t) for t in token_sets])
    expected = [xxhash.xxh3_64_intdigest(t.astype("<i4").tobytes(), seed=sd) for t, sd in zip(token_sets, seeds)]
    return {
        "tokens": np.concatenate(token_sets).astype(np.int32),
        "offsets": offsets,
        "seeds": np.array(seeds, np.uint64),
        "expected": np.array(expected, np.uint64),
        "chain_first": np.array([len(token_sets) - 6 - len(REFERENCE_TOKEN_BLOCKS)], np.int64),
    }


def load_xxh3_vectors(path: Path = HERE / "xxh3_vectors.npz"):
    with np.load(path) as z:
        return {k: z[k] for k in z.files}


def write(out_dir: Path = HERE) -> None:
    flat = {}
    for name, case in attention_cases().items():
        for key, arr in case.items():
            flat[f"{name}__{key}"] = arr
    np.savez_compressed(out_dir / "attention_cases.npz", **flat)
    np.savez_compressed(out_dir / "block_tables.npz", **block_table_log())
    np.savez_compressed(out_dir / "xxh3_vectors.npz", **xxh3_vectors())


def load_attention_cases(path: Path = HERE / "attention_cases.npz"):
    """{case name: {key: array}} from the committed file."""
    cases = {}
    with np.load(path) as z:
        for key in z.files:
            name, field = key.split("__", 1)
            cases.setdefault(name, {})[field] = z[key]
    return cases


def load_block_tables(path: Path = HERE / "block_tables.npz"):
    with np.load(path) as z:
        return {k: z[k] for k in z.files}


if __name__ == "__main__":
    write(Path(sys.argv[1]) if len(sys.argv) > 1 else HERE)
