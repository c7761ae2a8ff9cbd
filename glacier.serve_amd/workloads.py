"""Synthetic engine steps for the paged-attention path.

Each generator returns a ``Step``: the ragged batch an engine tick hands to
the attention step (positions, BlockTable.TokenCount, the CSR-concatenated
BlockTable.AsSpan() ids, query lengths) plus the head geometry and pool size.
Values (Q, K, V ~ N(0, 1)) are drawn separately by the caller, on the host
with numpy or on the device with torch, from the step's seed.

The five measured shapes:
  qwen05b_decode   14/2 heads, d=64, 8 rows, ctx U[1,256], 1024-block pool, fp32
  qwen7b_decode    28/4 heads, d=128, 64 rows, ctx log-uniform [128,4096], 32768 blocks, fp32
  llama8b_decode   32/8 heads, d=128, 256 rows, ctx lognormal(median 1024, sigma 1) clipped
                   to [16,8192], fp16, 65536 blocks, tables from 2000 admit/evict steps of
                   the LIFO free stack
  qwen7b_mixed     28/4 heads, d=128, 48 decode rows ctx U[256,4096] + 16 prefill rows
                   (prior U[0,2048], chunk U[32,512], causal), 32768 blocks, fp32
  longctx_decode   64/8 heads, d=128, 16 rows, ctx U[16384,32768], fp16, 32768 blocks
Beside them, refmodel_decode: the reference's test-model attention (2/1 heads, d=32,
8-token pages) at 256 rows, ctx log-uniform [128,4096], fp32, 65536 blocks.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Callable, List, Optional, Tuple

import numpy as np

SEED_BASE = 0x6C616369657201
BLOCK_SIZE = 16


@dataclass
class Step:
    name: str
    n_heads: int
    n_kv: int
    head_dim: int
    kv_dtype: str  # "f32" | "f16"
    total_blocks: int
    max_seq_len: int
    positions: np.ndarray
    token_counts: np.ndarray
    bt_offsets: np.ndarray
    bt_ids: np.ndarray
    q_lens: Optional[np.ndarray] = None
    seed: int = 0
    notes: dict = field(default_factory=dict)
    block_size: int = BLOCK_SIZE
    v_head_dim: Optional[int] = None  # None: head_dim

    @property
    def dv(self) -> int:
        return self.v_head_dim if self.v_head_dim else self.head_dim

    @property
    def num_rows(self) -> int:
        return len(self.positions)

    @property
    def lens(self) -> np.ndarray:
        return self.q_lens if self.q_lens is not None else np.ones(self.num_rows, np.int32)

    @property
    def total_q(self) -> int:
        return int(self.lens.sum())

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.head_dim)

    @property
    def elem_bytes(self) -> int:
        return 2 if self.kv_dtype == "f16" else 4

    def row_ctx(self) -> np.ndarray:
        """Tokens each row reads: min(TokenCount, pos + q_len) (its last query's total); 0 without queries."""
        lens = self.lens.astype(np.int64)
        ctx = np.minimum(self.token_counts.astype(np.int64), self.positions.astype(np.int64) + lens)
        return np.where(lens > 0, ctx, 0)

    def kv_tokens(self) -> int:
        return int(self.row_ctx().sum())

    def kv_bytes(self) -> int:
        """Algorithmic KV bytes of one step: every valid K and V element once."""
        return self.kv_tokens() * self.n_kv * (self.head_dim + self.dv) * self.elem_bytes

    def decode_mask(self) -> np.ndarray:
        return self.lens == 1

    def prefill_flops(self) -> int:
        """4*d*nH per (query, attended key) pair over the rows with q_len > 1."""
        total = 0
        for b in np.nonzero(self.lens > 1)[0]:
            pos = int(self.positions[b])
            tc = int(self.token_counts[b])
            for i in range(int(self.lens[b])):
                total += min(tc, pos + i + 1)
        return 4 * self.head_dim * self.n_heads * total

    def table(self, b: int) -> np.ndarray:
        return self.bt_ids[self.bt_offsets[b]:self.bt_offsets[b + 1]]

    def subset(self, rows) -> Tuple["Step", np.ndarray]:
        """The step restricted to `rows` (same pool and seed), and the indices of
        its query tokens within this step's q / out rows."""
        rows = np.asarray(rows, np.int64)
        lens = self.lens.astype(np.int64)
        starts = np.concatenate([[0], np.cumsum(lens)])
        q_index = np.concatenate([np.arange(starts[b], starts[b + 1]) for b in rows]) if len(rows) else \
            np.zeros(0, np.int64)
        spans = [self.table(int(b)) for b in rows]
        offsets = np.concatenate([[0], np.cumsum([len(t) for t in spans])]).astype(np.int32)
        ids = np.concatenate(spans).astype(np.int32) if spans else np.zeros(0, np.int32)
        q_lens = None if self.q_lens is None else self.q_lens[rows].astype(np.int32)
        sub = Step(self.name, self.n_heads, self.n_kv, self.head_dim, self.kv_dtype, self.total_blocks,
                   self.max_seq_len, positions=self.positions[rows].astype(np.int32),
                   token_counts=self.token_counts[rows].astype(np.int32), bt_offsets=offsets, bt_ids=ids,
                   q_lens=q_lens, seed=self.seed, notes=dict(self.notes), block_size=self.block_size,
                   v_head_dim=self.v_head_dim)
        return sub, q_index


def _slices(rng: np.random.Generator, total_blocks: int, pages: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """Fisher-Yates permutation of the pool, cut into consecutive per-row slices."""
    need = int(pages.sum())
    if need > total_blocks:
        raise ValueError(f"{need} pages do not fit a {total_blocks}-block pool")
    perm = rng.permutation(total_blocks).astype(np.int32)
    offsets = np.zeros(len(pages) + 1, np.int32)
    offsets[1:] = np.cumsum(pages)
    return offsets, np.ascontiguousarray(perm[:need])


def _pages(tokens, block_size: int = BLOCK_SIZE) -> np.ndarray:
    return ((np.asarray(tokens, np.int64) + block_size - 1) // block_size).astype(np.int32)


def decode_step(name: str, rng: np.random.Generator, ctx: np.ndarray, n_heads: int, n_kv: int, head_dim: int,
                kv_dtype: str, total_blocks: int, max_seq_len: int, seed: int, block_size: int = BLOCK_SIZE,
                v_head_dim: Optional[int] = None) -> Step:
    ctx = np.asarray(ctx, np.int32)
    offsets, ids = _slices(rng, total_blocks, _pages(ctx, block_size))
    return Step(name, n_heads, n_kv, head_dim, kv_dtype, total_blocks, max_seq_len, positions=ctx - 1,
                token_counts=ctx.copy(), bt_offsets=offsets, bt_ids=ids, seed=seed, block_size=block_size,
                v_head_dim=v_head_dim)


def qwen05b_decode(seed: int = SEED_BASE + 1) -> Step:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(1, 257, size=8)
    return decode_step("qwen05b_decode", rng, ctx, 14, 2, 64, "f32", 1024, 4096, seed)


def qwen7b_decode(seed: int = SEED_BASE + 2) -> Step:
    rng = np.random.default_rng(seed)
    ctx = np.rint(np.exp(rng.uniform(math.log(128), math.log(4096), size=64))).astype(np.int32)
    return decode_step("qwen7b_decode", rng, ctx, 28, 4, 128, "f32", 32768, 4096, seed)


def longctx_decode(seed: int = SEED_BASE + 5) -> Step:
    rng = np.random.default_rng(seed)
    ctx = rng.integers(16384, 32769, size=16)
    return decode_step("longctx_decode", rng, ctx, 64, 8, 128, "f16", 32768, 32768, seed)


def qwen7b_mixed(seed: int = SEED_BASE + 4) -> Step:
    rng = np.random.default_rng(seed)
    dec_ctx = rng.integers(256, 4097, size=48)
    prior = rng.integers(0, 2049, size=16)
    chunk = rng.integers(32, 513, size=16)
    tokens = np.concatenate([dec_ctx, prior + chunk]).astype(np.int32)
    offsets, ids = _slices(rng, 32768, _pages(tokens))
    positions = np.concatenate([dec_ctx - 1, prior]).astype(np.int32)
    q_lens = np.concatenate([np.ones(48, np.int64), chunk]).astype(np.int32)
    return Step("qwen7b_mixed", 28, 4, 128, "f32", 32768, 4096, positions=positions, token_counts=tokens,
                bt_offsets=offsets, bt_ids=ids, q_lens=q_lens, seed=seed)


def lognormal_len(rng: np.random.Generator, median: float = 1024.0, sigma: float = 1.0, lo: int = 16,
                  hi: int = 8192) -> int:
    return int(min(hi, max(lo, round(math.exp(rng.normal(math.log(median), sigma))))))


def simulate_free_stack(make_alloc: Callable, make_table: Callable, rng: np.random.Generator, total_blocks: int,
                        steps: int, rows: int, p_admit: float = 0.55, sigma: float = 1.0):
    """Admit/evict churn against the LIFO free stack (PagedBlockPool.cs:178-279).

    Each step either admits a sequence of lognormal length (BlockTable.AppendToken
    per token, BlockTable.cs:46-80) or evicts a random live one (ReleaseAll,
    BlockTable.cs:108-116).  Afterwards the live set is topped up or sampled down
    to `rows` sequences.  Returns (tables, token_counts) of the chosen rows in
    admission order; the allocator and tables come from the factories so the
    same decisions can drive the product and the oracle restatement.
    """
    alloc = make_alloc(total_blocks)
    live: List = []

    def admit() -> bool:
        n = lognormal_len(rng, sigma=sigma)
        t = make_table(alloc)
        if t.append_tokens(n) < n:
            t.release_all()
            return False
        live.append(t)
        return True

    for _ in range(steps):
        if live and rng.random() >= p_admit:
            victim = live.pop(int(rng.integers(len(live))))
            victim.release_all()
        else:
            admit()
    while len(live) < rows:
        if not admit():
            raise RuntimeError("pool exhausted while topping up the live set")
    if len(live) > rows:
        keep = np.sort(rng.choice(len(live), size=rows, replace=False))
        live = [live[i] for i in keep]
    return alloc, live


def llama8b_decode(seed: int = SEED_BASE + 3, make_alloc: Optional[Callable] = None,
                   make_table: Optional[Callable] = None, steps: int = 2000) -> Step:
    if make_alloc is None or make_table is None:
        from glacier_paged import BlockAllocator, BlockTable  # product host metadata
        make_alloc = make_alloc or (lambda n: BlockAllocator(n))
        make_table = make_table or (lambda a: BlockTable(a))
    rng = np.random.default_rng(seed)
    total_blocks = 65536
    alloc, live = simulate_free_stack(make_alloc, make_table, rng, total_blocks, steps, 256)
    spans = [np.asarray(t.as_span(), np.int32) for t in live]
    ctx = np.array([t.token_count for t in live], np.int32)
    offsets = np.zeros(len(spans) + 1, np.int32)
    offsets[1:] = np.cumsum([len(s) for s in spans])
    ids = np.concatenate(spans).astype(np.int32)
    step = Step("llama8b_decode", 32, 8, 128, "f16", total_blocks, 8192, positions=ctx - 1, token_counts=ctx,
                bt_offsets=offsets, bt_ids=ids, seed=seed,
                notes={"admit_evict_steps": steps, "p_admit": 0.55, "sigma": 1.0})
    step.notes["allocated_blocks"] = total_blocks - int(alloc.free_blocks_count)
    return step


def refmodel_decode(seed: int = SEED_BASE + 6) -> Step:
    """The attention geometry of the reference's own GPU test model (2 query / 1 KV heads, head_dim 32,
    8-token pages; PhaseCServeRemediationTests.cs:330-352), at serving batch: 256 rows, contexts
    log-uniform in [128, 4096], fp32, a 65536-block pool.  It runs the decode kernel's general form
    (run-time widths and page size)."""
    rng = np.random.default_rng(seed)
    ctx = np.rint(np.exp(rng.uniform(math.log(128), math.log(4096), size=256))).astype(np.int32)
    return decode_step("refmodel_decode", rng, ctx, 2, 1, 32, "f32", 65536, 4096, seed, block_size=8)


CONFIGS = {
    1: qwen05b_decode,
    2: qwen7b_decode,
    3: llama8b_decode,
    4: qwen7b_mixed,
    5: longctx_decode,
}


def small_step(seed: int, rows: int, n_heads: int, n_kv: int, head_dim: int, kv_dtype: str = "f32",
               ctx_lo: int = 1, ctx_hi: int = 64, total_blocks: int = 256, max_seq_len: int = 4096,
               q_lens: Optional[np.ndarray] = None, block_size: int = BLOCK_SIZE,
               v_head_dim: Optional[int] = None) -> Step:
    """A small seeded ragged step for parity tests; rows with q_len > 1 are causal prefill rows."""
    rng = np.random.default_rng(seed)
    if q_lens is None:
        ctx = rng.integers(ctx_lo, ctx_hi + 1, size=rows).astype(np.int32)
        st = decode_step(f"small{seed}", rng, ctx, n_heads, n_kv, head_dim, kv_dtype, total_blocks, max_seq_len,
                         seed, block_size=block_size, v_head_dim=v_head_dim)
        return st
    q_lens = np.asarray(q_lens, np.int32)
    prior = rng.integers(ctx_lo - 1 if ctx_lo > 0 else 0, ctx_hi + 1, size=rows).astype(np.int32)
    tokens = prior + q_lens
    offsets, ids = _slices(rng, total_blocks, _pages(tokens, block_size))
    return Step(f"small{seed}", n_heads, n_kv, head_dim, kv_dtype, total_blocks, max_seq_len, positions=prior,
                token_counts=tokens, bt_offsets=offsets, bt_ids=ids, q_lens=q_lens, seed=seed,
                block_size=block_size, v_head_dim=v_head_dim)


def device_values(torch, step: Step, layers: int = 1):
    """Q and full pool arenas ~ N(0,1) drawn on the GPU from the step's seed.

    Returns (q fp32 [total_q, nH, d], k, v [blocks, layers, nKV, 16, d] in the
    pool dtype); fp16 arenas are fp32 draws rounded once to nearest even.
    """
    g = torch.Generator(device="cuda")
    g.manual_seed(int(step.seed) & 0x7FFFFFFFFFFFFFFF)
    q = torch.randn((step.total_q, step.n_heads, step.head_dim), generator=g, device="cuda", dtype=torch.float32)
    dt = torch.float16 if step.kv_dtype == "f16" else torch.float32
    arenas = []
    for dim in (step.head_dim, step.dv):
        shape = (step.total_blocks, layers, step.n_kv, step.block_size, dim)
        a = torch.empty(shape, device="cuda", dtype=dt)
        flat = a.view(step.total_blocks, -1)
        for b0 in range(0, step.total_blocks, 4096):  # bounded fp32 temporaries
            b1 = min(step.total_blocks, b0 + 4096)
            flat[b0:b1] = torch.randn((b1 - b0, flat.shape[1]), generator=g, device="cuda",
                                      dtype=torch.float32).to(dt)
        arenas.append(a)
    return q, arenas[0], arenas[1]


def host_values(step: Step, rng: Optional[np.random.Generator] = None, layers: int = 1):
    """Q [total_q, nH, d] and pool arenas [blocks, layers, nKV, 16, d] ~ N(0,1), fp32.

    fp16 steps round K/V to fp16 once (RNE) and keep them as exactly upcast fp32.
    """
    rng = rng or np.random.default_rng(step.seed ^ 0x5EED)
    q = rng.standard_normal((step.total_q, step.n_heads, step.head_dim), dtype=np.float32)
    k = rng.standard_normal((step.total_blocks, layers, step.n_kv, step.block_size, step.head_dim), dtype=np.float32)
    v = rng.standard_normal((step.total_blocks, layers, step.n_kv, step.block_size, step.dv), dtype=np.float32)
    if step.kv_dtype == "f16":
        k = k.astype(np.float16).astype(np.float32)
        v = v.astype(np.float16).astype(np.float32)
    return q, k, v
