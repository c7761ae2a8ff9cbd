"""GPU parity of the matrix-core prefill tiles (rows with q_len > 1) against the CPU oracle.

Query token i of a prefill row attends to min(TokenCount, pos + i + 1) tokens
(PagedAttentionKernel.cs:41, PagedTransformerRunner.cs:454-474).  The tiles
cover 16 query tokens x one KV head x up to 8 query heads; these cases pin the
ragged last tile (q_len % 16), tiles that straddle page boundaries, the first
chunk of a sequence (pos 0), token counts below pos + q_len, rows with
TokenCount 0, GQA groups above 8 (several head chunks per tile) and steps that
mix decode units with tiles.  Tiles over fp32 pages run both ways: from the
split records written once per step (the default) and splitting their pages
themselves.  Bar: max abs error <= 1e-4 (fp32 KV), <= 2e-3 (fp16 KV).
"""
import numpy as np
import pytest

import workloads
from conftest import threads
from gpu_helpers import TOL, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu

PREFILL_PATHS = {"tiles": 1, "auto": 0, "per_token": 2}
SPLITS = {"records": 0, "in_tile": 1}

GEOMS = [
    (28, 4, 128, "f32"),  # group 7
    (20, 4, 128, "f32"),  # group 5: waves 1-3 compute one tile, wave 0 two
    (24, 4, 64, "f32"),   # group 6: waves 2-3 compute one tile
    (14, 2, 64, "f32"),   # group 7, d64
    (32, 8, 128, "f16"),  # group 4
    (8, 1, 128, "f32"),   # group 8: one full head chunk
    (1, 1, 64, "f32"),    # MHA, group 1
    (32, 2, 128, "f32"),  # group 16: two head chunks
    (24, 2, 64, "f16"),   # group 12: a full and a partial head chunk
    (40, 2, 64, "f32"),   # group 20: three chunks; decode units run two tiles of heads
]


def run_step(torch, gsp, ctx, step, q, pool, prefill_path, layer=0, split_pages=0, fill=np.nan, split="records"):
    ctx.set_split_pages(split_pages)
    ctx.set_prefill_path(prefill_path)
    ctx.set_prefill_split(SPLITS[split])
    try:
        ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                      q_lens=step.q_lens)
        info = ctx.step_info()
        qd = torch.from_numpy(np.ascontiguousarray(q, dtype=np.float32)).cuda()
        out = torch.full((step.total_q, step.n_heads, step.head_dim), float(fill), dtype=torch.float32,
                         device="cuda")
        torch.cuda.synchronize()
        ctx.attention_step(pool, layer, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
        ctx.sync()
        return out.cpu().numpy(), info
    finally:
        ctx.set_split_pages(0)
        ctx.set_prefill_path(0)
        ctx.set_prefill_split(0)


def expected_tiles(step, min_q):
    lens = step.lens
    return sum(-(-int(ql) // 16) * step.n_kv for ql, tc in zip(lens, step.token_counts) if ql >= min_q and tc > 0)


@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0]}q{g[1]}kv_d{g[2]}_{g[3]}")
@pytest.mark.parametrize("path", list(PREFILL_PATHS))
@pytest.mark.parametrize("split", list(SPLITS))
def test_prefill_tiles_match_oracle(torch_mod, gsp, ctx, geom, path, split):
    nh, nkv, d, dt = geom
    if split == "in_tile" and (dt == "f16" or path == "per_token"):
        pytest.skip("the split mode only concerns tiles over fp32 pages")
    print(f"case prefill {geom} path={path} split={split}", flush=True)
    q_lens = np.array([2, 15, 16, 17, 33, 64, 1, 5, 48, 31], np.int32)
    step = workloads.small_step(seed=nh * 17 + nkv * 3 + d, rows=len(q_lens), n_heads=nh, n_kv=nkv, head_dim=d,
                                kv_dtype=dt, ctx_lo=0, ctx_hi=150, total_blocks=256, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    got, info = run_step(torch_mod, gsp, ctx, step, q, pool, PREFILL_PATHS[path], split=split)
    ref = oracle_step(step, q, k, v, threads=threads())
    pool.destroy()
    min_q = {"tiles": 2, "auto": 16, "per_token": 1 << 30}[path]
    assert info.prefill_tiles == expected_tiles(step, min_q)
    assert not np.isnan(got).any()
    assert max_err(got, ref) <= TOL[dt]


def test_first_chunk_and_clamped_token_counts(torch_mod, gsp, ctx):
    """pos 0 chunks, TokenCount below pos + q_len (later tokens see TokenCount keys) and TokenCount 0."""
    rng = np.random.default_rng(5)
    q_lens = np.array([16, 40, 23, 18, 32], np.int32)
    positions = np.array([0, 0, 30, 100, 7], np.int32)
    token_counts = np.array([16, 25, 41, 0, 39], np.int32)  # row 3 empty; rows 1, 2, 4 clamp
    pages = [max(1, -(-int(min(tc, p + ql)) // 16)) for tc, p, ql in zip(token_counts, positions, q_lens)]
    offsets = np.concatenate([[0], np.cumsum(pages)]).astype(np.int32)
    ids = rng.permutation(64)[: offsets[-1]].astype(np.int32)
    step = workloads.Step("clamp", 28, 4, 128, "f32", 64, 4096, positions=positions, token_counts=token_counts,
                          bt_offsets=offsets, bt_ids=ids, q_lens=q_lens, seed=5)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    got, info = run_step(torch_mod, gsp, ctx, step, q, pool, 1, fill=1234.5)
    ref = oracle_step(step, q, k, v, fill=1234.5)
    pool.destroy()
    r3 = slice(int(q_lens[:3].sum()), int(q_lens[:4].sum()))
    assert np.all(got[r3] == 1234.5)  # TokenCount 0: every query token has total 0, out untouched
    assert info.prefill_tiles == (1 + 3 + 2 + 2) * 4
    assert max_err(got, ref) <= 1e-4


@pytest.mark.parametrize("split", list(SPLITS))
def test_stale_slots_past_token_count_do_not_leak(torch_mod, gsp, ctx, split):
    """Slots past a prefill row's TokenCount may hold NaN / Inf; tiles (and split records) never read them."""
    q_lens = np.array([20, 37, 16], np.int32)
    step = workloads.small_step(seed=44, rows=3, n_heads=28, n_kv=4, head_dim=128, ctx_lo=0, ctx_hi=60,
                                total_blocks=64, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    kn, vn = k.copy(), v.copy()
    for b in range(step.num_rows):
        tot = int(step.token_counts[b])
        last, used = step.table(b)[(tot - 1) // 16], (tot - 1) % 16 + 1
        kn[last, :, :, used:] = np.nan
        vn[last, :, :, used:] = np.inf
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, kn, vn)
    got, _ = run_step(torch_mod, gsp, ctx, step, q, pool, 1, split=split)
    pool.destroy()
    assert max_err(got, oracle_step(step, q, k, v)) <= 1e-4


@pytest.mark.parametrize("dt,split", [("f32", "records"), ("f32", "in_tile"), ("f16", "records")])
def test_mixed_decode_and_prefill_step(torch_mod, gsp, ctx, dt, split):
    """Decode units (split-KV) and prefill tiles of one packed step, over two layers (the
    records of the second layer overwrite the first's)."""
    rng = np.random.default_rng(12)
    q_lens = np.array([1, 1, 96, 1, 19, 1, 1, 250, 1], np.int32)
    step = workloads.small_step(seed=12, rows=len(q_lens), n_heads=28, n_kv=4, head_dim=128, kv_dtype=dt,
                                ctx_lo=0, ctx_hi=500, total_blocks=512, q_lens=q_lens)
    q, _, _ = workloads.host_values(step)
    shape = (512, 2, 4, 16, 128)
    k = rng.standard_normal(shape, dtype=np.float32)
    v = rng.standard_normal(shape, dtype=np.float32)
    if dt == "f16":
        k, v = k.astype(np.float16), v.astype(np.float16)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    for layer, sp in ((0, 0), (1, 3)):
        got, info = run_step(torch_mod, gsp, ctx, step, q, pool, 0, layer=layer, split_pages=sp, split=split)
        assert info.prefill_tiles == expected_tiles(step, 16) and info.decode_units > 0
        ref = oracle_step(step, q, k.astype(np.float32), v.astype(np.float32), layer=layer, threads=threads())
        assert max_err(got, ref) <= TOL[dt]
    pool.destroy()


def test_tiles_equal_per_token_path(torch_mod, gsp, ctx):
    """The two prefill routes agree with each other to the fp32 bar on a long causal chunk."""
    q_lens = np.array([300, 129], np.int32)
    step = workloads.small_step(seed=8, rows=2, n_heads=32, n_kv=8, head_dim=128, ctx_lo=0, ctx_hi=900,
                                total_blocks=256, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    tiles, _ = run_step(torch_mod, gsp, ctx, step, q, pool, 1)
    per_token, _ = run_step(torch_mod, gsp, ctx, step, q, pool, 2)
    pool.destroy()
    assert max_err(tiles, per_token) <= 1e-4
    assert max_err(tiles, oracle_step(step, q, k, v, threads=threads())) <= 1e-4


def fp64_reference(step, q, k, v):
    """Exact-arithmetic (float64) attention of every query token, from the oracle's fp64 path."""
    import glacier_oracle as orc

    pool = orc.HostPool(k, v)
    out = np.zeros((step.total_q, step.n_heads, step.head_dim), np.float64)
    qi = 0
    for b in range(step.num_rows):
        for i in range(int(step.lens[b])):
            pos = int(step.positions[b]) + i
            out[qi] = orc.attention_fp64(pool, step.table(b), int(step.token_counts[b]), 0, pos, q[qi], step.n_heads,
                                         step.scale, step.max_seq_len).reshape(step.n_heads, step.head_dim)
            qi += 1
    return out


@pytest.mark.parametrize("case", ["peaked_scores", "mixed_v_pages", "beyond_fp16_range", "small_v", "tiny_values"])
@pytest.mark.parametrize("split", list(SPLITS))
def test_prefill_tiles_hold_fp32_range(torch_mod, gsp, ctx, case, split):
    """fp32 pages enter the fp16 matrix cores as scaled hi + lo pairs.  Values far outside fp16's
    range, pages whose V magnitudes differ by 1e9, tiny values and near-one-hot softmaxes stay
    within 4x of fp32 arithmetic's own error against float64 (the fp32 oracle's error; for
    peaked scores |S| ~ 1e3 it is ~1e-4 relative), plus 1e-6 of the output's magnitude."""
    q_lens = np.array([40, 16, 23], np.int32)
    step = workloads.small_step(seed=321, rows=3, n_heads=14, n_kv=2, head_dim=128, ctx_lo=0, ctx_hi=90,
                                total_blocks=64, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    rng = np.random.default_rng(9)
    if case == "peaked_scores":
        q, k = q * 40.0, k * 25.0
    elif case == "mixed_v_pages":
        page_scale = 10.0 ** rng.uniform(-4, 5, size=(k.shape[0], 1, 1, 1, 1))
        v = v * page_scale
    elif case == "beyond_fp16_range":
        q, k, v = q * 3e4, k * 2e5, v * 1e7
    elif case == "small_v":
        v = v * 1e-20  # the zero slots of a partial last page must not set the V scale
    else:
        q, k, v = q * 1e-6, k * 1e-7, v * 1e-30
    q, k, v = q.astype(np.float32), k.astype(np.float32), v.astype(np.float32)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    got, info = run_step(torch_mod, gsp, ctx, step, q, pool, 1, split=split)
    pool.destroy()
    assert info.prefill_tiles > 0
    exact = fp64_reference(step, q, k, v)
    fp32_err = max_err(oracle_step(step, q, k, v), exact)
    mag = float(np.abs(exact).max())
    assert np.isfinite(got).all()
    assert max_err(got, exact) <= 4.0 * fp32_err + 1e-6 * mag


def test_split_records_equal_in_tile_split(torch_mod, gsp, ctx):
    """Records and in-tile splitting agree to the fp32 bar, and records are what the default
    pack selects for fp32 pools.  Rows of several tiles share records; rows end mid-pair
    (odd page counts) as well as on a pair."""
    q_lens = np.array([130, 47, 16, 200], np.int32)
    step = workloads.small_step(seed=77, rows=4, n_heads=28, n_kv=4, head_dim=128, ctx_lo=0, ctx_hi=700,
                                total_blocks=256, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    rec, info_rec = run_step(torch_mod, gsp, ctx, step, q, pool, 1, split="records")
    own, info_own = run_step(torch_mod, gsp, ctx, step, q, pool, 1, split="in_tile")
    pool.destroy()
    pairs = [(-(-min(int(tc), int(p) + int(ql)) // 16) + 1) // 2
             for tc, p, ql in zip(step.token_counts, step.positions, q_lens) if tc > 0]
    assert info_rec.split_records == sum(pairs) * step.n_kv and info_own.split_records == 0
    assert any(-(-min(int(tc), int(p) + int(ql)) // 16) % 2 for tc, p, ql in
               zip(step.token_counts, step.positions, q_lens))
    assert max_err(rec, own) <= 1e-4
    assert max_err(rec, oracle_step(step, q, k, v, threads=threads())) <= 1e-4
