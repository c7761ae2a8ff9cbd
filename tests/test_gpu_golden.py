"""The HIP path against the committed golden fixtures, through the C ABI.

Expected outputs are float64 dense attention computed by
tests/golden/make_golden.py from the fixture's own pool pages; they never
pass through the oracle.  Every kernel path the packer can pick is run: DPP
and matrix-core decode, forced split-KV with its merge, matrix-core prefill
tiles and per-token prefill.
"""
import numpy as np
import pytest

import make_golden
import workloads
from gpu_helpers import TOL, gpu_step, to_device_pool

pytestmark = pytest.mark.gpu

CASES = make_golden.load_attention_cases()
TABLES = make_golden.load_block_tables()

# (decode path, prefill path, split pages)
PATHS = [
    ("auto", "auto", 0),
    ("dpp", "per_token", 0),
    ("mfma", "tiles", 0),
    ("mfma", "per_token", 1),
    ("dpp", "tiles", 1),
]


def fixture_step(c):
    n_heads, n_kv, d, f16, layers, layer, max_seq_len, blocks = (int(x) for x in c["meta"])
    step = workloads.Step("golden", n_heads, n_kv, d, "f16" if f16 else "f32", blocks, max_seq_len,
                          c["positions"], c["token_counts"], c["bt_offsets"], c["bt_ids"], c["q_lens"])
    return step, layer


@pytest.mark.parametrize("paths", PATHS, ids=lambda p: f"{p[0]}-{p[1]}-split{p[2]}")
@pytest.mark.parametrize("name", sorted(CASES))
def test_hip_path_matches_golden(torch_mod, gsp, ctx, name, paths):
    c = CASES[name]
    step, layer = fixture_step(c)
    decode, prefill, split = paths
    group = step.n_heads // step.n_kv
    ql = c["q_lens"]
    tiled = (prefill != "per_token") & (ql >= 2) & ((prefill == "tiles") | (ql >= 16))
    has_decode_units = bool(((ql >= 1) & ~tiled).any())
    if decode == "dpp" and group > 8 and has_decode_units:
        pytest.skip("the DPP decode kernel covers GQA groups up to 8")
    print(f"golden case {name} paths {paths}", flush=True)
    ctx.set_decode_path({"auto": gsp.DECODE_AUTO, "dpp": gsp.DECODE_DPP, "mfma": gsp.DECODE_MFMA}[decode])
    ctx.set_prefill_path({"auto": gsp.PREFILL_AUTO, "tiles": gsp.PREFILL_TILES,
                          "per_token": gsp.PREFILL_PER_TOKEN}[prefill])
    try:
        pool, keep = to_device_pool(torch_mod, gsp, ctx, step, c["k"], c["v"])
        out = gpu_step(torch_mod, gsp, ctx, step, c["q"], pool, layer=layer, split_pages=split)
        pool.destroy()
    finally:
        ctx.set_decode_path(gsp.DECODE_AUTO)
        ctx.set_prefill_path(gsp.PREFILL_AUTO)
    exp = c["expected"]
    untouched = np.isnan(exp)
    assert np.array_equal(np.isnan(out), untouched), "rows that attend to no token must stay untouched"
    err = float(np.abs(out[~untouched].astype(np.float64) - exp[~untouched]).max())
    assert err <= TOL[step.kv_dtype], err


def test_packing_matches_block_table_fixture(gsp, ctx):
    """The CSR packing of the fixture's live tables (BlockTable.AsSpan() of each,
    BlockTable.cs:103) is copied bit-exactly, each row cut to ceil(TokenCount/16)."""
    total = int(TABLES["total_blocks"][0])
    tc = TABLES["token_counts"]
    pool = gsp.Pool.create(ctx, total_blocks=total, layers=1, heads_kv=1, head_dim=64)
    try:
        ctx.pack_step(pool, tc - 1, tc, TABLES["bt_offsets"], TABLES["bt_ids"], int(tc.max()))
    finally:
        pool.destroy()
    rows, ids, ctxs = ctx.download_step()
    assert np.array_equal(rows, TABLES["bt_offsets"])
    assert np.array_equal(ids, TABLES["bt_ids"])
    assert np.array_equal(ctxs, tc)
