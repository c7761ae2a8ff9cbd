"""GPU parity of gsp_attention_step / gsp_compute_attention against the CPU oracle.

Bar: max abs error <= 1e-4 with fp32 KV and <= 2e-3 with fp16 KV (the oracle
reads the same fp16-rounded values, exactly upcast).  Rows whose total is 0
must leave `out` untouched (PagedAttentionKernel.cs:41-42).
"""
import math

import numpy as np
import pytest

import workloads
from conftest import threads
from gpu_helpers import TOL, gpu_step, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu

GEOMS = [
    # (n_heads, n_kv, head_dim, kv dtype): GQA groups 1..8, both dims, both dtypes
    (14, 2, 64, "f32"),
    (28, 4, 128, "f32"),
    (32, 8, 128, "f16"),
    (64, 8, 128, "f16"),
    (8, 1, 128, "f32"),
    (1, 1, 64, "f32"),
    (12, 4, 64, "f16"),
    (10, 2, 128, "f32"),
    (12, 2, 64, "f32"),
    (4, 2, 128, "f16"),
    (8, 8, 64, "f16"),
    (32, 2, 128, "f32"),  # group 16: the matrix-core tile exactly
    (24, 2, 64, "f16"),   # group 12
]

PATHS = {"mfma": 2, "dpp": 1}


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0]}q{g[1]}kv_d{g[2]}_{g[3]}")
@pytest.mark.parametrize("split_pages", [0, 1, 3, 8])
def test_decode_matches_oracle(torch_mod, gsp, ctx, geom, split_pages, path):
    nh, nkv, d, dt = geom
    if path == "dpp" and nh // nkv > 8:
        pytest.skip("the DPP kernel serves GQA groups up to 8")
    print(f"case decode {geom} split={split_pages} path={path}", flush=True)
    step = workloads.small_step(seed=nh * 131 + d + nkv, rows=11, n_heads=nh, n_kv=nkv, head_dim=d, kv_dtype=dt,
                                ctx_lo=1, ctx_hi=300, total_blocks=256)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    ctx.set_decode_path(PATHS[path])
    try:
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, split_pages=split_pages)
    finally:
        ctx.set_decode_path(0)
    ref = oracle_step(step, q, k, v, threads=threads())
    pool.destroy()
    assert not np.isnan(got).any()
    assert max_err(got, ref) <= TOL[dt]


@pytest.mark.parametrize("path", list(PATHS))
@pytest.mark.parametrize("bins", [1, 3, 64, 1000])
@pytest.mark.parametrize("split_pages", [0, 2])
def test_decode_bins_match_oracle(torch_mod, gsp, ctx, bins, split_pages, path):
    """Persistent bins: one workgroup runs a bin's units back to back (bins=1 runs every unit,
    merging its own split pieces; bins above the unit count leave one unit per workgroup)."""
    print(f"case bins={bins} split={split_pages} path={path}", flush=True)
    step = workloads.small_step(seed=400 + bins, rows=13, n_heads=28, n_kv=4, head_dim=128, ctx_lo=1, ctx_hi=400,
                                total_blocks=512)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    ctx.set_decode_path(PATHS[path])
    try:
        ctx.set_decode_bins(bins)
        info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                             step.max_seq_len)
        ctx.set_decode_bins(0)
        assert info.decode_bins == min(bins, info.decode_units)
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, split_pages=split_pages, bins=bins)
    finally:
        ctx.set_decode_path(0)
        ctx.set_decode_bins(0)
    ref = oracle_step(step, q, k, v, threads=threads())
    pool.destroy()
    assert max_err(got, ref) <= 1e-4


def test_stale_nan_slots_do_not_leak(torch_mod, gsp, ctx):
    """Slots past a row's context may hold anything (a wrapped pool is caller memory): NaN there is ignored."""
    step = workloads.small_step(seed=91, rows=8, n_heads=28, n_kv=4, head_dim=128, ctx_lo=1, ctx_hi=90,
                                total_blocks=64)
    q, k, v = workloads.host_values(step)
    kn, vn = k.copy(), v.copy()
    for b in range(step.num_rows):
        tot = int(step.token_counts[b])
        tbl = step.table(b)
        last, used = tbl[(tot - 1) // 16], (tot - 1) % 16 + 1
        kn[last, :, :, used:] = np.nan
        vn[last, :, :, used:] = np.inf
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, kn, vn)
    for path in (2, 1):
        ctx.set_decode_path(path)
        try:
            got = gpu_step(torch_mod, gsp, ctx, step, q, pool)
        finally:
            ctx.set_decode_path(0)
        ref = oracle_step(step, q, k, v)
        assert max_err(got, ref) <= 1e-4
    pool.destroy()


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_page_boundaries_and_single_token(torch_mod, gsp, ctx, dt):
    ctxs = np.array([1, 2, 15, 16, 17, 31, 32, 33, 48, 63, 64, 65, 255, 256, 257], np.int32)
    rng = np.random.default_rng(7)
    step = workloads.decode_step("edges", rng, ctxs, 28, 4, 128, dt, 512, 4096, 7)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    for sp in (0, 1, 2):
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, split_pages=sp)
        ref = oracle_step(step, q, k, v, threads=threads())
        assert max_err(got, ref) <= TOL[dt]
    # ctx == 1: the output is v_0 of the head's KV head exactly (softmax of one score is 1).
    one = got[0]
    blk = step.bt_ids[step.bt_offsets[0]]
    for h in range(28):
        np.testing.assert_allclose(one[h], v[blk, 0, h // 7, 0], atol=TOL[dt])
    pool.destroy()


def test_zero_total_rows_leave_out_untouched(torch_mod, gsp, ctx):
    """Rows with TokenCount 0 produce no write; pos beyond TokenCount reads TokenCount tokens."""
    rng = np.random.default_rng(9)
    ctxs = np.array([20, 40, 33], np.int32)
    step = workloads.decode_step("zero", rng, ctxs, 8, 2, 64, "f32", 64, 4096, 9)
    step.token_counts = np.array([20, 0, 33], np.int32)   # row 1: empty table content
    step.positions = np.array([19, 5, 50], np.int32)       # row 2: pos > TokenCount - 1
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    got = gpu_step(torch_mod, gsp, ctx, step, q, pool, fill=1234.5)
    ref = oracle_step(step, q, k, v, fill=1234.5)
    assert np.all(got[1] == 1234.5)
    assert max_err(got, ref) <= 1e-4
    pool.destroy()


def test_steps_with_nothing_to_attend(torch_mod, gsp, ctx):
    """A step of no rows, and one whose rows all have TokenCount 0, launch nothing and write nothing;
    the context then runs an ordinary step."""
    torch = torch_mod
    rng = np.random.default_rng(12)
    ctxs = np.array([20, 40, 33], np.int32)
    step = workloads.decode_step("empty", rng, ctxs, 8, 2, 64, "f32", 64, 4096, 12)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    qd = torch.from_numpy(np.ascontiguousarray(q, dtype=np.float32)).cuda()

    info = ctx.pack_step(pool, [], [], [0], [], 4096)
    assert info.num_rows == 0 and info.decode_units == 0 and info.prefill_tiles == 0
    out = torch.full((3, 8, 64), 7.0, dtype=torch.float32, device="cuda")
    ctx.attention_step(pool, 0, 8, qd.data_ptr(), out.data_ptr(), step.scale)
    ctx.sync()
    assert bool((out == 7.0).all())

    idle = workloads.Step(step.name, step.n_heads, step.n_kv, step.head_dim, step.kv_dtype, step.total_blocks,
                          step.max_seq_len, step.positions, np.zeros(3, np.int32), step.bt_offsets, step.bt_ids,
                          step.q_lens, step.seed, dict(step.notes), step.block_size, step.v_head_dim)
    got = gpu_step(torch, gsp, ctx, idle, q, pool, fill=7.0)
    assert ctx.step_info().decode_units == 0
    assert np.all(got == 7.0)

    got = gpu_step(torch, gsp, ctx, step, q, pool)
    assert max_err(got, oracle_step(step, q, k, v)) <= 1e-4
    pool.destroy()


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_prefill_rows_are_causal(torch_mod, gsp, ctx, dt):
    """Rows with q_len > 1: query i attends to min(TokenCount, pos + i + 1) tokens."""
    q_lens = np.array([5, 1, 17, 1, 40, 2], np.int32)
    step = workloads.small_step(seed=21, rows=6, n_heads=28, n_kv=4, head_dim=128, kv_dtype=dt, ctx_hi=120,
                                total_blocks=128, q_lens=q_lens)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    for sp in (0, 1):
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, split_pages=sp)
        ref = oracle_step(step, q, k, v)
        assert max_err(got, ref) <= TOL[dt]
    pool.destroy()


def test_layer_selection(torch_mod, gsp, ctx):
    """stage_layer picks the pool layer (PagedAttentionKernel.cs:63): layer 2 of a 3-layer pool."""
    step = workloads.small_step(seed=33, rows=5, n_heads=14, n_kv=2, head_dim=64, ctx_hi=200, total_blocks=128)
    q, _, _ = workloads.host_values(step)
    rng = np.random.default_rng(4)
    k = rng.standard_normal((128, 3, 2, 16, 64), dtype=np.float32)
    v = rng.standard_normal((128, 3, 2, 16, 64), dtype=np.float32)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    for layer in (0, 2):
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, layer=layer)
        ref = oracle_step(step, q, k, v, layer=layer)
        assert max_err(got, ref) <= 1e-4
    pool.destroy()


def test_compute_attention_single_sequence(torch_mod, gsp, ctx, oracle):
    """The reference-shaped drop-in: one BlockTable, one position."""
    torch = torch_mod
    alloc = gsp.BlockAllocator(64)
    table = gsp.BlockTable(alloc)
    assert table.append_tokens(70) == 70
    rng = np.random.default_rng(2)
    k = rng.standard_normal((64, 1, 4, 16, 128), dtype=np.float32)
    v = rng.standard_normal((64, 1, 4, 16, 128), dtype=np.float32)
    kd = torch.from_numpy(k).cuda()
    vd = torch.from_numpy(v).cuda()
    pool = gsp.Pool.wrap(ctx, kd.data_ptr(), vd.data_ptr(), 64, 1, 4, 128)
    q = rng.standard_normal((28, 128), dtype=np.float32)
    qd = torch.from_numpy(q).cuda()
    out = torch.zeros((28, 128), device="cuda")
    torch.cuda.synchronize()
    scale = 1 / math.sqrt(128)
    ctx.compute_attention(0, 0, 69, qd.data_ptr(), out.data_ptr(), table, pool, 28, 4, 128, 128, scale, 4096)
    ctx.sync()
    ref = oracle.compute_attention(oracle.HostPool(k, v), table.as_span(), 70, 0, 69, q, 28, scale, 4096)
    assert max_err(out.cpu().numpy().reshape(-1), ref) <= 1e-4
    # Reference bounds (PhaseCServeRemediationTests.cs:117-175) become GSP_E_INVALID_ARG.
    for pos, msl in ((16, 16), (-1, 16)):
        with pytest.raises(gsp.InvalidArgument):
            ctx.compute_attention(0, 0, pos, qd.data_ptr(), out.data_ptr(), [0], pool, 28, 4, 128, 128, scale, msl,
                                  token_count=1)
    with pytest.raises(gsp.InvalidArgument):  # head geometry must match the pool
        ctx.compute_attention(0, 0, 5, qd.data_ptr(), out.data_ptr(), table, pool, 28, 2, 128, 128, scale, 4096)
    with pytest.raises(gsp.Unsupported):  # sinks are rejected, as the reference GPU runner does
        ctx.compute_attention(0, 0, 5, qd.data_ptr(), out.data_ptr(), table, pool, 28, 4, 128, 128, scale, 4096,
                              sink_logit=0.0)
    pool.destroy()


def test_repeated_steps_reuse_counters(torch_mod, gsp, ctx):
    """Split-KV counters reset themselves: many steps in a row stay exact."""
    step = workloads.small_step(seed=77, rows=9, n_heads=28, n_kv=4, head_dim=128, ctx_lo=100, ctx_hi=900,
                                total_blocks=512)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch_mod, gsp, ctx, step, k, v)
    ref = oracle_step(step, q, k, v, threads=threads())
    for i in range(6):
        got = gpu_step(torch_mod, gsp, ctx, step, q, pool, split_pages=[1, 2, 5, 0, 3, 1][i])
        assert max_err(got, ref) <= 1e-4
    pool.destroy()


@pytest.mark.parametrize("kv_dtype", ["f32", "f16"])
def test_split_merges_are_bit_reproducible(torch_mod, gsp, ctx, kv_dtype):
    """A split pair is merged by whichever workgroup counts its last piece, inside
    its unit loop (general form) or after its last unit (wide form), so the form
    depends on timing.  Both run the same arithmetic, so pairs of many pieces
    (1- and 2-page splits: up to 60 pieces) give the same bits on every run."""
    from gpu_helpers import TOL, gpu_step, max_err, oracle_step, to_device_pool

    torch = torch_mod
    step = workloads.small_step(seed=81, rows=20, n_heads=28, n_kv=4, head_dim=128, kv_dtype=kv_dtype, ctx_lo=300,
                                ctx_hi=960, total_blocks=2048)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        ref = oracle_step(step, q, k, v)
        for split in (1, 2):
            print(f"case reproducible merges {kv_dtype} split={split}", flush=True)
            outs = [gpu_step(torch, gsp, ctx, step, q, pool, split_pages=split) for _ in range(6)]
            assert max_err(outs[0], ref) <= TOL[kv_dtype]
            for r, o in enumerate(outs[1:], 1):
                assert np.array_equal(o, outs[0]), f"split {split}: run {r} differs from run 0"
    finally:
        pool.destroy()
