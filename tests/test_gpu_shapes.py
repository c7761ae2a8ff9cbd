"""The attention step over the reference runner's whole shape domain, against the oracle.

The reference GPU runner admits any even head_dim up to 256 and takes its page
size as an argument (CudaPagedTransformerRunner.cs:402-412, :78-190); the CPU
kernel has a generic path for any head_dim and a v_head_dim that differs from
head_dim (PagedAttentionKernel.cs:326-370), and no bound on the GQA group
(:44-50).  These cases run that domain through the C ABI:
  - the reference's own model shapes: head_dim 32 with 8-token pages
    (PhaseCServeRemediationTests.cs:321-346) and head_dim 32 / v_head_dim 64
    with 4-token pages (:257-319);
  - head dims 1 .. 256, multiples of 4, even and odd (loads of 4, 2 and 1 dims);
  - page sizes 1 .. 16, and above (17, 24, 32, 48, 64: each pool page read as
    equal kernel pages of at most 16 tokens);
  - GQA groups 17 .. 32 (tiles of 16 heads over grid.y), with forced splits;
  - v_head_dim above and below head_dim;
  - prefill rows on pools the prefill tiles do not serve (per-query units);
  - fp32 and fp16 pages.
The fixed-shape fast paths (head_dim 64/128, 16-token pages) keep their own tests.
"""
import math
import zlib

import numpy as np
import pytest

import glacier_oracle as orc
import workloads
from gpu_helpers import TOL, gpu_step, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu

# (n_heads, n_kv, head_dim, v_head_dim, block_size, kv dtype, ctx_hi, split pages)
CASES = [
    (2, 1, 32, 32, 8, "f32", 64, 0),       # the reference's GPU parity model
    (2, 1, 32, 64, 4, "f32", 32, 0),       # the reference's asymmetric-V model
    (2, 1, 32, 32, 8, "f16", 64, 2),
    (8, 1, 256, 256, 16, "f32", 300, 0),   # Gemma-like d = 256
    (8, 1, 256, 256, 16, "f16", 300, 3),
    (16, 2, 80, 80, 16, "f32", 500, 2),
    (12, 4, 96, 96, 16, "f16", 500, 0),
    (12, 2, 192, 192, 16, "f32", 200, 0),
    (6, 2, 112, 112, 8, "f32", 300, 2),
    (4, 2, 34, 34, 16, "f32", 200, 0),     # head_dim % 4 == 2: loads of two dims
    (4, 2, 130, 130, 16, "f16", 200, 2),
    (4, 1, 2, 2, 16, "f32", 100, 0),
    (32, 1, 128, 128, 16, "f32", 600, 0),  # MQA: a group of 32 heads, two tiles
    (32, 1, 128, 128, 16, "f16", 600, 2),
    (20, 1, 64, 64, 16, "f32", 400, 1),    # tiles of 16 and 4 heads, one-page splits
    (17, 1, 128, 128, 8, "f32", 300, 3),
    (28, 4, 128, 64, 16, "f32", 400, 2),   # v_head_dim < head_dim
    (28, 4, 64, 128, 16, "f16", 400, 0),   # v_head_dim > head_dim
    (8, 2, 96, 80, 12, "f32", 300, 2),
    (14, 2, 64, 64, 1, "f32", 48, 0),      # one token per page
    (14, 2, 64, 64, 4, "f32", 200, 3),
    (28, 4, 128, 128, 8, "f16", 700, 0),
    (28, 4, 128, 128, 12, "f32", 700, 4),
    # Pool pages above 16 tokens, read as kernel pages (the largest divisor up to 16):
    (28, 4, 128, 128, 32, "f32", 900, 0),  # 16-token parts: the fixed-shape kernel
    (28, 4, 128, 128, 32, "f32", 900, 3),
    (32, 8, 128, 128, 64, "f16", 900, 2),
    (2, 1, 32, 64, 48, "f32", 300, 1),     # v_head_dim != head_dim, 16-token parts
    (8, 2, 64, 64, 24, "f32", 300, 0),     # 12-token parts
    (4, 2, 32, 32, 17, "f16", 100, 2),     # a prime page size: single-token parts
    # Odd widths (the CPU kernel's generic path): loads of one dim.
    (4, 2, 33, 33, 16, "f32", 200, 0),
    (4, 2, 33, 35, 8, "f16", 200, 2),
    (2, 1, 1, 1, 16, "f32", 100, 0),
    (8, 2, 127, 129, 16, "f32", 300, 3),
    (6, 3, 255, 255, 16, "f16", 200, 0),
    (4, 2, 33, 64, 24, "f32", 300, 1),
    (20, 1, 65, 63, 4, "f32", 120, 2),     # odd widths with two tiles of heads
]


def _case_id(c):
    return f"{c[0]}q{c[1]}kv_d{c[2]}_dv{c[3]}_bs{c[4]}_{c[5]}_s{c[7]}"


@pytest.mark.parametrize("case", CASES, ids=_case_id)
def test_general_shapes_match_oracle(torch_mod, gsp, ctx, case):
    torch = torch_mod
    nh, nkv, d, dv, bs, dt, ctx_hi, split = case
    print(f"case shape {_case_id(case)}", flush=True)
    pages = -(-ctx_hi // bs)
    seed = zlib.crc32(_case_id(case).encode()) & 0xFFFF
    step = workloads.small_step(seed=seed, rows=9, n_heads=nh, n_kv=nkv, head_dim=d, kv_dtype=dt, ctx_lo=1,
                                ctx_hi=ctx_hi, total_blocks=9 * pages + 8, block_size=bs, v_head_dim=dv)
    q, k, v = workloads.host_values(step, layers=2)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        for layer in (0, 1):
            got = gpu_step(torch, gsp, ctx, step, q, pool, layer=layer, split_pages=split)
            ref = oracle_step(step, q, k, v, layer=layer)
            assert max_err(got, ref) <= TOL[dt], f"layer {layer}"
    finally:
        pool.destroy()


@pytest.mark.parametrize("shape", [(32, 64, 4, "f32"), (96, 80, 8, "f16"), (128, 128, 8, "f32"), (48, 48, 16, "f32"),
                                   (128, 128, 32, "f32"), (64, 64, 64, "f16"), (128, 128, 24, "f32")],
                         ids=lambda s: f"d{s[0]}_dv{s[1]}_bs{s[2]}_{s[3]}")
def test_prefill_rows_outside_the_tile_shapes(torch_mod, gsp, ctx, shape):
    """Chunked-prefill rows of a pool the prefill tiles do not serve run as per-query
    decode units, causal as the reference runs them (PagedTransformerRunner.cs:454-474).  Pool
    pages of 32 or 64 tokens are read as 16-token kernel pages, which the tiles do serve."""
    torch = torch_mod
    d, dv, bs, dt = shape
    print(f"case prefill shape d={d} dv={dv} bs={bs} {dt}", flush=True)
    q_lens = np.array([1, 24, 7, 1, 40, 0, 16], np.int32)
    step = workloads.small_step(seed=d * 7 + bs, rows=len(q_lens), n_heads=8, n_kv=2, head_dim=d, kv_dtype=dt,
                                ctx_lo=0, ctx_hi=150, total_blocks=512, q_lens=q_lens, block_size=bs,
                                v_head_dim=dv)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        ctx.set_split_pages(2)
        info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                             step.max_seq_len, q_lens=step.q_lens)
        ctx.set_split_pages(0)
        kernel_bs = max(x for x in range(1, 17) if bs % x == 0)
        if not (kernel_bs == 16 and d == dv and d in (64, 128)):
            assert info.prefill_tiles == 0
        else:
            assert info.prefill_tiles > 0
        got = gpu_step(torch, gsp, ctx, step, q, pool)
        ref = oracle_step(step, q, k, v)
        assert max_err(got, ref) <= TOL[dt]
        # Rows with no query tokens leave out untouched.
        rows = np.cumsum(np.concatenate([[0], q_lens]))
        assert np.all(np.isnan(got[rows[5]:rows[6]]))
    finally:
        ctx.set_split_pages(0)
        pool.destroy()


@pytest.mark.parametrize("dims", [(32, 64), (33, 37)], ids=["d32_dv64", "d33_dv37"])
def test_compute_attention_with_asymmetric_v(torch_mod, gsp, ctx, dims):
    """ComputeAttention's argument list with vHeadDim != headDim and 4-token pages, the
    reference's asymmetric model (PhaseCServeRemediationTests.cs:257-319), and odd widths,
    which its generic path takes (PagedAttentionKernel.cs:326-370): out is [nHeads][vHeadDim]."""
    torch = torch_mod
    (d, dv), nh, nkv, bs = dims, 2, 1, 4
    step = workloads.small_step(seed=5, rows=1, n_heads=nh, n_kv=nkv, head_dim=d, ctx_lo=6, ctx_hi=6,
                                total_blocks=8, block_size=bs, v_head_dim=dv)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        qd = torch.from_numpy(q).cuda()
        out = torch.full((nh, dv), float("nan"), device="cuda")
        torch.cuda.synchronize()
        table = step.table(0)
        ctx.compute_attention(0, 0, 5, qd.data_ptr(), out.data_ptr(), table, pool, nh, nkv, d, dv,
                              1.0 / math.sqrt(d), 32, token_count=6)
        ctx.sync()
        ref = orc.compute_attention(orc.HostPool(k, v, block_size=bs), table, 6, 0, 5, q[0], nh,
                                    1.0 / math.sqrt(d), 32)
        assert max_err(out.cpu().numpy().reshape(-1), ref.reshape(-1)) <= TOL["f32"]
        with pytest.raises(gsp.InvalidArgument):  # pos >= maxSeqLen throws in the reference
            ctx.compute_attention(0, 0, 32, qd.data_ptr(), out.data_ptr(), table, pool, nh, nkv, d, dv, 0.1, 32,
                                  token_count=6)
    finally:
        pool.destroy()


def test_unsupported_shapes_are_refused(torch_mod, gsp, ctx):
    torch = torch_mod
    z = torch.zeros(4096, device="cuda")
    with pytest.raises(gsp.Unsupported):  # pages above GSP_MAX_BLOCK_SIZE (4096) tokens
        gsp.Pool.wrap(ctx, z.data_ptr(), z.data_ptr(), 1, 1, 1, 2, block_size=4097)
    big = gsp.Pool.wrap(ctx, z.data_ptr(), z.data_ptr(), 1, 1, 1, 258, block_size=2)
    try:
        ctx.pack_step(big, [0], [1], [0, 1], [0], 16)
        with pytest.raises(gsp.Unsupported):  # above 256, as the reference runner refuses
            ctx.attention_step(big, 0, 1, z.data_ptr(), z.data_ptr(), 0.1)
        general = gsp.Pool.wrap(ctx, z.data_ptr(), z.data_ptr(), 4, 1, 1, 32, block_size=8)
        ctx.pack_step(general, [0], [1], [0, 1], [0], 16)
        ctx.set_decode_path(gsp.DECODE_DPP)
        try:
            with pytest.raises(gsp.Unsupported):  # the DPP kernel keeps its fixed shapes
                ctx.attention_step(general, 0, 1, z.data_ptr(), z.data_ptr(), 0.1)
        finally:
            ctx.set_decode_path(gsp.DECODE_AUTO)
        other = gsp.Pool.wrap(ctx, z.data_ptr(), z.data_ptr(), 4, 1, 1, 32, block_size=4)
        with pytest.raises(gsp.InvalidArgument):  # packed for 8-token pages
            ctx.attention_step(other, 0, 1, z.data_ptr(), z.data_ptr(), 0.1)
        other.destroy()
        general.destroy()
    finally:
        ctx.sync()
        big.destroy()


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_pool_ops_with_asymmetric_v_and_small_pages(torch_mod, gsp, ctx, dt):
    """Store, RoPE + Store and the copy-on-write page copy on a pool with head_dim 32,
    v_head_dim 48 and 4-token pages: every slot lands where the reference layout puts it
    (PagedBlockPool.cs:77-83, 128-161, 304-327)."""
    torch = torch_mod
    nkv, d, dv, bs, blocks, layers = 2, 32, 48, 4, 6, 2
    kind = gsp.KV_F16 if dt == "f16" else gsp.KV_F32
    npdt = np.float16 if dt == "f16" else np.float32
    pool = gsp.Pool.create(ctx, total_blocks=blocks, layers=layers, heads_kv=nkv, head_dim=d, kv_dtype=kind,
                           v_head_dim=dv, block_size=bs)
    rng = np.random.default_rng(3)
    n = 5
    blk = np.array([1, 1, 4, 2, 5], np.int32)
    slot = np.array([0, 3, 2, 1, 3], np.int32)
    pos = np.array([4, 7, 18, 9, 23], np.int32)
    k = rng.standard_normal((n, nkv, d)).astype(np.float32)
    v = rng.standard_normal((n, nkv, dv)).astype(np.float32)
    kd = torch.from_numpy(k).cuda()
    vd = torch.from_numpy(v).cuda()
    torch.cuda.synchronize()
    pool.write_tokens(1, blk[:2], slot[:2], kd.data_ptr(), vd.data_ptr())
    pool.rope_write_tokens(0, pos[2:], blk[2:], slot[2:], 0, 10000.0, gsp.ROPE_PAIRS, 0,
                           kd[2:].data_ptr(), vd[2:].data_ptr())
    pool.copy_block_data(1, 3, 4)
    ctx.sync()
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(npdt).reshape(blocks, layers, nkv, bs, d)
    V = pool.download(1, vb).view(npdt).reshape(blocks, layers, nkv, bs, dv)
    tol = 2e-3 if dt == "f16" else 2e-6
    for i in range(2):
        assert np.array_equal(K[blk[i], 1, :, slot[i]], k[i].astype(npdt))
        assert np.array_equal(V[blk[i], 1, :, slot[i]], v[i].astype(npdt))
    for i in range(2, n):
        ref = orc.rope(k[i], int(pos[i]), 10000.0, 0)
        assert max_err(K[blk[i], 0, :, slot[i]].astype(np.float32), ref) <= tol
        assert np.array_equal(V[blk[i], 0, :, slot[i]], v[i].astype(npdt))
    # The fork copied every layer and head of block 1 into block 3.
    assert np.array_equal(K[3], K[1]) and np.array_equal(V[3], V[1])
    # Nothing else was written.
    written = {(1, 1, 0), (1, 1, 3), (4, 0, 2), (2, 0, 1), (5, 0, 3), (3, 1, 0), (3, 1, 3)}
    for b in range(blocks):
        for lay in range(layers):
            for s in range(bs):
                if (b, lay, s) not in written:
                    assert not K[b, lay, :, s].any() and not V[b, lay, :, s].any(), (b, lay, s)
    pool.destroy()


def test_noalloc_with_tiles_of_heads(torch_mod, gsp, ctx):
    """The allocation-free entry point on a group of 32 heads (two tiles, each with its own
    partials and counters) and a general shape, bit for bit against gsp_attention_step."""
    torch = torch_mod
    step = workloads.small_step(seed=88, rows=6, n_heads=32, n_kv=1, head_dim=96, ctx_lo=50, ctx_hi=500,
                                total_blocks=512, block_size=8, v_head_dim=64)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        ctx.set_split_pages(3)
        info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                             step.max_seq_len)
        ctx.set_split_pages(0)
        assert info.split_pairs > 0
        qd = torch.from_numpy(q).cuda()
        a = torch.full((step.total_q, step.n_heads, step.dv), float("nan"), device="cuda")
        b = torch.full_like(a, float("nan"))
        torch.cuda.synchronize()
        ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), a.data_ptr(), step.scale)
        ctx.sync()
        ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), b.data_ptr(), step.scale)
        ctx.sync()
        assert torch.equal(a, b)
        assert max_err(b.cpu().numpy(), oracle_step(step, q, k, v)) <= TOL["f32"]
    finally:
        ctx.set_split_pages(0)
        pool.destroy()
