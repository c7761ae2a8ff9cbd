"""gsp_attention_step_noalloc against gsp_attention_step.

The allocation-free entry point runs the same kernels with the split-KV
partials and counters in the library's fixed per-GPU scratch array; its fp32
prefill tiles split their pages themselves (the step's split records are not
in the array).  Its output must equal gsp_attention_step's bit for bit when
that runs the same kernels (same schedule, same merge order; for fp32 tiles,
a pack told to split in the tiles), stay within the oracle's tolerance and,
against the records form, within it too, on two calls in a row,
the second with a smaller step; a captured noalloc step must replay equal to
the eager one; a step whose workspace exceeds the array is refused before
anything is enqueued.
"""
import numpy as np
import pytest

import workloads
from gpu_helpers import TOL, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu


def _pack(ctx, pool, step, split_pages=0, prefill_split=0):
    ctx.set_split_pages(split_pages)
    ctx.set_prefill_split(prefill_split)
    try:
        return ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                             step.max_seq_len, q_lens=step.q_lens)
    finally:
        ctx.set_split_pages(0)
        ctx.set_prefill_split(0)


def _both(torch, ctx, pool, step, qd):
    """Runs the step through gsp_attention_step, then gsp_attention_step_noalloc."""
    shape = (step.total_q, step.n_heads, step.head_dim)
    ref = torch.full(shape, float("nan"), device="cuda")
    got = torch.full(shape, float("nan"), device="cuda")
    # torch fills on its own stream; the library runs on the context's stream.
    torch.cuda.synchronize()
    ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), ref.data_ptr(), step.scale)
    ctx.sync()
    ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), got.data_ptr(), step.scale)
    ctx.sync()
    return ref.cpu().numpy(), got.cpu().numpy()


@pytest.mark.parametrize("kv_dtype", ["f32", "f16"])
def test_noalloc_matches_attention_step_twice(torch_mod, gsp, ctx, kv_dtype):
    torch = torch_mod
    big = workloads.small_step(seed=71, rows=24, n_heads=28, n_kv=4, head_dim=128, kv_dtype=kv_dtype, ctx_lo=64,
                               ctx_hi=1500, total_blocks=4096)
    small = workloads.small_step(seed=72, rows=5, n_heads=28, n_kv=4, head_dim=128, kv_dtype=kv_dtype, ctx_lo=20,
                                 ctx_hi=400, total_blocks=4096)
    for name, step, split in (("big", big, 5), ("small", small, 3)):
        print(f"noalloc case {kv_dtype} {name}: rows={step.num_rows} split={split}", flush=True)
        q, k, v = workloads.host_values(step)
        pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
        try:
            info = _pack(ctx, pool, step, split)
            assert info.split_pairs > 0  # the scratch partials and counters are in use
            qd = torch.from_numpy(q).cuda()
            ref, got = _both(torch, ctx, pool, step, qd)
            assert np.array_equal(got, ref, equal_nan=True), f"{name}: noalloc differs from gsp_attention_step"
            assert max_err(got, oracle_step(step, q, k, v)) <= TOL[kv_dtype]
        finally:
            pool.destroy()


def test_noalloc_mixed_step_and_repeat(torch_mod, gsp, ctx):
    """Decode units with splits beside prefill tiles, run twice in a row through the scratch."""
    torch = torch_mod
    q_lens = np.array([1, 33, 1, 1, 20, 1], np.int32)
    step = workloads.small_step(seed=73, rows=6, n_heads=28, n_kv=4, head_dim=128, ctx_hi=700, total_blocks=1024,
                                q_lens=q_lens)
    print("noalloc case mixed", flush=True)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    try:
        qd = torch.from_numpy(q).cuda()
        info = _pack(ctx, pool, step, 2)
        assert info.prefill_tiles > 0 and info.split_pairs > 0 and info.split_records > 0
        records, got = _both(torch, ctx, pool, step, qd)
        assert max_err(got, records) <= TOL["f32"]
        info = _pack(ctx, pool, step, 2, prefill_split=1)  # the tiles split their pages, as noalloc's do
        assert info.split_records == 0
        ref, got = _both(torch, ctx, pool, step, qd)
        assert np.array_equal(got, ref, equal_nan=True)
        again = torch.full_like(torch.from_numpy(got).cuda(), float("nan"))
        torch.cuda.synchronize()
        ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), again.data_ptr(), step.scale)
        ctx.sync()
        assert np.array_equal(again.cpu().numpy(), ref, equal_nan=True)
        assert max_err(got, oracle_step(step, q, k, v)) <= TOL["f32"]
    finally:
        pool.destroy()


def test_noalloc_captured_replays_match_eager(torch_mod, gsp, ctx):
    torch = torch_mod
    step = workloads.small_step(seed=74, rows=12, n_heads=28, n_kv=4, head_dim=128, ctx_lo=100, ctx_hi=900,
                                total_blocks=1024)
    print("noalloc case graph", flush=True)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        info = _pack(ctx, pool, step, 3)
        assert info.split_pairs > 0
        qd = torch.from_numpy(q).cuda()
        eager = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
        stream.synchronize()
        out = torch.full_like(eager, float("nan"))
        ctx.sync()  # the step's upload is known complete: a capture may read it
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
        for rep in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} differs from the eager step"
            with torch.cuda.stream(stream):  # eager work through the same scratch between replays
                ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
            stream.synchronize()
        del graph
    finally:
        ctx.set_stream(None)
        pool.destroy()


def test_noalloc_refuses_a_step_beyond_the_scratch(torch_mod, gsp, ctx):
    """One-page splits of a long step need more partials than the array holds."""
    torch = torch_mod
    step = workloads.small_step(seed=75, rows=8, n_heads=28, n_kv=4, head_dim=128, ctx_lo=3000, ctx_hi=4000,
                                total_blocks=2048)
    print("noalloc case oversized", flush=True)
    shape = (step.total_blocks, 1, step.n_kv, 16, step.head_dim)
    kd = torch.zeros(shape, device="cuda")
    vd = torch.zeros(shape, device="cuda")
    pool = gsp.Pool.wrap(ctx, kd.data_ptr(), vd.data_ptr(), step.total_blocks, 1, step.n_kv, step.head_dim)
    try:
        info = _pack(ctx, pool, step, 1)
        need = info.partial_slots * (step.n_heads // step.n_kv) * (step.head_dim + 2) * 4
        assert need > gsp.NOALLOC_SCRATCH_BYTES
        qd = torch.zeros((step.total_q, step.n_heads, step.head_dim), device="cuda")
        out = torch.full((step.total_q, step.n_heads, step.head_dim), 7.0, device="cuda")
        torch.cuda.synchronize()
        with pytest.raises(gsp.InvalidArgument, match="allocation-free"):
            ctx.attention_step_noalloc(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
        ctx.sync()
        assert bool((out == 7.0).all())  # nothing was enqueued
    finally:
        pool.destroy()
