"""A packed step captured into a HIP graph and replayed.

gsp_attention_step only launches kernels (and, for a step with both decode
units and prefill tiles, forks the tiles onto a second stream and joins them
back), so an engine may capture it once per packed step shape and replay it.
The split-KV counters return to zero at the end of every launch, so replays
need no reset.  Every replay is checked against the eager result, with eager
work and synchronisations between replays.
"""
import numpy as np
import pytest

import workloads
from gpu_helpers import TOL, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("kind", ["mixed", "decode_split"])
def test_captured_step_replays_match_eager(torch_mod, gsp, ctx, kind):
    torch = torch_mod
    if kind == "mixed":
        q_lens = np.array([1, 24, 1, 40, 1, 3, 1, 17], np.int32)
        step = workloads.small_step(seed=41, rows=8, n_heads=28, n_kv=4, head_dim=128, ctx_hi=300,
                                    total_blocks=512, q_lens=q_lens)
    else:
        step = workloads.small_step(seed=42, rows=16, n_heads=28, n_kv=4, head_dim=128, ctx_lo=100, ctx_hi=900,
                                    total_blocks=1024)
    print(f"graph case {kind}", flush=True)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        ctx.set_split_pages(3 if kind == "decode_split" else 0)
        info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                             q_lens=step.q_lens)
        ctx.set_split_pages(0)
        if kind == "mixed":
            assert info.prefill_tiles > 0 and info.decode_units > 0
        else:
            assert info.split_pairs > 0
        qd = torch.from_numpy(q).cuda()
        eager = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
        with torch.cuda.stream(stream):
            ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
        stream.synchronize()
        ref = oracle_step(step, q, k, v)
        assert max_err(eager.cpu().numpy(), ref) <= TOL[step.kv_dtype]

        out = torch.full_like(eager, float("nan"))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
        for rep in range(4):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} differs from the eager step"
            # Eager work between replays: the same step, run directly.
            with torch.cuda.stream(stream):
                ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
            stream.synchronize()
        del graph
    finally:
        ctx.set_stream(None)  # back to the context's own stream
        pool.destroy()
