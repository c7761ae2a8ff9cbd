"""A packed step, and the projection GEMM's fp16 forms, captured into a HIP graph and replayed.

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


@pytest.mark.parametrize("kind", ["mixed", "decode_split", "decode_group32"])
def test_captured_step_replays_match_eager(torch_mod, gsp, ctx, kind):
    """For a GQA group above 16 (two head tiles) the eager call before the capture grows the split
    workspace to the step's tiles, as the header asks."""
    torch = torch_mod
    if kind == "mixed":
        q_lens = np.array([1, 24, 1, 40, 1, 3, 1, 17], np.int32)
        step = workloads.small_step(seed=41, rows=8, n_heads=28, n_kv=4, head_dim=128, ctx_hi=300,
                                    total_blocks=512, q_lens=q_lens)
    elif kind == "decode_group32":
        step = workloads.small_step(seed=43, rows=9, n_heads=32, n_kv=1, head_dim=128, ctx_lo=100, ctx_hi=900,
                                    total_blocks=1024)
    else:
        step = workloads.small_step(seed=42, rows=16, n_heads=28, n_kv=4, head_dim=128, ctx_lo=100, ctx_hi=900,
                                    total_blocks=1024)
    print(f"graph case {kind}", flush=True)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        ctx.set_split_pages(3 if kind.startswith("decode") else 0)
        info = ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                             q_lens=step.q_lens)
        ctx.set_split_pages(0)
        if kind == "mixed":
            assert info.prefill_tiles > 0 and info.decode_units > 0
        else:
            assert info.split_pairs > 0
        qd = torch.from_numpy(q).cuda()
        eager = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
        torch.cuda.synchronize()  # torch fills on its own stream
        with torch.cuda.stream(stream):
            ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
        stream.synchronize()
        ref = oracle_step(step, q, k, v)
        assert max_err(eager.cpu().numpy(), ref) <= TOL[step.kv_dtype]

        out = torch.full_like(eager, float("nan"))
        ctx.sync()  # the step's upload is known complete: a capture may read it
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


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_capture_that_would_grow_the_workspace_fails_cleanly(torch_mod, gsp):
    """A fresh context packs a group-32 step (workspace sized for one head tile) and captures its
    first gsp_attention_step: the call must refuse with a state error before enqueuing anything,
    and an eager call afterwards must work."""
    torch = torch_mod
    step = workloads.small_step(seed=44, rows=6, n_heads=32, n_kv=1, head_dim=128, ctx_lo=100, ctx_hi=600,
                                total_blocks=512)
    print("graph case capture-without-eager group 32", flush=True)
    q, k, v = workloads.host_values(step)
    with gsp.Context(0) as fresh:
        pool, keep = to_device_pool(torch, gsp, fresh, step, k, v)
        stream = torch.cuda.Stream()
        fresh.set_stream(stream.cuda_stream)
        try:
            fresh.set_split_pages(3)
            info = fresh.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                                   step.max_seq_len)
            assert info.split_pairs > 0
            qd = torch.from_numpy(q).cuda()
            out = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
            fresh.sync()
            torch.cuda.synchronize()
            graph = torch.cuda.CUDAGraph()
            with pytest.raises(gsp.StateError):
                with torch.cuda.graph(graph, stream=stream):
                    fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
            del graph
            torch.cuda.synchronize()
            with torch.cuda.stream(stream):
                fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
            stream.synchronize()
            assert max_err(out.cpu().numpy(), oracle_step(step, q, k, v)) <= TOL[step.kv_dtype]
        finally:
            fresh.set_stream(None)
            pool.destroy()


def _graph_node_types(graph) -> list:
    """Node types of a captured graph (hipGraphNodeType values), read through the HIP
    runtime torch already loaded."""
    import ctypes

    path = next(ln.split()[-1] for ln in open("/proc/self/maps") if "libamdhip64" in ln)
    hip = ctypes.CDLL(path)
    hip.hipGraphGetNodes.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.POINTER(ctypes.c_size_t)]
    hip.hipGraphNodeGetType.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int)]
    handle = ctypes.c_void_p(int(graph.raw_cuda_graph()))
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(handle, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * max(1, n.value))()
    assert hip.hipGraphGetNodes(handle, nodes, ctypes.byref(n)) == 0
    types = []
    for i in range(n.value):
        t = ctypes.c_int(-1)
        assert hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t)) == 0
        types.append(t.value)
    return types


HIP_GRAPH_NODE_KERNEL, HIP_GRAPH_NODE_MEMCPY, HIP_GRAPH_NODE_MEMSET = 0, 1, 2


def test_capture_of_a_step_larger_than_any_earlier(torch_mod, gsp):
    """A fresh context packs a split step and captures it with no eager run first:
    gsp_step_pack sized the workspace, so the capture holds kernels only (no
    memset, copy or event node) and every replay equals the eager step.  A
    capture before gsp_sync (the step's upload not yet known complete), packing,
    and a workspace that would have to grow are refused during the capture."""
    torch = torch_mod
    step = workloads.small_step(seed=44, rows=20, n_heads=28, n_kv=4, head_dim=128, ctx_lo=200, ctx_hi=1500,
                                total_blocks=4096)
    print("graph case fresh-context capture", flush=True)
    q, k, v = workloads.host_values(step)
    fresh = gsp.Context(0)
    pool, keep = to_device_pool(torch, gsp, fresh, step, k, v)
    stream = torch.cuda.Stream()
    fresh.set_stream(stream.cuda_stream)
    try:
        fresh.set_split_pages(4)
        info = fresh.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                               step.max_seq_len)
        fresh.set_split_pages(0)
        assert info.split_pairs > 0
        qd = torch.from_numpy(q).cuda()
        w = torch.randn((64, 4096), device="cuda")
        x = torch.randn((16, 4096), device="cuda")
        y = torch.empty((16, 64), device="cuda")
        out = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
        torch.cuda.synchronize()
        early = torch.cuda.CUDAGraph()
        with torch.cuda.graph(early, stream=stream):
            out.add_(0.0)  # something for the capture to hold
            with pytest.raises(gsp.StateError, match="gsp_sync"):
                fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
        del early
        fresh.sync()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, stream=stream):
            fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
            with pytest.raises(gsp.StateError, match="capturing"):
                fresh.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                                step.max_seq_len)
            # The first split-K product of this context would grow its partials.
            with pytest.raises(gsp.StateError, match="capturing"):
                fresh.matmul_batch(gsp.WTYPE_F32, w.data_ptr(), x.data_ptr(), y.data_ptr(), 4096, 64, 16)
        types = _graph_node_types(graph)
        assert HIP_GRAPH_NODE_KERNEL in types
        assert set(types) == {HIP_GRAPH_NODE_KERNEL}, types
        graph.instantiate()
        # The refused pack left the packed step intact: the eager run after it uses it.
        eager = torch.full_like(out, float("nan"))
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
        stream.synchronize()
        assert max_err(eager.cpu().numpy(), oracle_step(step, q, k, v)) <= TOL[step.kv_dtype]
        for rep in range(3):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} differs from the eager step"
            with torch.cuda.stream(stream):
                fresh.attention_step(pool, 0, step.n_heads, qd.data_ptr(), eager.data_ptr(), step.scale)
            stream.synchronize()
        del graph
    finally:
        fresh.set_stream(None)
        pool.destroy()
        fresh.close()


def _raw_weights(rng, w_type, out_dim, in_dim):
    """Random weight bytes of one GGUF type, valid encodings: random quants and scales with small
    finite fp16 super-block (or block) scales."""
    if w_type == 8:  # Q8_0: fp16 d, then 32 int8
        b = rng.integers(0, 256, (out_dim, in_dim // 32, 34), dtype=np.uint8)
        b[..., 0:2] = (rng.uniform(1e-3, 2e-2, (out_dim, in_dim // 32, 1))).astype(np.float16).view(np.uint8)
    elif w_type == 12:  # Q4_K: fp16 d, fp16 dmin, scales, quants
        b = rng.integers(0, 256, (out_dim, in_dim // 256, 144), dtype=np.uint8)
        b[..., 0:4] = (rng.uniform(1e-4, 2e-2, (out_dim, in_dim // 256, 2))).astype(np.float16).view(np.uint8)
    else:  # Q6_K: quants, scales, then fp16 d
        b = rng.integers(0, 256, (out_dim, in_dim // 256, 210), dtype=np.uint8)
        b[..., 208:210] = (rng.uniform(1e-5, 1e-3, (out_dim, in_dim // 256, 1))).astype(np.float16).view(np.uint8)
    return np.ascontiguousarray(b).reshape(-1)


@pytest.mark.parametrize(
    "w_type, shape",
    [
        (8, (3584, 3584, 64)),    # Q8_0 small-batch form: 8 K ranges merged in the kernel
        (12, (3584, 3584, 64)),   # Q4_K small-batch form
        (14, (3584, 3584, 64)),   # Q6_K small-batch form
        (8, (5120, 1040, 64)),    # Q8_0 small-batch form walking its ranges in two passes
        (12, (2048, 2048, 100)),  # Q4_K fp16 form above 64 rows: pre-pass, product, split-K reduce
        (14, (2048, 2048, 100)),  # Q6_K fp16 form above 64 rows
    ],
    ids=["q8_small", "q4k_small", "q6k_small", "q8_passes", "q4k_large", "q6k_large"],
)
def test_captured_projection_replays_match_eager(torch_mod, gsp, ctx, w_type, shape):
    """gsp_matmul_batch on the fp16 forms, captured after one eager call (which sizes the context's
    buffers) and replayed: the small forms' per-tile counters return to zero at the end of every
    launch, so every replay matches the eager product bit for bit, with eager work between replays,
    and the graph holds kernel nodes only."""
    torch = torch_mod
    in_dim, out_dim, batch = shape
    print(f"graph case matmul type={w_type} {shape}", flush=True)
    rng = np.random.default_rng(1000 + w_type + batch)
    wd = torch.from_numpy(_raw_weights(rng, w_type, out_dim, in_dim)).cuda()
    xd = torch.from_numpy(rng.standard_normal((batch, in_dim)).astype(np.float32)).cuda()
    eager = torch.full((batch, out_dim), float("nan"), device="cuda")
    stream = torch.cuda.Stream()
    ctx.set_stream(stream.cuda_stream)
    try:
        torch.cuda.synchronize()
        with torch.cuda.stream(stream):
            ctx.matmul_batch(w_type, wd.data_ptr(), xd.data_ptr(), eager.data_ptr(), in_dim, out_dim, batch)
        stream.synchronize()
        assert torch.isfinite(eager).all()
        out = torch.full_like(eager, float("nan"))
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph(keep_graph=True)
        with torch.cuda.graph(graph, stream=stream):
            ctx.matmul_batch(w_type, wd.data_ptr(), xd.data_ptr(), out.data_ptr(), in_dim, out_dim, batch)
        types = _graph_node_types(graph)
        assert set(types) == {HIP_GRAPH_NODE_KERNEL}, types
        graph.instantiate()
        for rep in range(4):
            out.fill_(float("nan"))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager), f"replay {rep} differs from the eager product"
            with torch.cuda.stream(stream):
                ctx.matmul_batch(w_type, wd.data_ptr(), xd.data_ptr(), eager.data_ptr(), in_dim, out_dim, batch)
            stream.synchronize()
        del graph
    finally:
        ctx.set_stream(None)
