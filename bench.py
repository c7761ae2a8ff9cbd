#!/usr/bin/env python3
"""Benchmark of the ragged continuous-batch paged-attention step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload qwen7b_decode] [--all]

A step is one gsp_attention_step over one packed engine step (one layer, all
rows), with Q, the KV pool and the packed tables already resident in HBM.
Prints ONE JSON line (per workload with --all):
  value        KV GB/s = algorithmic KV bytes / ms_per_step (every valid K/V
               element counted once), unit GB/s
  roofline     the dominant kernel: decode = algorithmic KV bytes / its mean
               launch time (K launches back to back between HIP events on the
               launch stream) vs 8 TB/s; for steps with prefill rows each kernel is
               also timed alone on its rows (roofline_decode, roofline_prefill;
               prefill = 4*d*nH FLOPs per causal (query, key) pair vs the
               157.3 TFLOP/s fp32 matrix peak; the kernel reaches it through
               fp16 matrix cores with hi + lo operand pairs, so its share of
               the fp16 peak is reported too)
  cpu_baseline the CPU oracle (C++ restatement of the reference kernel) timed
               on this host on the same inputs
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "glacier.serve_amd"))

HBM_PEAK_GBS = 8000.0
METRIC = "paged-attn decode KV GB/s (% HBM peak) + seq-steps/sec, Qwen2.5-7B shape"
WORKLOADS = ["qwen05b_decode", "qwen7b_decode", "llama8b_decode", "qwen7b_mixed", "longctx_decode"]
DEFAULT_WORKLOAD = "qwen7b_decode"
KERNEL_NAME = "paged_decode_mfma_kernel"
PREFILL_KERNEL_NAME = "paged_prefill_mfma_kernel"
FP32_MFMA_PEAK_TFS = 157.3  # MI355X dense fp32 matrix peak
FP16_MFMA_PEAK_TFS = 2500.0  # MI355X dense fp16 matrix peak
PREFILL_TILE_MIN_Q = 16     # rows the library runs as prefill tiles by default


def cpu_threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except Exception:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def time_substep(gsp, torch, ctx, stream, pool, sub, q, q_index, steps: int) -> float:
    """Mean ms of one gsp_attention_step over `sub` (a subset of the step's rows,
    same pool; one kernel launch per step): `steps` steps back to back between
    two HIP events on the launch stream."""
    idx = torch.from_numpy(q_index).to(q.device)
    qs = q.index_select(0, idx).contiguous()
    out = torch.empty((sub.total_q, sub.n_heads, sub.head_dim), device=q.device, dtype=torch.float32)
    ctx.pack_step(pool, sub.positions, sub.token_counts, sub.bt_offsets, sub.bt_ids, sub.max_seq_len,
                  q_lens=sub.q_lens)
    for _ in range(3):
        ctx.attention_step(pool, 0, sub.n_heads, qs.data_ptr(), out.data_ptr(), sub.scale)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(steps):
        ctx.attention_step(pool, 0, sub.n_heads, qs.data_ptr(), out.data_ptr(), sub.scale)
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / steps


def profiled_traffic(workload: str, kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary of this workload (profiles/), or None when none is recorded."""
    path = ROOT / "profiles" / f"{kernel}_{workload}.md"
    try:
        for line in path.read_text().splitlines():
            if line.startswith("traffic_bytes_per_launch:"):
                return int(float(line.split(":", 1)[1]))
    except OSError:
        pass
    return None


def describe(step) -> dict:
    import numpy as np

    ctx = step.row_ctx()
    d = {
        "workload": step.name,
        "rows": step.num_rows,
        "query_tokens": step.total_q,
        "heads_q": step.n_heads,
        "heads_kv": step.n_kv,
        "head_dim": step.head_dim,
        "kv_dtype": step.kv_dtype,
        "block_size": 16,
        "pool_blocks": step.total_blocks,
        "ctx_min": int(ctx.min()),
        "ctx_mean": round(float(ctx.mean()), 1),
        "ctx_max": int(ctx.max()),
        "kv_tokens": step.kv_tokens(),
        "kv_bytes": step.kv_bytes(),
        "seed": int(step.seed),
    }
    if step.q_lens is not None and int(np.max(step.q_lens)) > 1:
        d["prefill_rows"] = int((step.q_lens > 1).sum())
        d["prefill_gflop"] = round(step.prefill_flops() / 1e9, 3)
    return d


def run_workload(name: str, steps: int, warmup: int, cpu: bool, cpu_budget_s: float) -> dict:
    import numpy as np
    import torch

    import glacier_paged as gsp
    import workloads

    step = getattr(workloads, name)()
    q, k, v = workloads.device_values(torch, step)
    torch.cuda.synchronize()
    ctx = gsp.Context(0)
    # A dedicated torch stream: the library launches on it and the events below
    # are recorded on it (torch's default stream is the null handle).
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    pool = gsp.Pool.wrap(ctx, k.data_ptr(), v.data_ptr(), step.total_blocks, 1, step.n_kv, step.head_dim,
                         gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32)
    out = torch.empty((step.total_q, step.n_heads, step.head_dim), device="cuda", dtype=torch.float32)

    def pack():
        return ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                             q_lens=step.q_lens)

    def attend():
        ctx.attention_step(pool, 0, step.n_heads, q.data_ptr(), out.data_ptr(), step.scale)

    info = pack()
    for _ in range(warmup):
        attend()
    torch.cuda.synchronize()

    # Timed region: K steps back to back, events on the launch stream.
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(steps):
        attend()
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = e0.elapsed_time(e1) / steps

    # A decode-only step is one launch of the decode kernel, so its mean launch
    # duration over the timed region is ms_per_step.  (Events around every
    # launch would add their own gaps; rocprofv3's kernel trace agrees with
    # ms_per_step to about 1%.)
    kernel_ms = ms_per_step

    # Engine-step time: pinned pack + one H2D copy + kernel, host-synchronous per step.
    n_step = max(10, steps // 4)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(n_step):
        pack()
        attend()
    torch.cuda.synchronize()
    t_step_ms = (time.perf_counter() - t0) * 1e3 / n_step

    # Distribution of single steps: each between its own events on the launch
    # stream and waited for alone, so it includes one launch's start-up that the
    # back-to-back mean hides.  Reported beside ms_per_step, never as value.
    singles = []
    for _ in range(max(20, min(200, steps))):
        a0 = torch.cuda.Event(enable_timing=True)
        a1 = torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        attend()
        a1.record(stream)
        a1.synchronize()
        singles.append(a0.elapsed_time(a1))
    p10, p50, p90 = (float(x) for x in np.percentile(singles, [10, 50, 90]))

    kv_bytes = step.kv_bytes()
    gbs = kv_bytes / (ms_per_step * 1e-3) / 1e9
    kernel_gbs = kv_bytes / (kernel_ms * 1e-3) / 1e9
    got = out.cpu().numpy()

    decode_roof = {
        "bound": "hbm",
        "kernel": KERNEL_NAME,
        "achieved": round(kernel_gbs, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(kernel_gbs / HBM_PEAK_GBS, 4),
        "traffic": profiled_traffic(name, KERNEL_NAME),
        "algorithmic_bytes_per_launch": kv_bytes,
        "mean_launch_ms": round(kernel_ms, 5),
    }
    roofline = decode_roof
    extra = {}
    tiled = np.nonzero(step.lens >= PREFILL_TILE_MIN_Q)[0]
    if len(tiled):
        # Rows of both kinds: time each kernel alone on its rows' sub-step
        # (one launch of one kernel per step), and report the longer one.
        rows_d = np.nonzero(step.lens < PREFILL_TILE_MIN_Q)[0]
        sub_p, qi_p = step.subset(tiled)
        pre_ms = time_substep(gsp, torch, ctx, stream, pool, sub_p, q, qi_p, steps)
        flops = sub_p.prefill_flops()
        tfs = flops / (pre_ms * 1e-3) / 1e12
        products = 3 if step.kv_dtype == "f32" else 2
        prefill_roof = {
            "bound": "mfma",
            "kernel": PREFILL_KERNEL_NAME,
            "achieved": round(tfs, 2),
            "peak": FP32_MFMA_PEAK_TFS,
            "unit": "TFLOP/s",
            "frac": round(tfs / FP32_MFMA_PEAK_TFS, 4),
            "traffic": profiled_traffic(name, PREFILL_KERNEL_NAME),
            "algorithmic_flops_per_launch": int(flops),
            "mean_launch_ms": round(pre_ms, 5),
            # The algorithm is fp32 and `frac` is against the fp32 matrix peak.  The
            # kernel runs it on the fp16 matrix cores with operands split into hi + lo
            # fp16 pairs: `products` fp16 products per fp32 one, so it can pass the
            # fp32 peak; this is the same work against the fp16 matrix peak.
            "matrix_unit": "fp16 (operands as hi + lo fp16 pairs)",
            "products_per_fp32_product": products,
            "frac_of_fp16_matrix_peak": round(tfs * products / FP16_MFMA_PEAK_TFS, 4),
        }
        if len(rows_d):
            sub_d, qi_d = step.subset(rows_d)
            dec_ms = time_substep(gsp, torch, ctx, stream, pool, sub_d, q, qi_d, steps)
            dgbs = sub_d.kv_bytes() / (dec_ms * 1e-3) / 1e9
            decode_roof.update({"achieved": round(dgbs, 1), "frac": round(dgbs / HBM_PEAK_GBS, 4),
                                "algorithmic_bytes_per_launch": sub_d.kv_bytes(), "mean_launch_ms": round(dec_ms, 5),
                                "rows": "decode rows alone"})
        else:
            dec_ms = 0.0
        extra["roofline_decode"] = decode_roof
        extra["roofline_prefill"] = prefill_roof
        roofline = prefill_roof if pre_ms >= dec_ms else decode_roof

    result = {
        "metric": METRIC,
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": step.kv_dtype,
        "data": "synthetic: Q, K, V ~ N(0,1) drawn on the GPU from the recorded seed",
        "config": describe(step),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
        "seq_steps_per_s": round(step.num_rows / (ms_per_step * 1e-3), 1),
        "t_step_ms_incl_pack_upload": round(t_step_ms, 5),
        "single_step_ms": {"p10": round(p10, 5), "median": round(p50, 5), "p90": round(p90, 5),
                           "samples": len(singles), "note": "one step at a time, each waited for"},
        "seq_steps_per_s_incl_pack_upload": round(step.num_rows / (t_step_ms * 1e-3), 1),
        "kv_gbs_incl_pack_upload": round(kv_bytes / (t_step_ms * 1e-3) / 1e9, 1),
        "wall_ms_timed_region": round(wall_ms, 3),
        "step_info": {"decode_units": info.decode_units, "split_pairs": info.split_pairs,
                      "partial_slots": info.partial_slots, "pages_per_split": info.pages_per_split,
                      "packed_pages": info.packed_pages, "staging_bytes": int(info.staging_bytes)},
        "roofline": roofline,
    }
    result.update(extra)
    result["host_prefix_cache"] = host_prefix_cache(gsp, step)
    result["rope_write"] = rope_write_timing(gsp, torch, ctx, stream, step)
    result["matmul"] = matmul_timing(gsp, torch, ctx, stream, step)

    if cpu:
        result["cpu_baseline"], ref = cpu_baseline(step, q, k, v, cpu_budget_s)
        err = float(np.nanmax(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
        tol = 2e-3 if step.kv_dtype == "f16" else 1e-4
        result["parity"] = {"max_abs_err_vs_oracle": err, "tol": tol, "ok": bool(err <= tol)}
    pool.destroy()
    ctx.close()
    return result


def matmul_timing(gsp, torch, ctx, stream, step, calls: int = 50) -> dict:
    """Device cost of the step's Q projection (QuantKernels.MatMulBatch, PagedTransformerRunner.cs:601):
    hidden = n_heads * head_dim in and out, one batch row per query token of the step, random
    weights as Q8_0 and as F32.  The products are fp32 on the fp32 matrix cores, so the roofline
    is 157.3 TFLOP/s; weight streaming bounds it only for small batches."""
    hidden = step.n_heads * step.head_dim
    batch = int(step.total_q)
    gen = torch.Generator(device="cuda").manual_seed(step.seed)
    x = torch.randn((batch, hidden), device="cuda", generator=gen)
    y = torch.empty((batch, hidden), device="cuda")
    nb = hidden // 32
    d = (torch.randn((hidden, nb, 1), device="cuda", generator=gen) * 0.01).half().view(torch.uint8)
    q = torch.randint(-127, 128, (hidden, nb, 32), device="cuda", generator=gen, dtype=torch.int8).view(torch.uint8)
    weights = {"q8_0": (gsp.WTYPE_Q8_0, torch.cat([d, q], dim=2).contiguous(), hidden * nb * 34),
               "f32": (gsp.WTYPE_F32, torch.randn((hidden, hidden), device="cuda", generator=gen), hidden * hidden * 4)}
    torch.cuda.synchronize()
    flops = 2.0 * batch * hidden * hidden
    out = {"in_dim": hidden, "out_dim": hidden, "batch": batch}
    for name, (wt, w, wbytes) in weights.items():
        args = (wt, w.data_ptr(), x.data_ptr(), y.data_ptr(), hidden, hidden, batch)
        with torch.cuda.stream(stream):
            for _ in range(5):
                ctx.matmul_batch(*args)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(calls):
                ctx.matmul_batch(*args)
            e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / calls * 1e3
        out[name] = {"us_per_call": round(us, 2), "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                     "frac_fp32_matrix_peak": round(flops / (us * 1e-6) / 1e12 / 157.3, 4),
                     "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1)}
    return out


def rope_write_timing(gsp, torch, ctx, stream, step, calls: int = 100) -> dict:
    """Device cost of the step's K/V write with RoPE (QuantKernels.RoPE then
    PagedBlockPool.Store, PagedTransformerRunner.cs:620-634, fused): one new token
    per decode row and the chunk's tokens for prefill rows, into a scratch pool of
    the step's geometry.  Each call restages positions, blocks and slots from the
    host, as an engine tick does."""
    import numpy as np

    n = step.total_q
    pos = np.concatenate([int(p) + np.arange(int(l)) for p, l in zip(step.positions, step.lens)]).astype(np.int32)
    blocks = (np.arange(n) // 16).astype(np.int32)
    slots = (np.arange(n) % 16).astype(np.int32)
    pool = gsp.Pool.create(ctx, total_blocks=int(blocks[-1]) + 1, layers=1, heads_kv=step.n_kv, head_dim=step.head_dim,
                           kv_dtype=gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32)
    gen = torch.Generator(device="cuda").manual_seed(step.seed)
    q = torch.randn((n, step.n_heads, step.head_dim), device="cuda", generator=gen)
    k = torch.randn((n, step.n_kv, step.head_dim), device="cuda", generator=gen)
    v = torch.randn((n, step.n_kv, step.head_dim), device="cuda", generator=gen)
    args = (0, pos, blocks, slots, step.n_heads, 1000000.0, gsp.ROPE_HALVES, q.data_ptr(), k.data_ptr(), v.data_ptr())
    with torch.cuda.stream(stream):
        for _ in range(5):
            pool.rope_write_tokens(*args)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(calls):
            pool.rope_write_tokens(*args)
        e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / calls * 1e3
    elem = 2 if step.kv_dtype == "f16" else 4
    moved = n * (2 * step.n_heads * step.head_dim * 4 + 2 * step.n_kv * step.head_dim * 4
                 + 2 * step.n_kv * step.head_dim * elem)
    pool.destroy()
    return {"tokens": n, "us_per_call": round(us, 2), "bytes_per_call": moved,
            "gbs": round(moved / (us * 1e-6) / 1e9, 1),
            "note": "Q rotated in place, K rotated and stored, V stored; includes the per-call host staging"}


def host_prefix_cache(gsp, step) -> dict:
    """Host cost of the prefix cache for this step's rows: the XXH3 hash chain
    over every full 16-token block of every row (what admitting those prompts
    costs, ContinuousBatchEngine.cs:223-263), and a cache lookup per block."""
    import numpy as np

    rng = np.random.default_rng(step.seed)
    blocks = int(sum(int(t) // 16 for t in step.token_counts))
    tokens = rng.integers(0, 150000, size=max(16, blocks * 16), dtype=np.int64).astype(np.int32)
    alloc = gsp.BlockAllocator(max(1, blocks), 16)
    gsp.prefix_hash_chain(0, tokens[:16])  # load and warm
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        hashes = gsp.prefix_hash_chain(0, tokens[:blocks * 16])  # one call per step's worth of blocks
    t1 = time.perf_counter()
    for h in hashes[:2000]:
        alloc.try_find_prefix_block(int(h))
    t2 = time.perf_counter()
    alloc.close()
    n = max(1, blocks)
    return {"blocks": blocks, "hash_ns_per_block": round((t1 - t0) / (reps * n) * 1e9, 1),
            "hash_gbs": round(reps * n * 64 / (t1 - t0) / 1e9, 2),
            "find_us_per_call": round((t2 - t1) / max(1, min(2000, len(hashes))) * 1e6, 3),
            "note": "one host thread; the chain is one C call, finds go through the Python binding per call"}


def cpu_baseline(step, q, k, v, budget_s: float):
    """Times the CPU oracle (C++ restatement of PagedAttentionKernel.ComputeAttention,
    called per row like PagedTransformerRunner.ForwardBatch, Parallel.For over query
    heads) on the same inputs.  Returns (record, oracle output)."""
    import numpy as np
    import torch

    sys.path.insert(0, str(ROOT / "oracle"))
    import glacier_oracle as orc

    # The oracle reads only the pages the step uses: gather and upcast them.
    used, inv = np.unique(step.bt_ids, return_inverse=True)
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    kh = k.index_select(0, idx).float().cpu().numpy()
    vh = v.index_select(0, idx).float().cpu().numpy()
    qh = q.cpu().numpy()
    ids = inv.astype(np.int32)
    pool = orc.HostPool(kh, vh)
    nt = cpu_threads()
    out = np.zeros((step.total_q, step.n_heads, step.head_dim), np.float32)

    def one():
        orc.attention_step(pool, 0, step.positions, step.token_counts, step.bt_offsets, ids, qh, step.n_heads,
                           step.scale, step.max_seq_len, q_lens=step.q_lens, out=out, n_threads=nt)

    one()  # warm-up (also the parity reference)
    times = []
    t_start = time.perf_counter()
    while len(times) < 20 and (time.perf_counter() - t_start) < budget_s:
        t0 = time.perf_counter()
        one()
        times.append(time.perf_counter() - t0)
    med = statistics.median(times)
    rec = {
        "value": round(step.kv_bytes() / med / 1e9, 3),
        "unit": "GB/s",
        "cores": nt,
        "kind": "port",
        "sample": f"whole {step.name} step ({step.num_rows} rows), median of {len(times)} steps "
                  f"(budget {budget_s:.0f} s), {nt} threads on '{cpu_model()}', ISA level {orc.host_isa()} "
                  f"(2=AVX-512, 1=AVX2); C++ restatement of the reference C# kernel",
        "ms_per_step": round(med * 1e3, 3),
        "seq_steps_per_s": round(step.num_rows / med, 1),
    }
    return rec, out.copy()


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default=DEFAULT_WORKLOAD, choices=WORKLOADS)
    ap.add_argument("--all", action="store_true", help="one line per workload")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-budget", type=float, default=20.0, help="seconds of CPU baseline timing")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="also run a device copy of this many MiB (a known-size kernel that scales "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this path is not sharded across GPUs "
              "in this build", file=sys.stderr)
        return 2
    names = WORKLOADS if args.all else [args.workload]
    for name in names:
        res = run_workload(name, args.steps, args.warmup, cpu=not args.no_cpu, cpu_budget_s=args.cpu_budget)
        print(json.dumps(res), flush=True)
    if args.copy_calibration > 0:
        import torch

        n = args.copy_calibration * (1 << 20) // 4
        src = torch.ones(n, device="cuda", dtype=torch.float32)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_calibration_bytes_read": n * 4, "copy_calibration_bytes_written": n * 4}),
              file=sys.stderr, flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
