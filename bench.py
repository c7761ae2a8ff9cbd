#!/usr/bin/env python3
"""Benchmark of the ragged continuous-batch paged-attention step on one MI355X.

    python bench.py [--steps K] [--warmup W] [--workload qwen7b_decode] [--all] [--layers L]
    python bench.py --summarize-trace KERNEL_TRACE.csv --kernel NAME --last K
    python bench.py --summarize-pmc COUNTER_COLLECTION.csv --kernel NAME --last K

A step is one gsp_attention_step over one packed engine step (one layer, all
rows), with Q, the KV pool and the packed tables already resident in HBM.
The pool holds L layers (default 4) and step i attends layer i mod L, as the
layers of an engine tick do, so no step re-reads pages that an earlier step
left in the 256 MB Infinity Cache.  Prints ONE JSON line (per workload with
--all):
  value        KV GB/s = algorithmic KV bytes / ms_per_step (every valid K/V
               element counted once), unit GB/s
  roofline     the dominant kernel: decode = algorithmic KV bytes / its mean
               launch time (K launches back to back between HIP events on the
               launch stream) vs 8 TB/s; for steps with prefill rows each kernel is
               also timed alone on its rows (roofline_decode, roofline_prefill).
               The prefill kernel computes fp32 attention (4*d*nH FLOPs per
               causal (query, key) pair) on the fp16 matrix cores as hi + lo
               operand pairs, 3 fp16 products per fp32 product (2 for fp16
               pages): its roofline is those fp16 products against the
               2.5 PFLOP/s dense fp16 matrix peak.
  stream_ceiling  (decode-only steps) a plain non-temporal streaming read of
               the same bytes, over L buffers in turn and timed the same way,
               on the same GPU in the same run: what this GPU streams cold at
               all, and the decode kernel's rate as a share of it
  cpu_baseline the CPU oracle (C++ restatement of the reference kernel) timed
               on this host on the same inputs
--profile-only runs only the packed step's warmup and timed launches (and, for
steps with prefill rows, each kernel alone on its rows), so that a rocprofv3
trace of it holds exactly those launches; --summarize-trace / --summarize-pmc
then average the last K launches of a kernel in that trace or counter file.
"""
from __future__ import annotations

import argparse
import gc
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
WORKLOADS = ["qwen05b_decode", "qwen7b_decode", "llama8b_decode", "qwen7b_mixed", "longctx_decode",
             "refmodel_decode"]
DEFAULT_WORKLOAD = "qwen7b_decode"
KERNEL_NAME = "paged_decode_mfma_kernel"
PREFILL_KERNEL_NAME = "paged_prefill_mfma_kernel"
FP32_MFMA_PEAK_TFS = 157.3  # MI355X dense fp32 matrix peak
FP16_MFMA_PEAK_TFS = 2500.0  # MI355X dense fp16 matrix peak
PREFILL_TILE_MIN_Q = 16     # rows the library runs as prefill tiles by default


# Host threads a job may use per GPU on the measurement hosts: their CPU share
# is 16 cores per GPU, whatever sched_getaffinity shows.
HOST_CPU_SHARE = 16
CPU_WARMUP_STEPS = 5  # untimed CPU baseline steps before the timed ones


def visible_cores() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except Exception:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """Every core this process may run on, up to the host's per-GPU CPU share."""
    return max(1, min(HOST_CPU_SHARE, visible_cores()))


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except Exception:
        pass
    return "unknown"


def time_substep(gsp, torch, ctx, stream, pool, sub, q, q_index, steps: int, layers: int) -> float:
    """Mean ms of one gsp_attention_step over `sub` (a subset of the step's rows,
    same pool; one kernel launch per step): `steps` steps back to back between
    two HIP events on the launch stream, step i on layer i mod `layers`."""
    idx = torch.from_numpy(q_index).to(q.device)
    qs = q.index_select(0, idx).contiguous()
    out = torch.empty((sub.total_q, sub.n_heads, sub.head_dim), device=q.device, dtype=torch.float32)
    ctx.pack_step(pool, sub.positions, sub.token_counts, sub.bt_offsets, sub.bt_ids, sub.max_seq_len,
                  q_lens=sub.q_lens)
    for i in range(3):
        ctx.attention_step(pool, i % layers, sub.n_heads, qs.data_ptr(), out.data_ptr(), sub.scale)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    # One untimed step ahead of e0 (on layer L - 1, so that step 0 stays cold):
    # the device is busy while the host issues the first timed launch, so e0
    # does not time the host's launch latency.
    ctx.attention_step(pool, layers - 1, sub.n_heads, qs.data_ptr(), out.data_ptr(), sub.scale)
    e0.record(stream)
    for i in range(steps):
        ctx.attention_step(pool, i % layers, sub.n_heads, qs.data_ptr(), out.data_ptr(), sub.scale)
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
                return int(float(line.split(":", 1)[1].split()[0]))
    except OSError:
        pass
    return None


def describe(step, layers: int) -> dict:
    import numpy as np

    ctx = step.row_ctx()
    d = {
        "workload": step.name,
        "rows": step.num_rows,
        "query_tokens": step.total_q,
        "heads_q": step.n_heads,
        "heads_kv": step.n_kv,
        "head_dim": step.head_dim,
        "v_head_dim": step.dv,
        "kv_dtype": step.kv_dtype,
        "block_size": step.block_size,
        "pool_blocks": step.total_blocks,
        "pool_layers": layers,
        "layer_per_step": "step i attends layer i mod pool_layers",
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


def run_workload(name: str, steps: int, warmup: int, cpu: bool, cpu_budget_s: float, layers: int = 4,
                 decode_path: str = "auto", profile_only: bool = False, prefill_split: str = "records",
                 split_pages: int = 0, decode_bins: int = 0) -> dict:
    import numpy as np
    import torch

    import glacier_paged as gsp
    import workloads

    step = getattr(workloads, name)()
    q, k, v = workloads.device_values(torch, step, layers=layers)
    torch.cuda.synchronize()
    ctx = gsp.Context(0)
    ctx.set_decode_path({"auto": gsp.DECODE_AUTO, "dpp": gsp.DECODE_DPP, "mfma": gsp.DECODE_MFMA}[decode_path])
    ctx.set_prefill_split({"records": gsp.SPLIT_RECORDS, "in_tile": gsp.SPLIT_IN_TILE}[prefill_split])
    ctx.set_split_pages(split_pages)  # 0: the library's own choice
    ctx.set_decode_bins(decode_bins)
    # A dedicated torch stream: the library launches on it and the events below
    # are recorded on it (torch's default stream is the null handle).
    stream = torch.cuda.Stream()
    torch.cuda.set_stream(stream)
    ctx.set_stream(stream.cuda_stream)
    pool = gsp.Pool.wrap(ctx, k.data_ptr(), v.data_ptr(), step.total_blocks, layers, step.n_kv, step.head_dim,
                         gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32, v_head_dim=step.dv,
                         block_size=step.block_size)
    out = torch.empty((step.total_q, step.n_heads, step.dv), device="cuda", dtype=torch.float32)

    def pack():
        return ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                             q_lens=step.q_lens)

    def attend(layer):
        ctx.attention_step(pool, layer, step.n_heads, q.data_ptr(), out.data_ptr(), step.scale)

    info = pack()
    for i in range(warmup):
        attend(i % layers)
    torch.cuda.synchronize()

    # Timed region: K steps back to back, step i on layer i mod L, events on the
    # launch stream.
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    # One untimed step ahead of e0 (on layer L - 1, so that step 0 stays cold):
    # the device is busy while the host issues the first timed launch, so e0
    # does not time the host's launch latency.  The wall clock covers it.
    attend(layers - 1)
    e0.record(stream)
    for i in range(steps):
        attend(i % layers)
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    ms_per_step = e0.elapsed_time(e1) / steps

    # A decode-only step is one launch of the decode kernel, so its mean launch
    # duration over the timed region is ms_per_step.
    kernel_ms = ms_per_step
    kv_bytes = step.kv_bytes()
    gbs = kv_bytes / (ms_per_step * 1e-3) / 1e9

    decode_roof = {
        "bound": "hbm",
        "kernel": KERNEL_NAME if decode_path != "dpp" else "paged_decode_kernel",
        "achieved": round(kv_bytes / (kernel_ms * 1e-3) / 1e9, 1),
        "peak": HBM_PEAK_GBS,
        "unit": "GB/s",
        "frac": round(kv_bytes / (kernel_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
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
        pre_ms = time_substep(gsp, torch, ctx, stream, pool, sub_p, q, qi_p, steps, layers)
        flops = sub_p.prefill_flops()
        tfs = flops / (pre_ms * 1e-3) / 1e12
        products = 3 if step.kv_dtype == "f32" else 2
        prefill_roof = {
            "bound": "mfma",
            "kernel": PREFILL_KERNEL_NAME,
            # fp16 matrix-core products per second: fp32 attention runs as
            # `products` fp16 products (hi + lo operand pairs) per fp32 product.
            "achieved": round(tfs * products, 2),
            "peak": FP16_MFMA_PEAK_TFS,
            "unit": "TFLOP/s",
            "frac": round(tfs * products / FP16_MFMA_PEAK_TFS, 4),
            "traffic": profiled_traffic(name, PREFILL_KERNEL_NAME),
            "algorithmic_flops_per_launch": int(flops),
            "fp16_products_per_fp32_product": products,
            "fp32_attention_tflops": round(tfs, 2),
            "mean_launch_ms": round(pre_ms, 5),
            # fp32 pages: "records" times the split-record kernel and the tiles together.
            "prefill_split": prefill_split if step.kv_dtype == "f32" else "none",
        }
        if len(rows_d):
            sub_d, qi_d = step.subset(rows_d)
            dec_ms = time_substep(gsp, torch, ctx, stream, pool, sub_d, q, qi_d, steps, layers)
            dgbs = sub_d.kv_bytes() / (dec_ms * 1e-3) / 1e9
            decode_roof.update({"achieved": round(dgbs, 1), "frac": round(dgbs / HBM_PEAK_GBS, 4),
                                "algorithmic_bytes_per_launch": sub_d.kv_bytes(), "mean_launch_ms": round(dec_ms, 5),
                                "rows": "decode rows alone"})
        else:
            dec_ms = 0.0
        extra["roofline_decode"] = decode_roof
        extra["roofline_prefill"] = prefill_roof
        extra["mixed_vs_parts"] = round(ms_per_step / (pre_ms + dec_ms), 4)
        roofline = prefill_roof if pre_ms >= dec_ms else decode_roof
        pack()  # the full step again, for what follows

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
        "config": describe(step, layers),
        "pct_hbm_peak": round(100.0 * gbs / HBM_PEAK_GBS, 2),
    }
    if profile_only:
        result["roofline"] = roofline
        result.update(extra)
        pool.destroy()
        ctx.close()
        return result

    # Engine-step time t_step: the host pack (validation, scheduling, one
    # pinned staging buffer and one host-to-device copy) plus the attention of
    # one layer, issued back to back as an engine loop issues them.  Step i+1
    # is packed on the host while step i's kernel runs; its copy follows that
    # kernel on the stream.
    # t_step is the median period of the loop once it is in steady state (host
    # hiccups of a millisecond show up in the mean, reported beside it).
    n_step = max(40, steps)
    for i in range(5):
        pack()
        attend(i % layers)
    pack_ns, wait_ns, periods = [], [], []
    torch.cuda.synchronize()
    t0 = t_prev = time.perf_counter()
    for i in range(n_step):
        info_i = pack()
        attend(i % layers)
        t_now = time.perf_counter()
        periods.append(t_now - t_prev)
        t_prev = t_now
        pack_ns.append(info_i.pack_host_ns)
        wait_ns.append(info_i.pack_wait_ns)
    torch.cuda.synchronize()
    t_step_mean_ms = (time.perf_counter() - t0) * 1e3 / n_step
    t_step_ms = float(np.median(periods[n_step // 4:])) * 1e3
    # The step's upload on the device: events around the pack's copy kernel, each enqueued
    # behind a running attention step (the host packs while that kernel runs), so the interval
    # is the copy kernel with its launch and the two events' own latency, not the host's packing.
    ups = []
    for i in range(20):
        attend(i % layers)
        u0 = torch.cuda.Event(enable_timing=True)
        u1 = torch.cuda.Event(enable_timing=True)
        u0.record(stream)
        pack()
        u1.record(stream)
        ups.append((u0, u1))
    torch.cuda.synchronize()
    upload_us = float(np.median([a.elapsed_time(b) for a, b in ups])) * 1e3

    # Distribution of single steps: each between its own events on the launch
    # stream and waited for alone, so it includes one launch's start-up that the
    # back-to-back mean hides.  Reported beside ms_per_step, never as value.
    singles = []
    for i in range(max(20, min(200, steps))):
        a0 = torch.cuda.Event(enable_timing=True)
        a1 = torch.cuda.Event(enable_timing=True)
        a0.record(stream)
        attend(i % layers)
        a1.record(stream)
        a1.synchronize()
        singles.append(a0.elapsed_time(a1))
    p10, p50, p90 = (float(x) for x in np.percentile(singles, [10, 50, 90]))

    # The output checked against the oracle: layer 0.
    attend(0)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    result.update({
        "seq_steps_per_s": round(step.num_rows / (t_step_ms * 1e-3), 1),
        "t_step_ms": round(t_step_ms, 5),
        "t_step_breakdown": {
            "definition": "seq_steps_per_s = B / t_step; t_step = one engine step: host pack (one upload) + "
                          "one layer's attention, issued back to back through the Python binding; median period",
            "t_step_ms_mean": round(t_step_mean_ms, 5),
            "t_step_ms_p90": round(float(np.percentile(periods[n_step // 4:], 90)) * 1e3, 5),
            "t_step_ms_max": round(max(periods) * 1e3, 3),
            "pack_host_us_median": round(float(np.median(pack_ns)) / 1e3, 2),
            "pack_wait_us_median": round(float(np.median(wait_ns)) / 1e3, 2),
            "pack_work_us_median": round(float(np.median(np.array(pack_ns) - np.array(wait_ns))) / 1e3, 2),
            "upload_interval_us_median": round(upload_us, 2),
            "kernel_ms": round(kernel_ms, 5),
            "step_overhead_us": round(t_step_ms * 1e3 - kernel_ms * 1e3, 2),
            "notes": "pack_host = pack_work (validation, plan, staging; on the host while the previous step's "
                     "kernel runs) + pack_wait (the host, ahead of the GPU, waiting for the staging slot's "
                     "upload of two steps before: back-pressure, off the device's path); step_overhead = "
                     "t_step - kernel_ms is what the device spends per step beyond the attention kernel (the "
                     "upload copy kernel and launch gaps); upload_interval brackets the copy kernel with two "
                     "events and so also holds their latency",
            "steps": n_step,
        },
        "seq_steps_per_s_kernel_only": round(step.num_rows / (ms_per_step * 1e-3), 1),
        "kv_gbs_incl_pack_upload": round(kv_bytes / (t_step_ms * 1e-3) / 1e9, 1),
        "single_step_ms": {"p10": round(p10, 5), "median": round(p50, 5), "p90": round(p90, 5),
                           "samples": len(singles), "note": "one step at a time, each waited for"},
        "wall_ms_timed_region": round(wall_ms, 3),
        "step_info": {"decode_units": info.decode_units, "split_pairs": info.split_pairs,
                      "partial_slots": info.partial_slots, "pages_per_split": info.pages_per_split,
                      "packed_pages": info.packed_pages, "staging_bytes": int(info.staging_bytes),
                      "decode_bins": info.decode_bins, "prefill_tiles": info.prefill_tiles},
        "roofline": roofline,
    })
    result.update(extra)
    if not len(tiled):
        ceiling = stream_ceiling(torch, stream, kv_bytes, layers, steps)
        ceiling["decode_vs_ceiling"] = round(gbs / ceiling["gbs"], 4)
        result["stream_ceiling"] = ceiling
    if cpu:
        result["cpu_baseline"], ref = cpu_baseline(step, q, k, v, cpu_budget_s)
        err = float(np.nanmax(np.abs(got.astype(np.float64) - ref.astype(np.float64))))
        tol = 2e-3 if step.kv_dtype == "f16" else 1e-4
        result["parity"] = {"max_abs_err_vs_oracle": err, "tol": tol, "ok": bool(err <= tol)}
    result["host_prefix_cache"] = host_prefix_cache(gsp, step)
    # Last, since it writes new K/V into the pool at each row's newest position.
    result["kv_write"] = kv_write_timing(gsp, torch, ctx, stream, step, pool, layers)
    result["matmul"] = matmul_timing(gsp, torch, ctx, stream, step)
    pool.destroy()
    ctx.close()
    return result


def stream_ceiling(torch, stream, nbytes: int, layers: int, steps: int) -> dict:
    """A plain non-temporal 16-byte streaming read of nbytes (libglacier_probe.so),
    over `layers` buffers in turn as the decode steps rotate layers, with one
    untimed launch ahead of the first event and `steps` launches back to back:
    the decode timing's bracket around a kernel that only streams.  Best of nine
    launch shapes (grids 512, 1024, 2048 x 2, 4, 8 loads in flight per lane)."""
    import ctypes

    lib = ctypes.CDLL(str(ROOT / "glacier.serve_amd" / "libglacier_probe.so"))
    fn = lib.gsp_probe_stream_read
    fn.argtypes = [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    fn.restype = ctypes.c_int
    n = (nbytes + 15) // 16 * 16
    grids = (512, 1024, 2048)
    depths = (2, 4, 8)
    bufs = [torch.zeros(n, dtype=torch.uint8, device="cuda") for _ in range(layers)]
    sink = torch.zeros(max(grids), dtype=torch.int32, device="cuda")

    def launch(i: int, grid: int, depth: int) -> None:
        rc = fn(bufs[i % layers].data_ptr(), n, grid, depth, sink.data_ptr(), stream.cuda_stream)
        if rc:
            raise RuntimeError(f"stream probe launch failed (code {rc})")

    best = None
    for grid in grids:
        for depth in depths:
            for i in range(layers):
                launch(i, grid, depth)
            launch(layers - 1, grid, depth)
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for i in range(steps):
                launch(i, grid, depth)
            e1.record(stream)
            torch.cuda.synchronize()
            us = e0.elapsed_time(e1) / steps * 1e3
            if best is None or us < best[0]:
                best = (us, grid, depth)
    del bufs, sink
    torch.cuda.empty_cache()
    us, grid, depth = best
    gbs = n / us / 1e3
    return {"us": round(us, 2), "gbs": round(gbs, 1), "frac_of_peak": round(gbs / HBM_PEAK_GBS, 4), "grid": grid,
            "loads_in_flight_per_lane": depth, "bytes": n,
            "note": f"plain non-temporal 16-byte streaming read of the step's KV bytes over {layers} buffers in turn, "
                    f"{steps} launches back to back, same GPU and run; best of grids {'/'.join(map(str, grids))} x "
                    f"{'/'.join(map(str, depths))} loads in flight per lane"}


def matmul_timing(gsp, torch, ctx, stream, step, calls: int = 50) -> dict:
    """Device cost of the step's Q projection (QuantKernels.MatMulBatch, PagedTransformerRunner.cs:601):
    hidden = n_heads * head_dim in and out, one batch row per query token of the step, random
    weights as Q8_0 and as F32.  Each call takes the next of enough weight copies to span 512 MB,
    twice the Infinity Cache, as a model's layers do (`us_per_call`); `us_per_call_warm` repeats one
    copy.  Q8_0, Q4_K and Q6_K run on the fp16 matrix cores (x as scaled fp16 pairs), F32 on the fp32
    ones (the K-quants are timed when hidden is a multiple of 256); the bytes bound is the weights at
    8 TB/s."""
    hidden = step.n_heads * step.head_dim
    batch = int(step.total_q)
    gen = torch.Generator(device="cuda").manual_seed(step.seed)
    x = torch.randn((batch, hidden), device="cuda", generator=gen)
    y = torch.empty((batch, hidden), device="cuda")
    nb = hidden // 32
    d = (torch.randn((hidden, nb, 1), device="cuda", generator=gen) * 0.01).half().view(torch.uint8)
    q = torch.randint(-127, 128, (hidden, nb, 32), device="cuda", generator=gen, dtype=torch.int8).view(torch.uint8)
    q8 = torch.cat([d, q], dim=2).contiguous()
    weights = {"q8_0": (gsp.WTYPE_Q8_0, q8, hidden * nb * 34),
               "f32": (gsp.WTYPE_F32, torch.randn((hidden, hidden), device="cuda", generator=gen), hidden * hidden * 4)}
    if hidden % 256 == 0:
        # K-quant super-blocks: random quant bytes with small finite fp16 scales.
        nk = hidden // 256
        q4 = torch.randint(0, 256, (hidden, nk, 144), device="cuda", generator=gen, dtype=torch.uint8)
        q4[:, :, 0:4] = (torch.rand((hidden, nk, 2), device="cuda", generator=gen) * 0.01).half().view(torch.uint8)
        q6 = torch.randint(0, 256, (hidden, nk, 210), device="cuda", generator=gen, dtype=torch.uint8)
        q6[:, :, 208:210] = (torch.rand((hidden, nk, 1), device="cuda", generator=gen) * 1e-3).half().view(torch.uint8)
        weights["q4_k"] = (gsp.WTYPE_Q4_K, q4.contiguous(), hidden * nk * 144)
        weights["q6_k"] = (gsp.WTYPE_Q6_K, q6.contiguous(), hidden * nk * 210)
    torch.cuda.synchronize()
    flops = 2.0 * batch * hidden * hidden
    out = {"in_dim": hidden, "out_dim": hidden, "batch": batch}
    for name, (wt, w, wbytes) in weights.items():
        copies = [w] + [w.clone() for _ in range(max(1, -(-(512 << 20) // wbytes)) - 1)]
        torch.cuda.synchronize()

        def timed(pick) -> float:
            with torch.cuda.stream(stream):
                for i in range(5):
                    ctx.matmul_batch(wt, pick(i).data_ptr(), x.data_ptr(), y.data_ptr(), hidden, hidden, batch)
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for i in range(calls):
                    ctx.matmul_batch(wt, pick(i).data_ptr(), x.data_ptr(), y.data_ptr(), hidden, hidden, batch)
                e1.record(stream)
            torch.cuda.synchronize()
            return e0.elapsed_time(e1) / calls * 1e3

        us = timed(lambda i: copies[i % len(copies)])
        us_warm = timed(lambda i: w)
        out[name] = {"us_per_call": round(us, 2), "us_per_call_warm": round(us_warm, 2), "weight_copies": len(copies),
                     "tflops": round(flops / (us * 1e-6) / 1e12, 2),
                     "weight_gbs": round(wbytes / (us * 1e-6) / 1e9, 1),
                     "frac_hbm_peak_weights": round(wbytes / (us * 1e-6) / 8e12, 4)}
        del copies
    return out


def kv_write_timing(gsp, torch, ctx, stream, step, pool, layers: int, calls: int = 100) -> dict:
    """Per-layer device cost of the step's own K/V write with RoPE (QuantKernels.RoPE then
    PagedBlockPool.Store, PagedTransformerRunner.cs:620-634, fused): each query token's new K/V
    into the slot of its position, layer i mod L per call.  gsp_rope_write_step reads positions,
    blocks and slots from the packed step (one upload per tick, none per layer);
    gsp_rope_write_tokens, timed beside it, restages host arrays on every call."""
    import numpy as np

    n = step.total_q
    gen = torch.Generator(device="cuda").manual_seed(step.seed)
    q = torch.randn((n, step.n_heads, step.head_dim), device="cuda", generator=gen)
    k = torch.randn((n, step.n_kv, step.head_dim), device="cuda", generator=gen)
    v = torch.randn((n, step.n_kv, step.dv), device="cuda", generator=gen)
    base, style = 1000000.0, gsp.ROPE_HALVES
    pos, blocks, slots = [], [], []
    for b in range(step.num_rows):
        for i in range(int(step.lens[b])):
            p = int(step.positions[b]) + i
            pos.append(p)
            blocks.append(int(step.table(b)[p // step.block_size]))
            slots.append(p % step.block_size)
    pos, blocks, slots = (np.array(x, np.int32) for x in (pos, blocks, slots))
    torch.cuda.synchronize()

    def timed(fn) -> float:
        for i in range(5):
            fn(i)
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for i in range(calls):
            fn(i)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / calls * 1e3

    def write_step(i):
        pool.rope_write_step(i % layers, step.n_heads, base, style, q.data_ptr(), k.data_ptr(), v.data_ptr())

    us_step = timed(write_step)
    us_host = timed(lambda i: pool.rope_write_tokens(i % layers, pos, blocks, slots, step.n_heads, base, style,
                                                     q.data_ptr(), k.data_ptr(), v.data_ptr()))
    # The same calls captured once and replayed as a graph: the device's own
    # cost per call, without the Python loop's pace (the eager figure above
    # can be bound by the host issuing the calls).
    us_graph = None
    try:
        ctx.sync()  # a capture reads the packed step only once its upload is known complete
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream):
            for i in range(calls):
                write_step(i)
        for _ in range(3):
            graph.replay()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        with torch.cuda.stream(stream):
            graph.replay()
        e1.record(stream)
        torch.cuda.synchronize()
        us_graph = round(e0.elapsed_time(e1) / calls * 1e3, 2)
        del graph
    except Exception as exc:  # the eager figures stand alone
        us_graph = "graph capture failed: " + str(exc)
    elem = 2 if step.kv_dtype == "f16" else 4
    moved = n * (2 * step.n_heads * step.head_dim * 4 + step.n_kv * (step.head_dim + step.dv) * 4
                 + step.n_kv * (step.head_dim + step.dv) * elem)
    return {"tokens": n, "us_per_layer_call": round(us_step, 2), "us_per_layer_call_graph": us_graph,
            "bytes_per_call": moved,
            "gbs": round(moved / (us_step * 1e-6) / 1e9, 1), "us_per_call_host_arrays": round(us_host, 2),
            "note": "gsp_rope_write_step: Q rotated in place, K rotated and stored, V stored, slots from the "
                    "packed step; the host-array form restages ids per call"}


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
    # Layer 0 only: the layer the GPU output is checked on.
    kh = k.index_select(0, idx)[:, :1].float().cpu().numpy()
    vh = v.index_select(0, idx)[:, :1].float().cpu().numpy()
    qh = q.cpu().numpy()
    ids = inv.astype(np.int32)
    pool = orc.HostPool(kh, vh, block_size=step.block_size)
    nt = cpu_threads()
    out = np.zeros((step.total_q, step.n_heads, step.dv), np.float32)

    def one():
        orc.attention_step(pool, 0, step.positions, step.token_counts, step.bt_offsets, ids, qh, step.n_heads,
                           step.scale, step.max_seq_len, q_lens=step.q_lens, out=out, n_threads=nt)

    # Five warm-up steps, as the reference benchmark warms up (Program.cs:101-115); the first is also
    # the parity reference.  Fewer when one step would eat a tenth of the budget.
    warm = 0
    t_warm = time.perf_counter()
    while warm < CPU_WARMUP_STEPS:
        one()
        warm += 1
        if time.perf_counter() - t_warm > budget_s / 10:
            break
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
        "sample": f"whole {step.name} step ({step.num_rows} rows), median of {len(times)} steps after {warm} "
                  f"warm-up steps (budget {budget_s:.0f} s), {nt} threads on '{cpu_model()}' ({visible_cores()} cores visible "
                  f"to the process, {HOST_CPU_SHARE} per GPU allotted to a job on this host), ISA level "
                  f"{orc.host_isa()} (2=AVX-512, 1=AVX2); C++ restatement of the reference C# kernel",
        "ms_per_step": round(med * 1e3, 3),
        "seq_steps_per_s": round(step.num_rows / med, 1),
    }
    return rec, out.copy()


def summarize_trace(path: str, kernel: str, last: int) -> dict:
    """Launch durations of `kernel` in a rocprofv3 kernel-trace CSV: all launches, and the
    last `last` of them in dispatch order (the timed region of a --profile-only run)."""
    import csv

    rows = []
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if kernel in r["Kernel_Name"]:
                rows.append((int(r["Dispatch_Id"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"])))
    rows.sort()
    durs = [e - s for _, s, e in rows]
    sel = rows[-last:] if last > 0 else rows
    if not sel:
        raise SystemExit(f"no launch of {kernel} in {path}")
    sel_d = [e - s for _, s, e in sel]
    out = {"kernel": kernel, "calls": len(durs), "avg_ns_all": round(statistics.mean(durs), 1),
           "max_ns_all": max(durs), "last": len(sel), "avg_ns_last": round(statistics.mean(sel_d), 1),
           "median_ns_last": statistics.median(sel_d), "min_ns_last": min(sel_d), "max_ns_last": max(sel_d)}
    if len(sel) > 1:
        # Start-to-start period of the selected launches (back to back in the
        # timed region): the kernel plus the gap before the next launch.
        out["avg_period_ns_last"] = round((sel[-1][1] - sel[0][1]) / (len(sel) - 1), 1)
    return out


def summarize_pmc(path: str, kernel: str, last: int) -> dict:
    """Per-dispatch counter values of `kernel` in a rocprofv3 counter-collection CSV,
    averaged over its last `last` dispatches."""
    import csv

    per = {}
    with open(path, newline="") as f:
        for r in csv.DictReader(f):
            if kernel in r["Kernel_Name"]:
                d = per.setdefault(int(r["Dispatch_Id"]), {})
                d[r["Counter_Name"]] = d.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    ids = sorted(per)
    sel = ids[-last:] if last > 0 else ids
    if not sel:
        raise SystemExit(f"no dispatch of {kernel} in {path}")
    names = sorted({c for i in sel for c in per[i]})
    return {"kernel": kernel, "dispatches": len(ids), "last": len(sel),
            "mean": {c: round(statistics.mean(per[i].get(c, 0.0) for i in sel), 3) for c in names}}


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
    ap.add_argument("--layers", type=int, default=4,
                    help="pool layers; step i attends layer i mod LAYERS (1 re-reads one layer every step)")
    ap.add_argument("--decode-path", default="auto", choices=["auto", "mfma", "dpp"],
                    help="decode kernel (auto = the matrix-core kernel)")
    ap.add_argument("--prefill-split", default="records", choices=["records", "in_tile"],
                    help="fp32 prefill tiles: split records written once per step (default) or split in each tile")
    ap.add_argument("--split-pages", type=int, default=0,
                    help="largest split-KV unit in pages (tuning; 0: the library's choice)")
    ap.add_argument("--decode-bins", type=int, default=0,
                    help="decode workgroups (tuning; 0: the library's choice)")
    ap.add_argument("--profile-only", action="store_true",
                    help="only the warmup and timed launches (plus each kernel alone for mixed steps)")
    ap.add_argument("--summarize-trace", metavar="CSV", help="summarize a rocprofv3 kernel-trace CSV and exit")
    ap.add_argument("--summarize-pmc", metavar="CSV", help="summarize a rocprofv3 counter-collection CSV and exit")
    ap.add_argument("--kernel", default=KERNEL_NAME, help="kernel name (substring) for the summaries")
    ap.add_argument("--last", type=int, default=0, help="average the last N launches only (0: all)")
    args = ap.parse_args()
    if args.summarize_trace or args.summarize_pmc:
        if args.summarize_trace:
            print(json.dumps(summarize_trace(args.summarize_trace, args.kernel, args.last)))
        if args.summarize_pmc:
            print(json.dumps(summarize_pmc(args.summarize_pmc, args.kernel, args.last)))
        return 0
    if args.layers < 1:
        print("--layers must be >= 1", file=sys.stderr)
        return 2
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); this path is not sharded across GPUs "
              "in this build", file=sys.stderr)
        return 2
    names = WORKLOADS if args.all else [args.workload]
    # Python's cyclic collector stops the host for tens of milliseconds now and
    # then (torch keeps a large object graph); the timed loops run without it.
    gc.collect()
    gc.disable()
    for name in names:
        res = run_workload(name, args.steps, args.warmup, cpu=not (args.no_cpu or args.profile_only),
                           cpu_budget_s=args.cpu_budget, layers=args.layers, decode_path=args.decode_path,
                           profile_only=args.profile_only, prefill_split=args.prefill_split,
                           split_pages=args.split_pages, decode_bins=args.decode_bins)
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
