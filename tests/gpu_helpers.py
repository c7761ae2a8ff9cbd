"""Shared helpers of the GPU parity tests: run a packed step through the C ABI
and the same step through the CPU oracle."""
from __future__ import annotations

import numpy as np

import glacier_oracle as orc
import workloads

TOL = {"f32": 1e-4, "f16": 2e-3}  # max abs error vs the oracle, per KV dtype


def to_device_pool(torch, gsp, ctx, step, k, v):
    """Uploads host arenas [blocks, layers, nKV, 16, d] and wraps them as a device pool."""
    dt = torch.float16 if step.kv_dtype == "f16" else torch.float32
    kd = torch.from_numpy(np.ascontiguousarray(k)).to(device="cuda", dtype=dt)
    vd = torch.from_numpy(np.ascontiguousarray(v)).to(device="cuda", dtype=dt)
    pool = gsp.Pool.wrap(ctx, kd.data_ptr(), vd.data_ptr(), step.total_blocks, k.shape[1], step.n_kv,
                         step.head_dim, gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32, v_head_dim=step.dv,
                         block_size=step.block_size)
    return pool, (kd, vd)


def gpu_step(torch, gsp, ctx, step, q, pool, layer=0, split_pages=0, fill=np.nan, bins=0):
    """Packs the step, runs gsp_attention_step and returns out [total_q, nH, d] on the host."""
    ctx.set_split_pages(split_pages)
    ctx.set_decode_bins(bins)
    try:
        ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                      q_lens=step.q_lens)
    finally:
        ctx.set_split_pages(0)
        ctx.set_decode_bins(0)
    qd = torch.from_numpy(np.ascontiguousarray(q, dtype=np.float32)).cuda()
    out = torch.full((step.total_q, step.n_heads, step.dv), float(fill), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    ctx.attention_step(pool, layer, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
    ctx.sync()
    return out.cpu().numpy()


def oracle_step(step, q, k, v, layer=0, threads=8, fill=np.nan):
    pool = orc.HostPool(k, v, block_size=step.block_size)
    out = np.full((step.total_q, step.n_heads, step.dv), fill, np.float32)
    orc.attention_step(pool, layer, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, q, step.n_heads,
                       step.scale, step.max_seq_len, q_lens=step.q_lens, out=out, n_threads=threads)
    return out


def max_err(a, b):
    return float(np.nanmax(np.abs(a.astype(np.float64) - b.astype(np.float64)))) if a.size else 0.0


def compact(step: workloads.Step):
    """Remaps a step onto only the blocks it uses: (step', used_ids) with ids 0..n_used-1."""
    used, inv = np.unique(step.bt_ids, return_inverse=True)
    s = workloads.Step(step.name, step.n_heads, step.n_kv, step.head_dim, step.kv_dtype, len(used),
                       step.max_seq_len, step.positions, step.token_counts, step.bt_offsets,
                       inv.astype(np.int32), step.q_lens, step.seed, dict(step.notes), step.block_size,
                       step.v_head_dim)
    return s, used
