"""Parity soak of the split-KV handoff: many seeded ragged steps against the oracle.

A split piece publishes its partial with agent-scope coherent stores, waits for
their completion, and then counts itself on the pair's counter; the last piece
reads every partial with coherent loads and merges.  A mistake in that handoff
would show as a rare wrong value, which fixed-seed tests can miss.  This soak runs
several hundred seeded steps with forced 1- to 3-page splits (many pieces per
pair) and 1 to 1000 workgroups (so pieces of one pair land on different CUs and
XCDs, in every order), over several geometries, fp32 and fp16 pages, decode and
prefill rows, and stops at the first output that differs from the oracle.
"""
import os

import numpy as np
import pytest

import workloads
from gpu_helpers import TOL, max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu

GEOMS = [
    # (n_heads, n_kv, head_dim, v_head_dim, block_size, kv dtype)
    (28, 4, 128, 128, 16, "f32"),
    (32, 8, 128, 128, 16, "f16"),
    (14, 2, 64, 64, 16, "f32"),
    (64, 8, 128, 128, 16, "f16"),
    (32, 1, 96, 80, 8, "f32"),
]
# GSP_SOAK_STEPS lengthens the soak (steps per geometry).
STEPS_PER_GEOM = int(os.environ.get("GSP_SOAK_STEPS", "60"))


@pytest.mark.parametrize("geom", GEOMS, ids=lambda g: f"{g[0]}q{g[1]}kv_d{g[2]}_dv{g[3]}_bs{g[4]}_{g[5]}")
def test_split_handoff_soak(torch_mod, gsp, ctx, geom):
    torch = torch_mod
    nh, nkv, d, dv, bs, dt = geom
    rng = np.random.default_rng(d * 1000 + nh * 10 + bs)
    base = workloads.small_step(seed=int(rng.integers(1 << 30)), rows=24, n_heads=nh, n_kv=nkv, head_dim=d,
                                kv_dtype=dt, ctx_lo=1, ctx_hi=700, total_blocks=24 * (-(-700 // bs)) + 8,
                                block_size=bs, v_head_dim=dv)
    _, k, v = workloads.host_values(base)
    pool, keep = to_device_pool(torch, gsp, ctx, base, k, v)
    try:
        for it in range(STEPS_PER_GEOM):
            rows = np.sort(rng.choice(base.num_rows, size=int(rng.integers(1, base.num_rows + 1)), replace=False))
            step, _ = base.subset(rows)
            # Some rows become causal prefill rows over their last tokens.
            if rng.random() < 0.3:
                ql = np.ones(step.num_rows, np.int32)
                for r in range(step.num_rows):
                    if rng.random() < 0.4:
                        ql[r] = int(min(rng.integers(2, 40), step.token_counts[r]))
                step.positions = (step.token_counts - ql).astype(np.int32)
                step.q_lens = ql
            split = int(rng.integers(1, 4))
            bins = int(rng.choice([1, 2, 7, 64, 333, 1000]))
            ctx.set_split_pages(split)
            ctx.set_decode_bins(bins)
            try:
                ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids,
                              step.max_seq_len, q_lens=step.q_lens, want_info=False)
            finally:
                ctx.set_split_pages(0)
                ctx.set_decode_bins(0)
            # Q and out sized for this step's query tokens.
            q = rng.standard_normal((step.total_q, nh, d), dtype=np.float32)
            qd = torch.from_numpy(q).cuda()
            o = torch.full((step.total_q, nh, dv), float("nan"), device="cuda")
            torch.cuda.synchronize()
            ctx.attention_step(pool, 0, nh, qd.data_ptr(), o.data_ptr(), step.scale)
            ctx.sync()
            got = o.cpu().numpy()
            ref = oracle_step(step, q, k, v)
            err = max_err(got, ref)
            assert err <= TOL[dt], f"step {it}: rows {len(rows)}, split {split}, bins {bins}: err {err}"
    finally:
        pool.destroy()
