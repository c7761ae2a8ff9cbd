"""The five measured shapes at full size: every query token against the oracle.

Values are drawn on the GPU; the oracle reads exactly the pages the step
uses (downloaded and upcast), so fp16 shapes compare identical inputs.
"""
import numpy as np
import pytest

import glacier_oracle as orc
import workloads
from conftest import threads
from gpu_helpers import TOL, compact, max_err

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("cfg", [1, 2, 3, 4, 5])
def test_full_size_config_matches_oracle(torch_mod, gsp, ctx, cfg):
    torch = torch_mod
    step = workloads.CONFIGS[cfg]()
    print(f"case config {cfg} {step.name}: rows={step.num_rows} total_q={step.total_q} "
          f"kv_tokens={step.kv_tokens()}", flush=True)
    q, k, v = workloads.device_values(torch, step)
    pool = gsp.Pool.wrap(ctx, k.data_ptr(), v.data_ptr(), step.total_blocks, 1, step.n_kv, step.head_dim,
                         gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32)
    out = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
    ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                  q_lens=step.q_lens)
    torch.cuda.synchronize()
    ctx.attention_step(pool, 0, step.n_heads, q.data_ptr(), out.data_ptr(), step.scale)
    ctx.sync()
    got = out.cpu().numpy()
    pool.destroy()

    cstep, used = compact(step)
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    kh = k.index_select(0, idx).float().cpu().numpy()
    vh = v.index_select(0, idx).float().cpu().numpy()
    qh = q.cpu().numpy()
    del k, v
    ref = np.full_like(got, np.nan)
    orc.attention_step(orc.HostPool(kh, vh), 0, cstep.positions, cstep.token_counts, cstep.bt_offsets, cstep.bt_ids,
                       qh, cstep.n_heads, cstep.scale, cstep.max_seq_len, q_lens=cstep.q_lens, out=ref,
                       n_threads=threads())
    err = max_err(got, ref)
    print(f"config {cfg}: max abs err {err:.3e}", flush=True)
    assert not np.isnan(got).any()
    assert err <= TOL[step.kv_dtype]


def _run(torch, gsp, ctx, step, q, k, v):
    pool = gsp.Pool.wrap(ctx, k.data_ptr(), v.data_ptr(), step.total_blocks, 1, step.n_kv, step.head_dim,
                         gsp.KV_F16 if step.kv_dtype == "f16" else gsp.KV_F32)
    out = torch.full((step.total_q, step.n_heads, step.head_dim), float("nan"), device="cuda")
    ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                  q_lens=step.q_lens)
    torch.cuda.synchronize()
    ctx.attention_step(pool, 0, step.n_heads, q.data_ptr(), out.data_ptr(), step.scale)
    ctx.sync()
    pool.destroy()
    return out


@pytest.mark.parametrize("cfg", [2, 3])
def test_full_size_physical_permutation_and_repeat_are_bit_exact(torch_mod, gsp, ctx, cfg):
    """Where a page lives must not matter: moving every block to another physical id (and its K/V
    with it) gives the same output bit for bit, and so does running the step again."""
    torch = torch_mod
    step = workloads.CONFIGS[cfg]()
    print(f"case permutation config {cfg}", flush=True)
    q, k, v = workloads.device_values(torch, step)
    base = _run(torch, gsp, ctx, step, q, k, v)
    again = _run(torch, gsp, ctx, step, q, k, v)
    assert torch.equal(base, again), "a repeated launch differs"
    perm = np.random.default_rng(cfg).permutation(step.total_blocks)  # block b moves to perm[b]
    inv = torch.from_numpy(np.argsort(perm).astype(np.int64)).cuda()  # new id -> old id
    kp = k.index_select(0, inv)
    vp = v.index_select(0, inv)
    del k, v
    moved = workloads.Step(step.name, step.n_heads, step.n_kv, step.head_dim, step.kv_dtype, step.total_blocks,
                           step.max_seq_len, step.positions, step.token_counts, step.bt_offsets,
                           perm[step.bt_ids].astype(np.int32), step.q_lens, step.seed)
    got = _run(torch, gsp, ctx, moved, q, kp, vp)
    assert torch.equal(base, got), "the output depends on where the pages live"


@pytest.mark.parametrize("cfg", [2, 3])
def test_full_size_uniform_values_give_that_value(torch_mod, gsp, ctx, cfg):
    """Every V row equal to one vector c: each output row is c whatever the scores (softmax weights
    sum to one)."""
    torch = torch_mod
    step = workloads.CONFIGS[cfg]()
    print(f"case uniform V config {cfg}", flush=True)
    q, k, v = workloads.device_values(torch, step)
    c = torch.linspace(-2.0, 2.0, step.head_dim, device="cuda")
    v.copy_(c.to(v.dtype).expand_as(v))
    out = _run(torch, gsp, ctx, step, q, k, v)
    want = c.to(v.dtype).float().expand_as(out)
    err = (out - want).abs().max().item()
    print(f"config {cfg}: max abs err {err:.3e}", flush=True)
    assert err <= (2e-5 if step.kv_dtype == "f32" else 2e-3)
