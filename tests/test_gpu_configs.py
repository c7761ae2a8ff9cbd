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
