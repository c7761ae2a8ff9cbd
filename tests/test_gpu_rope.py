"""gsp_rope_write_tokens: RoPE on Q and K fused with the KV store, against the oracle.

The oracle computes the textbook rotation in fp64 (orc_rope).  The device
forms each angle in fp64 and takes its cosine and sine in fp32, so fp32
results stay within a few 1e-7 of the oracle at any position (bar 2e-6 on
N(0, 1) inputs); fp16 pools hold the rotated value rounded to fp16 (bar one
fp16 ulp, 2e-3 at these magnitudes).  V is stored untouched, bit-exact.
"""
import numpy as np
import pytest

import glacier_oracle as orc
import workloads
from gpu_helpers import max_err, oracle_step, to_device_pool

pytestmark = pytest.mark.gpu

CASES = [
    # (n_heads, n_kv, head_dim, kv dtype, freq base)
    (28, 4, 128, "f32", 1000000.0),
    (14, 2, 64, "f32", 10000.0),
    (32, 8, 128, "f16", 500000.0),
    (8, 8, 64, "f16", 10000.0),
    (12, 4, 80, "f16", 10000.0),  # 16-byte kernel, half of 40 pairs
    (6, 2, 36, "f32", 10000.0),   # head_dim % 8 != 0: the per-element kernel
]


def _tokens(rng, n, total_blocks):
    blocks = rng.choice(total_blocks, size=n, replace=False).astype(np.int32)
    slots = rng.integers(0, 16, size=n).astype(np.int32)
    positions = rng.integers(0, 40000, size=n).astype(np.int32)
    positions[:3] = [0, 1, 32767]
    return positions, blocks, slots


@pytest.mark.parametrize("style", [0, 1], ids=["pairs", "halves"])
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}q{c[1]}kv_d{c[2]}_{c[3]}")
def test_rope_write_matches_oracle(torch_mod, gsp, ctx, case, style):
    torch = torch_mod
    nh, nkv, d, dt, base = case
    print(f"case rope {case} style={style}", flush=True)
    rng = np.random.default_rng(nh * 7 + d + style)
    n, total_blocks = 37, 64
    positions, blocks, slots = _tokens(rng, n, total_blocks)
    q = rng.standard_normal((n, nh, d)).astype(np.float32)
    k = rng.standard_normal((n, nkv, d)).astype(np.float32)
    v = rng.standard_normal((n, nkv, d)).astype(np.float32)
    pool = gsp.Pool.create(ctx, total_blocks=total_blocks, layers=2, heads_kv=nkv, head_dim=d,
                           kv_dtype=gsp.KV_F16 if dt == "f16" else gsp.KV_F32)
    qd = torch.from_numpy(q).cuda()
    kd = torch.from_numpy(k).cuda()
    vd = torch.from_numpy(v).cuda()
    torch.cuda.synchronize()
    pool.rope_write_tokens(1, positions, blocks, slots, nh, base, style, qd.data_ptr(), kd.data_ptr(), vd.data_ptr())
    ctx.sync()
    npdt = np.float16 if dt == "f16" else np.float32
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(npdt).reshape(total_blocks, 2, nkv, 16, d)
    V = pool.download(1, vb).view(npdt).reshape(total_blocks, 2, nkv, 16, d)
    got_q = qd.cpu().numpy()
    tol = 2e-3 if dt == "f16" else 2e-6
    for i in range(n):
        ref_q = orc.rope(q[i], int(positions[i]), base, style)
        ref_k = orc.rope(k[i], int(positions[i]), base, style)
        assert max_err(got_q[i], ref_q) <= 2e-6, f"q of token {i} at position {positions[i]}"
        assert max_err(K[blocks[i], 1, :, slots[i]].astype(np.float32), ref_k) <= tol, f"k of token {i}"
        assert np.array_equal(V[blocks[i], 1, :, slots[i]], v[i].astype(npdt)), f"v of token {i}"
    # Nothing else in the pool was written (pools start zeroed).
    mask = np.ones(K.shape, bool)
    mask[blocks, 1, :, slots] = False
    assert not K[mask].any() and not V[mask].any()
    pool.destroy()


def test_rope_write_without_q_and_errors(torch_mod, gsp, ctx):
    torch = torch_mod
    pool = gsp.Pool.create(ctx, total_blocks=8, layers=1, heads_kv=2, head_dim=64)
    k = torch.ones((2, 2, 64), device="cuda")
    q = torch.full((2, 4, 64), 5.0, device="cuda")
    torch.cuda.synchronize()
    pool.rope_write_tokens(0, [3, 4], [1, 2], [0, 0], 0, 10000.0, 0, 0, k.data_ptr(), k.data_ptr())
    ctx.sync()
    _, _, kb, _ = pool.arenas()
    K = pool.download(0, kb).view(np.float32).reshape(8, 1, 2, 16, 64)
    assert np.allclose(K[1, 0, 0, 0], orc.rope(np.ones(64, np.float32), 3, 10000.0), atol=2e-6)
    for bad in (dict(positions=[-1]), dict(slots=[16]), dict(blocks=[8]), dict(style=2), dict(base=0.0),
                dict(nh=4, qp=0)):
        with pytest.raises(gsp.InvalidArgument):
            pool.rope_write_tokens(0, bad.get("positions", [0]), bad.get("blocks", [0]), bad.get("slots", [0]),
                                   bad.get("nh", 0), bad.get("base", 10000.0), bad.get("style", 0),
                                   bad.get("qp", q.data_ptr()), k.data_ptr(), k.data_ptr())
    ctx.sync()
    pool.destroy()


@pytest.mark.parametrize("style", [0, 1], ids=["pairs", "halves"])
def test_rope_write_then_attention(torch_mod, gsp, ctx, style):
    """The reference decode order (PagedTransformerRunner.cs:605-656): RoPE, Store, then attention
    over the stored pages; the device path against the oracle's rotated Q and K."""
    torch = torch_mod
    print(f"case rope+attention style={style}", flush=True)
    base = 1000000.0
    step = workloads.small_step(seed=91 + style, rows=6, n_heads=28, n_kv=4, head_dim=128, ctx_lo=20, ctx_hi=200,
                                total_blocks=256)
    q, k, v = workloads.host_values(step)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    # Every row's newest token (position TokenCount - 1) gets fresh K/V through RoPE + Store.
    rng = np.random.default_rng(5)
    rows = step.num_rows
    pos = (step.token_counts - 1).astype(np.int32)
    blocks = np.array([step.table(b)[p // 16] for b, p in enumerate(pos)], np.int32)
    slots = (pos % 16).astype(np.int32)
    k_new = rng.standard_normal((rows, step.n_kv, step.head_dim)).astype(np.float32)
    v_new = rng.standard_normal((rows, step.n_kv, step.head_dim)).astype(np.float32)
    qd = torch.from_numpy(np.ascontiguousarray(q)).cuda()
    kn = torch.from_numpy(k_new).cuda()
    vn = torch.from_numpy(v_new).cuda()
    torch.cuda.synchronize()
    pool.rope_write_tokens(0, pos, blocks, slots, step.n_heads, base, style, qd.data_ptr(), kn.data_ptr(),
                           vn.data_ptr())
    ctx.pack_step(pool, pos, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len)
    out = torch.full((rows, step.n_heads, step.head_dim), float("nan"), device="cuda")
    torch.cuda.synchronize()  # torch fills on its own stream, the library on the context's
    ctx.attention_step(pool, 0, step.n_heads, qd.data_ptr(), out.data_ptr(), step.scale)
    ctx.sync()
    # Oracle: the same rotation and store on the host arenas, then the reference attention.
    k2, v2 = k.copy(), v.copy()
    qr = np.stack([orc.rope(q[b], int(pos[b]), base, style) for b in range(rows)])
    for b in range(rows):
        k2[blocks[b], 0, :, slots[b]] = orc.rope(k_new[b], int(pos[b]), base, style)
        v2[blocks[b], 0, :, slots[b]] = v_new[b]
    step2 = workloads.Step(step.name, step.n_heads, step.n_kv, step.head_dim, step.kv_dtype, step.total_blocks,
                           step.max_seq_len, pos, step.token_counts, step.bt_offsets, step.bt_ids, None, step.seed)
    ref = oracle_step(step2, qr, k2, v2)
    assert max_err(out.cpu().numpy(), ref) <= 1e-4
    pool.destroy()


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_step_writes_match_the_explicit_writes(torch_mod, gsp, ctx, dt):
    """gsp_rope_write_step / gsp_pool_write_step store each query token's K/V at the
    slot of its own position, read from the packed step: bit for bit what
    gsp_rope_write_tokens / gsp_pool_write_tokens store given the same positions,
    blocks and slots as host arrays, and checked against the oracle's rotation.  The
    step mixes decode rows, a prefill chunk, a row whose position lies past its
    TokenCount (no slot: nothing stored, Q still rotated) and an empty row."""
    torch = torch_mod
    nh, nkv, d, base = 28, 4, 128, 1000000.0
    q_lens = np.array([1, 19, 1, 0, 1], np.int32)
    step = workloads.small_step(seed=95, rows=5, n_heads=nh, n_kv=nkv, head_dim=d, kv_dtype=dt, ctx_lo=5,
                                ctx_hi=200, total_blocks=256, q_lens=q_lens)
    step.positions[2] = step.token_counts[2] + 3  # clamped row: attends TokenCount tokens, has no slot
    print(f"case step writes {dt}", flush=True)
    rng = np.random.default_rng(96)
    nq = step.total_q
    q = rng.standard_normal((nq, nh, d)).astype(np.float32)
    k = rng.standard_normal((nq, nkv, d)).astype(np.float32)
    v = rng.standard_normal((nq, nkv, d)).astype(np.float32)
    # Expected destinations, from the tables on the host.
    pos, blocks, slots, stored = [], [], [], []
    for b in range(step.num_rows):
        for i in range(int(step.lens[b])):
            p = int(step.positions[b]) + i
            pos.append(p)
            has = p < int(step.token_counts[b])
            stored.append(has)
            blocks.append(int(step.table(b)[p // 16]) if has else -1)
            slots.append(p % 16)
    pos, blocks, slots, stored = (np.array(x) for x in (pos, blocks, slots, stored))
    assert stored.sum() == nq - 1  # exactly the clamped row's token has no slot
    kind = gsp.KV_F16 if dt == "f16" else gsp.KV_F32
    npdt = np.float16 if dt == "f16" else np.float32
    pools = [gsp.Pool.create(ctx, total_blocks=step.total_blocks, layers=2, heads_kv=nkv, head_dim=d, kv_dtype=kind)
             for _ in range(4)]
    qs = [torch.from_numpy(q).cuda() for _ in range(2)]
    kd = torch.from_numpy(k).cuda()
    vd = torch.from_numpy(v).cuda()
    torch.cuda.synchronize()
    ctx.pack_step(pools[0], step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                  q_lens=step.q_lens)
    pools[0].rope_write_step(1, nh, base, 1, qs[0].data_ptr(), kd.data_ptr(), vd.data_ptr())
    pools[1].write_step(1, kd.data_ptr(), vd.data_ptr())
    sel = np.nonzero(stored)[0]
    qsel = torch.from_numpy(np.ascontiguousarray(q[sel])).cuda()
    ksel = torch.from_numpy(np.ascontiguousarray(k[sel])).cuda()
    vsel = torch.from_numpy(np.ascontiguousarray(v[sel])).cuda()
    torch.cuda.synchronize()
    pools[2].rope_write_tokens(1, pos[sel], blocks[sel], slots[sel], nh, base, 1, qsel.data_ptr(), ksel.data_ptr(),
                               vsel.data_ptr())
    pools[3].write_tokens(1, blocks[sel], slots[sel], ksel.data_ptr(), vsel.data_ptr())
    ctx.sync()
    _, _, kb, vb = pools[0].arenas()
    arenas = [(p.download(0, kb).view(npdt), p.download(1, vb).view(npdt)) for p in pools]
    assert np.array_equal(arenas[0][0], arenas[2][0]) and np.array_equal(arenas[0][1], arenas[2][1])
    assert np.array_equal(arenas[1][0], arenas[3][0]) and np.array_equal(arenas[1][1], arenas[3][1])
    got_q = qs[0].cpu().numpy()
    assert np.array_equal(got_q[sel], qsel.cpu().numpy())
    K = arenas[0][0].reshape(step.total_blocks, 2, nkv, 16, d)
    V = arenas[0][1].reshape(step.total_blocks, 2, nkv, 16, d)
    tol = 2e-3 if dt == "f16" else 2e-6
    for i in range(nq):
        assert max_err(got_q[i], orc.rope(q[i], int(pos[i]), base, 1)) <= 2e-6, f"q of token {i}"
        if stored[i]:
            got_k = K[blocks[i], 1, :, slots[i]].astype(np.float32)
            assert max_err(got_k, orc.rope(k[i], int(pos[i]), base, 1)) <= tol, f"k of token {i}"
            assert np.array_equal(V[blocks[i], 1, :, slots[i]], v[i].astype(npdt))
    mask = np.ones(K.shape, bool)
    mask[blocks[sel], 1, :, slots[sel]] = False
    assert not K[mask].any() and not V[mask].any()
    with pytest.raises(gsp.InvalidArgument):  # a layer outside the pool
        pools[1].write_step(2, kd.data_ptr(), vd.data_ptr())
    small = gsp.Pool.create(ctx, total_blocks=8, layers=1, heads_kv=nkv, head_dim=d, kv_dtype=kind)
    with pytest.raises(gsp.InvalidArgument):  # not the pool geometry the step was packed for
        small.write_step(0, kd.data_ptr(), vd.data_ptr())
    small.destroy()
    for p in pools:
        p.destroy()


@pytest.mark.parametrize("dt,bs", [("f32", 16), ("f16", 16), ("f32", 32)])
def test_engine_tick_sequence_over_layers(torch_mod, gsp, ctx, dt, bs):
    """The per-tick sequence the integration prescribes (PagedTransformerRunner.cs:605-659 per layer):
    one gsp_step_pack for the tick, then for every layer gsp_rope_write_step (Q rotated in place, K
    rotated and stored, V stored at each query token's own slot) followed by gsp_attention_step on
    that layer.  Three layers, decode rows plus a prefill chunk (stored whole before its causal
    attention), each layer with its own Q/K/V, against the oracle doing the same rotation, store and
    attention layer by layer on the host arenas."""
    torch = torch_mod
    nh, nkv, d, base, layers = 28, 4, 128, 1000000.0, 3
    q_lens = np.array([1, 1, 23, 1, 1], np.int32)
    step = workloads.small_step(seed=131, rows=5, n_heads=nh, n_kv=nkv, head_dim=d, kv_dtype=dt, ctx_lo=10,
                                ctx_hi=300, total_blocks=256, q_lens=q_lens, block_size=bs)
    # Decode rows attend their newest token: position = TokenCount - 1 (the slot the tick allocated).
    for b in range(step.num_rows):
        if step.lens[b] == 1:
            step.positions[b] = step.token_counts[b] - 1
    print(f"case engine tick {dt} bs={bs} layers={layers}", flush=True)
    rng = np.random.default_rng(132)
    _, k, v = workloads.host_values(step, layers=layers)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    nq = step.total_q
    qs = [rng.standard_normal((nq, nh, d)).astype(np.float32) for _ in range(layers)]
    ks = [rng.standard_normal((nq, nkv, d)).astype(np.float32) for _ in range(layers)]
    vs = [rng.standard_normal((nq, nkv, d)).astype(np.float32) for _ in range(layers)]
    ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                  q_lens=step.q_lens)
    outs = []
    for l in range(layers):
        qd = torch.from_numpy(qs[l]).cuda()
        kd = torch.from_numpy(ks[l]).cuda()
        vd = torch.from_numpy(vs[l]).cuda()
        out = torch.full((nq, nh, d), float("nan"), device="cuda")
        torch.cuda.synchronize()  # torch fills on its own stream, the library on the context's
        pool.rope_write_step(l, nh, base, 1, qd.data_ptr(), kd.data_ptr(), vd.data_ptr())
        ctx.attention_step(pool, l, nh, qd.data_ptr(), out.data_ptr(), step.scale)
        ctx.sync()
        outs.append(out.cpu().numpy())
        del qd, kd, vd
    pool.destroy()
    # Oracle: the same rotation and store per layer on the host arenas (fp16 pools keep the rotated
    # K and the V rounded once), then the reference attention of that layer.
    npdt = np.float16 if dt == "f16" else np.float32
    k2, v2 = k.copy(), v.copy()
    for l in range(layers):
        qr = np.empty_like(qs[l])
        i = 0
        for b in range(step.num_rows):
            for t in range(int(step.lens[b])):
                p = int(step.positions[b]) + t
                qr[i] = orc.rope(qs[l][i], p, base, 1)
                blk = int(step.table(b)[p // bs])
                k2[blk, l, :, p % bs] = orc.rope(ks[l][i], p, base, 1).astype(npdt).astype(np.float32)
                v2[blk, l, :, p % bs] = vs[l][i].astype(npdt).astype(np.float32)
                i += 1
        ref = oracle_step(step, qr, k2, v2, layer=l)
        err = max_err(outs[l], ref)
        print(f"layer {l}: max abs err {err:.3e}", flush=True)
        assert not np.isnan(outs[l]).any()
        assert err <= (1e-4 if dt == "f32" else 2e-3)
