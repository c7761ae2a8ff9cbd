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


# ---- The runner's optional RoPE arguments (gsp_rope_write_*_ex): ropeDim
# (partial rotation), invFreqTable (YaRN), ropeFreqs (frequency factors) and
# mscale, PagedTransformerRunner.cs:86-104 and :253-264, against orc_rope_ex.

def _factors(n):
    return np.linspace(1.0, 6.0, n).astype(np.float32)


EX_CASES = [
    # (n_heads, n_kv, head_dim, kv dtype, rope_dim, YaRN table, frequency factors, mscale)
    (16, 2, 128, "f32", 64, False, False, 0.0),   # partial, 16-byte kernel
    (16, 2, 128, "f16", 64, True, False, None),   # partial YaRN, fp16 pool
    (28, 4, 128, "f32", 0, True, False, None),    # full-head YaRN
    (8, 8, 64, "f32", 0, False, True, 0.0),       # frequency factors
    (12, 4, 128, "f16", 96, True, True, 1.25),    # all of them
    (6, 2, 64, "f32", 36, False, False, 0.0),     # rope_dim % 8 != 0: the per-element kernel
    (6, 2, 64, "f16", 20, True, True, 1.5),       # the same with tables
    (4, 2, 48, "f32", 16, True, False, None),     # 16-byte kernel, 48-dim heads
]


def _rope_of(gsp, case, style, base):
    nh, nkv, d, dt, rd, yarn, fac, ms = case
    half = (rd or d) // 2
    inv = orc.yarn_inv_freq(rd or d, base, 8.0, 4096) if yarn else None
    ff = _factors(half) if fac else None
    if ms is None:
        ms = orc.yarn_mscale(8.0)
    return gsp.Rope(base, style, rd, inv_freq=inv, freq_factors=ff, mscale=ms)


def _oracle_rot(x, pos, rope):
    return orc.rope_ex(x, pos, rope.freq_base, rope.style, rope.rope_dim, rope.inv_freq, rope.freq_factors,
                       rope.mscale or 1.0)


@pytest.mark.parametrize("style", [0, 1], ids=["pairs", "halves"])
@pytest.mark.parametrize("case", EX_CASES, ids=lambda c: f"{c[0]}q{c[1]}kv_d{c[2]}_r{c[4]}_{c[3]}"
                         f"{'_yarn' if c[5] else ''}{'_ff' if c[6] else ''}")
def test_rope_ex_write_matches_oracle(torch_mod, gsp, ctx, case, style):
    """Rotated dims within 2e-6 x mscale of the fp64 oracle (fp32), one fp16 ulp (fp16 pools); dims
    past rope_dim are Q's own values and K's values stored as they are, bit for bit; V bit-exact."""
    torch = torch_mod
    nh, nkv, d, dt, rd, yarn, fac, ms = case
    base = 1000000.0
    print(f"case rope_ex {case} style={style}", flush=True)
    rope = _rope_of(gsp, case, style, base)
    rng = np.random.default_rng(nh * 11 + d + rd + style)
    n, total_blocks = 29, 64
    positions, blocks, slots = _tokens(rng, n, total_blocks)
    positions[3] = 131071  # far past the original context of the YaRN table
    q = rng.standard_normal((n, nh, d)).astype(np.float32)
    k = rng.standard_normal((n, nkv, d)).astype(np.float32)
    v = rng.standard_normal((n, nkv, d)).astype(np.float32)
    pool = gsp.Pool.create(ctx, total_blocks=total_blocks, layers=2, heads_kv=nkv, head_dim=d,
                           kv_dtype=gsp.KV_F16 if dt == "f16" else gsp.KV_F32)
    qd = torch.from_numpy(q).cuda()
    kd = torch.from_numpy(k).cuda()
    vd = torch.from_numpy(v).cuda()
    torch.cuda.synchronize()
    pool.rope_write_tokens_ex(1, positions, blocks, slots, nh, rope, qd.data_ptr(), kd.data_ptr(), vd.data_ptr())
    ctx.sync()
    npdt = np.float16 if dt == "f16" else np.float32
    _, _, kb, vb = pool.arenas()
    K = pool.download(0, kb).view(npdt).reshape(total_blocks, 2, nkv, 16, d)
    V = pool.download(1, vb).view(npdt).reshape(total_blocks, 2, nkv, 16, d)
    got_q = qd.cpu().numpy()
    r = rd or d
    scale = max(1.0, rope.mscale)
    tol = 2e-3 * scale if dt == "f16" else 2e-6 * scale
    for i in range(n):
        ref_q = _oracle_rot(q[i], int(positions[i]), rope)
        ref_k = _oracle_rot(k[i], int(positions[i]), rope)
        assert max_err(got_q[i][:, :r], ref_q[:, :r]) <= 2e-6 * scale, f"q of token {i} at {positions[i]}"
        assert np.array_equal(got_q[i][:, r:], q[i][:, r:]), f"q tail of token {i}"
        got_k = K[blocks[i], 1, :, slots[i]]
        assert max_err(got_k[:, :r].astype(np.float32), ref_k[:, :r]) <= tol, f"k of token {i}"
        assert np.array_equal(got_k[:, r:], k[i][:, r:].astype(npdt)), f"k tail of token {i}"
        assert np.array_equal(V[blocks[i], 1, :, slots[i]], v[i].astype(npdt)), f"v of token {i}"
    mask = np.ones(K.shape, bool)
    mask[blocks, 1, :, slots] = False
    assert not K[mask].any() and not V[mask].any()
    pool.destroy()


def test_rope_ex_plain_spec_is_the_plain_call(torch_mod, gsp, ctx):
    """A spec with only freq_base and style set is gsp_rope_write_tokens, bit for bit."""
    torch = torch_mod
    rng = np.random.default_rng(201)
    n, nh, nkv, d = 17, 8, 2, 128
    positions, blocks, slots = _tokens(rng, n, 32)
    q = rng.standard_normal((n, nh, d)).astype(np.float32)
    k = rng.standard_normal((n, nkv, d)).astype(np.float32)
    pools = [gsp.Pool.create(ctx, total_blocks=32, layers=1, heads_kv=nkv, head_dim=d) for _ in range(2)]
    qs = [torch.from_numpy(q).cuda() for _ in range(2)]
    kd = torch.from_numpy(k).cuda()
    torch.cuda.synchronize()
    pools[0].rope_write_tokens(0, positions, blocks, slots, nh, 5e5, 1, qs[0].data_ptr(), kd.data_ptr(), kd.data_ptr())
    pools[1].rope_write_tokens_ex(0, positions, blocks, slots, nh, gsp.Rope(5e5, 1), qs[1].data_ptr(), kd.data_ptr(),
                                  kd.data_ptr())
    ctx.sync()
    assert torch.equal(qs[0], qs[1])
    _, _, kb, _ = pools[0].arenas()
    assert np.array_equal(pools[0].download(0, kb), pools[1].download(0, kb))
    for p in pools:
        p.destroy()


def test_rope_ex_errors_and_table_cache(torch_mod, gsp, ctx):
    """Malformed rotations are refused before anything is enqueued; more distinct tables than the
    context keeps on the device (16) still rotate by their own rates, each checked against the
    oracle, including a table evicted and set again."""
    torch = torch_mod
    import ctypes

    d = 64
    pool = gsp.Pool.create(ctx, total_blocks=8, layers=1, heads_kv=2, head_dim=d)
    k = torch.ones((2, 2, d), device="cuda")
    q = torch.full((2, 4, d), 0.5, device="cuda")
    torch.cuda.synchronize()
    bad = [
        gsp.Rope(1e4, 0, rope_dim=3), gsp.Rope(1e4, 0, rope_dim=66), gsp.Rope(1e4, 0, rope_dim=-2),
        gsp.Rope(1e4, 0, mscale=-1.0), gsp.Rope(1e4, 0, mscale=float("nan")), gsp.Rope(1e4, 2),
        gsp.Rope(0.0, 0), gsp.Rope(1e4, 0, inv_freq=np.full(32, np.nan)),
        gsp.Rope(1e4, 0, inv_freq=np.full(32, -1.0)), gsp.Rope(1e4, 0, freq_factors=np.zeros(32)),
        gsp.Rope(1e4, 0, freq_factors=np.full(32, np.inf)),
    ]
    for rope in bad:
        with pytest.raises(gsp.InvalidArgument):
            pool.rope_write_tokens_ex(0, [1], [0], [0], 4, rope, q.data_ptr(), k.data_ptr(), k.data_ptr())
    with pytest.raises(ValueError):  # the wrapper checks the table length the library will read
        pool.rope_write_tokens_ex(0, [1], [0], [0], 4, gsp.Rope(1e4, 0, inv_freq=np.ones(31)), q.data_ptr(),
                                  k.data_ptr(), k.data_ptr())
    rc = gsp.load().gsp_rope_write_tokens_ex(ctx.handle, pool.handle, 0, 1, (ctypes.c_int32 * 1)(1),
                                             (ctypes.c_int32 * 1)(0), (ctypes.c_int32 * 1)(0), 0, None, None,
                                             ctypes.c_void_p(k.data_ptr()), ctypes.c_void_p(k.data_ptr()))
    assert rc == gsp.GSP_E_INVALID_ARG
    # A table with inv_freq ignores freq_base, so a zero base is accepted with it.
    rng = np.random.default_rng(202)
    kv = rng.standard_normal((1, 2, d)).astype(np.float32)
    kd = torch.from_numpy(kv).cuda()
    torch.cuda.synchronize()
    _, _, kb, _ = pool.arenas()
    tables = [orc.yarn_inv_freq(d, 1e4, 1.0 + t, 2048) for t in range(18)] + [None]
    tables.append(orc.yarn_inv_freq(d, 1e4, 1.0, 2048))  # evicted by now: set again
    for t, tab in enumerate(tables):
        rope = gsp.Rope(0.0 if tab is not None else 1e4, 1, inv_freq=tab)
        pos = 1000 + 37 * t
        pool.rope_write_tokens_ex(0, [pos], [t % 8], [t % 16], 0, rope, 0, kd.data_ptr(), kd.data_ptr())
        ctx.sync()
        K = pool.download(0, kb).view(np.float32).reshape(8, 1, 2, 16, d)
        ref = orc.rope_ex(kv[0], pos, rope.freq_base, 1, inv_freq=tab)
        assert max_err(K[t % 8, 0, :, t % 16], ref) <= 2e-6, f"table {t}"
    pool.destroy()


@pytest.mark.parametrize("dt", ["f32", "f16"])
def test_yarn_engine_tick_over_layers(torch_mod, gsp, ctx, dt):
    """The engine tick with the CPU runner's YaRN setup on a partial-RoPE head: one gsp_step_pack,
    then per layer gsp_rope_write_step_ex (rope_dim 64 of 128, a YaRN table, mscale on Q and K) and
    gsp_attention_step at scale 1/sqrt(head_dim) (PagedTransformerRunner.cs:100-103 keeps the scale),
    against the oracle doing the same rotation, store and attention per layer; the step form's stores
    equal gsp_rope_write_tokens_ex's bit for bit."""
    torch = torch_mod
    nh, nkv, d, base, layers, rd = 16, 2, 128, 1000000.0, 2, 64
    rope = gsp.Rope(base, 1, rd, inv_freq=orc.yarn_inv_freq(rd, base, 4.0, 4096), mscale=orc.yarn_mscale(4.0))
    q_lens = np.array([1, 1, 21, 1], np.int32)
    step = workloads.small_step(seed=141, rows=4, n_heads=nh, n_kv=nkv, head_dim=d, kv_dtype=dt, ctx_lo=30,
                                ctx_hi=400, total_blocks=256, q_lens=q_lens)
    for b in range(step.num_rows):
        if step.lens[b] == 1:
            step.positions[b] = step.token_counts[b] - 1
    print(f"case yarn tick {dt}", flush=True)
    rng = np.random.default_rng(142)
    _, k, v = workloads.host_values(step, layers=layers)
    pool, keep = to_device_pool(torch, gsp, ctx, step, k, v)
    twin, keep2 = to_device_pool(torch, gsp, ctx, step, k, v)
    nq = step.total_q
    qs = [rng.standard_normal((nq, nh, d)).astype(np.float32) for _ in range(layers)]
    ks = [rng.standard_normal((nq, nkv, d)).astype(np.float32) for _ in range(layers)]
    vs = [rng.standard_normal((nq, nkv, d)).astype(np.float32) for _ in range(layers)]
    pos = np.concatenate([int(step.positions[b]) + np.arange(int(step.lens[b])) for b in range(step.num_rows)])
    blk = np.array([int(step.table(b)[p // 16]) for b in range(step.num_rows)
                    for p in int(step.positions[b]) + np.arange(int(step.lens[b]))], np.int32)
    ctx.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len,
                  q_lens=step.q_lens)
    outs = []
    for l in range(layers):
        qd = torch.from_numpy(qs[l]).cuda()
        q2 = torch.from_numpy(qs[l]).cuda()
        kd = torch.from_numpy(ks[l]).cuda()
        vd = torch.from_numpy(vs[l]).cuda()
        out = torch.full((nq, nh, d), float("nan"), device="cuda")
        torch.cuda.synchronize()
        pool.rope_write_step_ex(l, nh, rope, qd.data_ptr(), kd.data_ptr(), vd.data_ptr())
        twin.rope_write_tokens_ex(l, pos, blk, pos % 16, nh, rope, q2.data_ptr(), kd.data_ptr(), vd.data_ptr())
        ctx.attention_step(pool, l, nh, qd.data_ptr(), out.data_ptr(), step.scale)
        ctx.sync()
        assert torch.equal(qd, q2)
        outs.append(out.cpu().numpy())
    npdt = np.float16 if dt == "f16" else np.float32
    _, _, kb, vb = pool.arenas()
    assert np.array_equal(pool.download(0, kb), twin.download(0, kb))
    assert np.array_equal(pool.download(1, vb), twin.download(1, vb))
    pool.destroy()
    twin.destroy()
    k2, v2 = k.copy(), v.copy()
    for l in range(layers):
        qr = np.empty_like(qs[l])
        for i in range(nq):
            p = int(pos[i])
            qr[i] = _oracle_rot(qs[l][i], p, rope)
            k2[blk[i], l, :, p % 16] = _oracle_rot(ks[l][i], p, rope).astype(npdt).astype(np.float32)
            v2[blk[i], l, :, p % 16] = vs[l][i].astype(npdt).astype(np.float32)
        ref = oracle_step(step, qr, k2, v2, layer=l)
        err = max_err(outs[l], ref)
        print(f"layer {l}: max abs err {err:.3e}", flush=True)
        assert not np.isnan(outs[l]).any()
        assert err <= (1e-4 if dt == "f32" else 2e-3)


@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_rope_ex_step_capture(torch_mod, gsp):
    """gsp_rope_write_step_ex captured into a graph: a table set by an eager call replays with its
    rates (every replay equal to the eager write, eager work between replays); a table not yet on
    the device is refused during the capture with a state error."""
    torch = torch_mod
    nkv, d, base = 2, 128, 1e6
    step = workloads.small_step(seed=151, rows=6, n_heads=8, n_kv=nkv, head_dim=d, ctx_lo=20, ctx_hi=200,
                                total_blocks=128)
    for b in range(step.num_rows):
        step.positions[b] = step.token_counts[b] - 1
    rope = gsp.Rope(base, 1, 96, inv_freq=orc.yarn_inv_freq(96, base, 4.0, 4096), mscale=1.2)
    other = gsp.Rope(base, 1, 96, inv_freq=orc.yarn_inv_freq(96, base, 2.0, 4096))
    print("case rope_ex capture", flush=True)
    rng = np.random.default_rng(152)
    k = rng.standard_normal((step.total_q, nkv, d)).astype(np.float32)
    v = rng.standard_normal((step.total_q, nkv, d)).astype(np.float32)
    with gsp.Context(0) as fresh:
        pool = gsp.Pool.create(fresh, total_blocks=step.total_blocks, layers=1, heads_kv=nkv, head_dim=d)
        stream = torch.cuda.Stream()
        fresh.set_stream(stream.cuda_stream)
        try:
            kd = torch.from_numpy(k).cuda()
            vd = torch.from_numpy(v).cuda()
            torch.cuda.synchronize()
            fresh.pack_step(pool, step.positions, step.token_counts, step.bt_offsets, step.bt_ids, step.max_seq_len)
            pool.rope_write_step_ex(0, 0, rope, 0, kd.data_ptr(), vd.data_ptr())
            fresh.sync()
            _, _, kb, _ = pool.arenas()
            eager = pool.download(0, kb).copy()
            graph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(graph, stream=stream):
                pool.rope_write_step_ex(0, 0, rope, 0, kd.data_ptr(), vd.data_ptr())
            bad = torch.cuda.CUDAGraph()
            with pytest.raises(gsp.StateError):
                with torch.cuda.graph(bad, stream=stream):
                    pool.rope_write_step_ex(0, 0, other, 0, kd.data_ptr(), vd.data_ptr())
            del bad
            torch.cuda.synchronize()
            for rep in range(3):
                pool.upload(0, np.zeros(kb // 4, np.float32))
                fresh.sync()
                graph.replay()
                torch.cuda.synchronize()
                assert np.array_equal(pool.download(0, kb), eager), f"replay {rep}"
                # Eager work between replays, with the other table (now placed on the device too).
                pool.rope_write_step_ex(0, 0, other, 0, kd.data_ptr(), vd.data_ptr())
                fresh.sync()
            del graph
        finally:
            fresh.set_stream(None)
            pool.destroy()
