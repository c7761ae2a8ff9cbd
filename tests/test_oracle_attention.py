"""Pins the CPU oracle's ComputeAttention restatement (PagedAttentionKernel.cs:17-372).

Checks, each chosen so that a plausible slip in the oracle fails one:
  * the reference's own test case (PagedAttentionTests.cs:111-179) against its
    closed form and a fixed fp64 value;
  * the reference's bounds tests (PhaseCServeRemediationTests.cs:117-175);
  * a dense numpy/scipy attention over K/V gathered straight from the pool
    layout (PagedBlockPool.cs:128-131,140-143) for many head geometries and
    every ISA path (catches a transposed operand, a wrong GQA map, a dropped
    scale, a wrong page or slot index);
  * invariants: physical-id permutation, uniform V, ctx = 1, equal queries in
    a GQA group, prefill row == decode rows (PhaseCServeRemediationTests.cs:256-319).
"""
import math

import numpy as np
import pytest
from scipy.special import softmax

import glacier_oracle as orc

BS = 16


def make_pool(rng, blocks, layers, hkv, d, dv=None, f16=False):
    dv = dv or d
    k = rng.standard_normal((blocks, layers, hkv, BS, d), dtype=np.float32)
    v = rng.standard_normal((blocks, layers, hkv, BS, dv), dtype=np.float32)
    if f16:
        k = k.astype(np.float16).astype(np.float32)
        v = v.astype(np.float16).astype(np.float32)
    return k, v


def dense_reference(k, v, ids, total, layer, q, n_heads, scale):
    """softmax(q K^T * scale) V in fp64 over K/V gathered by (ids[t // 16], t % 16)."""
    hkv_n = k.shape[2]
    group = n_heads // hkv_n
    t = np.arange(total)
    blk = np.asarray(ids)[t // BS]
    slot = t % BS
    q = q.reshape(n_heads, -1).astype(np.float64)
    out = np.zeros((n_heads, v.shape[4]))
    for h in range(n_heads):
        kk = k[blk, layer, h // group, slot, :].astype(np.float64)
        vv = v[blk, layer, h // group, slot, :].astype(np.float64)
        p = softmax(kk @ q[h] * scale)
        out[h] = p @ vv
    return out


def test_reference_headdim128_case_closed_form():
    """PagedAttentionTests.cs:111-179: k_t = 0.01 (t+1), V = (t+1) / 2 (t+1), q = 1."""
    d, total, nh, nkv = 128, 32, 4, 2
    k = np.zeros((8, 1, nkv, BS, d), np.float32)
    v = np.zeros_like(k)
    ids = [0, 1]  # the first two pops of a fresh free stack
    for t in range(total):
        k[ids[t // BS], 0, :, t % BS, :] = np.float32(0.01) * (t + 1)
        v[ids[t // BS], 0, 0, t % BS, :] = t + 1
        v[ids[t // BS], 0, 1, t % BS, :] = 2.0 * (t + 1)
    pool = orc.HostPool(k, v)
    q = np.ones(nh * d, np.float32)
    scale = 1.0 / math.sqrt(d)
    for isa in (orc.ISA_SCALAR, orc.ISA_AVX2, orc.ISA_AVX512):
        if isa > orc.host_isa():
            continue
        out = orc.compute_attention(pool, ids, total, 0, total - 1, q, nh, scale, total, isa=isa).reshape(nh, d)
        # Closed form: scores s_t = 128 * 0.01 (t+1) / sqrt(128); out = sum softmax(s)_t * V_t.
        s = np.array([d * 0.01 * (t + 1) / math.sqrt(d) for t in range(total)])
        w = np.exp(s - s.max())
        w /= w.sum()
        expect0 = float(np.dot(w, np.arange(1, total + 1)))
        assert expect0 == pytest.approx(24.532020609, abs=1e-8)
        np.testing.assert_allclose(out[:2], expect0, atol=1e-4)
        np.testing.assert_allclose(out[2:], 2 * expect0, atol=1e-4)
        assert 2 * expect0 == pytest.approx(49.064041217, abs=1e-8)
        # The reference asserts per-head constancy to 4 decimals (:167-176).
        assert np.all(np.abs(out - out[:, :1]) < 5e-5)


def test_rejects_out_of_bounds_position():
    """PhaseCServeRemediationTests.cs:117-175: pos=16 with maxSeqLen=16, and pos=-1, throw."""
    k = np.zeros((4, 1, 1, BS, 32), np.float32)
    pool = orc.HostPool(k, k.copy())
    q = np.zeros(32, np.float32)
    for pos in (16, -1):
        with pytest.raises(orc.ArgumentOutOfRange):
            orc.compute_attention(pool, [0], 1, 0, pos, q, 1, 1 / math.sqrt(32), 16)
    with pytest.raises(orc.ArgumentOutOfRange):  # maxSeqLen <= 0 (:34-35)
        orc.compute_attention(pool, [0], 1, 0, 0, q, 1, 1.0, 0)
    with pytest.raises(orc.ArgumentOutOfRange):  # TokenCount > maxSeqLen (:38-39)
        orc.compute_attention(pool, [0, 1], 17, 0, 0, q, 1, 1.0, 16)


def test_zero_tokens_leaves_out_untouched():
    """totalTokens == 0 returns before writing out (PagedAttentionKernel.cs:41-42)."""
    k = np.ones((4, 1, 1, BS, 32), np.float32)
    pool = orc.HostPool(k, k.copy())
    out = np.full(32, 7.25, np.float32)
    orc.compute_attention(pool, [], 0, 0, 5, np.ones(32, np.float32), 1, 1.0, 16, out=out)
    assert np.all(out == 7.25)


GEOMS = [
    # (n_heads, n_kv, d, dv)
    (1, 1, 32, 32),
    (4, 2, 64, 64),
    (14, 2, 64, 64),
    (28, 4, 128, 128),
    (8, 8, 128, 128),
    (32, 8, 128, 128),
    (8, 1, 256, 256),
    (6, 3, 48, 48),
    (4, 2, 64, 32),   # asymmetric vHeadDim (generic PV path)
    (4, 1, 40, 24),   # non-multiple-of-8 dims (scalar tails)
]


@pytest.mark.parametrize("geom", GEOMS)
@pytest.mark.parametrize("isa", [orc.ISA_SCALAR, orc.ISA_AVX2, orc.ISA_AVX512])
def test_matches_dense_fp64(geom, isa):
    if isa > orc.host_isa():
        pytest.skip("ISA not available on this host")
    nh, nkv, d, dv = geom
    rng = np.random.default_rng(hash(geom) & 0xFFFF)
    k, v = make_pool(rng, 24, 2, nkv, d, dv)
    pool = orc.HostPool(k, v)
    ids = rng.permutation(24)[:7]
    for total in (1, 15, 16, 17, 100, 112):
        tc = total
        pos = total - 1
        q = rng.standard_normal(nh * d, dtype=np.float32)
        scale = 1 / math.sqrt(d)
        out = orc.compute_attention(pool, ids, tc, 1, pos, q, nh, scale, 4096, isa=isa, n_threads=3)
        ref = dense_reference(k, v, ids, total, 1, q, nh, scale)
        np.testing.assert_allclose(out.reshape(nh, dv), ref, atol=2e-6, rtol=1e-5)
        f64 = orc.attention_fp64(pool, ids, tc, 1, pos, q, nh, scale, 4096)
        np.testing.assert_allclose(f64.reshape(nh, dv), ref, atol=1e-12, rtol=1e-10)


def test_total_is_min_of_token_count_and_pos_plus_one():
    """totalTokens = min(TokenCount, pos + 1) (PagedAttentionKernel.cs:41)."""
    rng = np.random.default_rng(3)
    k, v = make_pool(rng, 8, 1, 2, 64)
    pool = orc.HostPool(k, v)
    ids = [5, 2, 7]
    q = rng.standard_normal(4 * 64, dtype=np.float32)
    # pos beyond TokenCount: attends to TokenCount tokens.
    a = orc.compute_attention(pool, ids, 40, 0, 45, q, 4, 0.125, 4096)
    np.testing.assert_allclose(a.reshape(4, 64), dense_reference(k, v, ids, 40, 0, q, 4, 0.125), atol=2e-6)
    # pos inside: causal cut at pos + 1.
    b = orc.compute_attention(pool, ids, 40, 0, 20, q, 4, 0.125, 4096)
    np.testing.assert_allclose(b.reshape(4, 64), dense_reference(k, v, ids, 21, 0, q, 4, 0.125), atol=2e-6)


def test_invariants():
    rng = np.random.default_rng(11)
    nh, nkv, d = 8, 2, 64
    k, v = make_pool(rng, 64, 1, nkv, d)
    pool = orc.HostPool(k, v)
    q = rng.standard_normal(nh * d, dtype=np.float32)
    ids = rng.permutation(64)[:5]
    base = orc.compute_attention(pool, ids, 70, 0, 69, q, nh, 0.125, 4096)

    # Moving the pages to other physical blocks changes nothing (bit-exact).
    perm = rng.permutation(64)
    k2 = np.empty_like(k)
    v2 = np.empty_like(v)
    k2[perm] = k
    v2[perm] = v
    moved = orc.compute_attention(orc.HostPool(k2, v2), perm[ids], 70, 0, 69, q, nh, 0.125, 4096)
    assert np.array_equal(base, moved)

    # ctx == 1 returns v_0 of each head's KV head.
    one = orc.compute_attention(pool, ids, 1, 0, 0, q, nh, 0.125, 4096).reshape(nh, d)
    for h in range(nh):
        np.testing.assert_allclose(one[h], v[ids[0], 0, h // (nh // nkv), 0], atol=1e-6)

    # Uniform V gives out == V whatever the scores.
    vu = np.broadcast_to(np.arange(d, dtype=np.float32), v.shape).copy()
    uni = orc.compute_attention(orc.HostPool(k, vu), ids, 70, 0, 69, q, nh, 0.125, 4096).reshape(nh, d)
    np.testing.assert_allclose(uni, np.broadcast_to(np.arange(d), (nh, d)), atol=1e-4)

    # Equal queries inside a GQA group give equal outputs; different groups differ.
    qg = np.repeat(rng.standard_normal((nkv, 1, d), dtype=np.float32), nh // nkv, axis=1).reshape(-1)
    g = orc.compute_attention(pool, ids, 70, 0, 69, qg, nh, 0.125, 4096).reshape(nkv, nh // nkv, d)
    assert np.array_equal(g, np.broadcast_to(g[:, :1], g.shape))
    assert not np.allclose(g[0, 0], g[1, 0])


def test_prefill_row_equals_decode_rows():
    """A chunk's query t equals a decode call at pos = start + t (PhaseCServeRemediationTests.cs:256-319)."""
    rng = np.random.default_rng(5)
    nh, nkv, d = 7, 1, 64
    k, v = make_pool(rng, 32, 1, nkv, d)
    pool = orc.HostPool(k, v)
    ids = rng.permutation(32)[:6]
    start, n = 37, 40  # chunk [37, 77) stored before attention, TokenCount = 77
    q = rng.standard_normal((n, nh, d), dtype=np.float32)
    out = orc.attention_step(pool, 0, [start], [start + n], [0, len(ids)], ids, q, nh, 0.125, 4096, q_lens=[n])
    for t in range(n):
        single = orc.compute_attention(pool, ids, start + n, 0, start + t, q[t], nh, 0.125, 4096)
        assert np.array_equal(out[t].reshape(-1), single)
        ref = dense_reference(k, v, ids, start + t + 1, 0, q[t], nh, 0.125)
        np.testing.assert_allclose(out[t], ref, atol=2e-6)


def test_sink_is_rejected():
    k = np.zeros((2, 1, 1, BS, 32), np.float32)
    pool = orc.HostPool(k, k.copy())
    with pytest.raises(NotImplementedError):
        orc.compute_attention(pool, [0], 1, 0, 0, np.zeros(32, np.float32), 1, 1.0, 16, sink_logit=0.5)


def test_bad_geometry_rejected():
    k = np.zeros((2, 1, 2, BS, 32), np.float32)
    pool = orc.HostPool(k, k.copy())
    q = np.zeros(3 * 32, np.float32)
    with pytest.raises(orc.ArgumentOutOfRange):  # 3 heads on 2 KV heads: head 2 maps to KV head 2
        orc.compute_attention(pool, [0], 1, 0, 0, q, 3, 1.0, 16)
    with pytest.raises(orc.ArgumentOutOfRange):  # table shorter than the tokens
        orc.compute_attention(pool, [0], 20, 0, 19, np.zeros(2 * 32, np.float32), 2, 1.0, 32)
    with pytest.raises(orc.ArgumentOutOfRange):  # block id outside the pool
        orc.compute_attention(pool, [5], 1, 0, 0, np.zeros(2 * 32, np.float32), 2, 1.0, 16)
