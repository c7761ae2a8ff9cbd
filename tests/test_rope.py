"""The oracle's rotary embedding (orc_rope), pinned without the reference.

QuantKernels.RoPE is closed code (PagedTransformerRunner.cs:253-267 calls it
before PagedBlockPool.Store), so the oracle restates the textbook definition
(Su et al., RoFormer): pair j of a head turns by pos * base^(-2j/d).  These
checks fix it by closed forms and invariants that a wrong exponent, a flipped
rotation, a swapped pairing or a lost position would break.
"""
import math

import numpy as np
import pytest

import glacier_oracle as orc

STYLES = [orc.ROPE_PAIRS, orc.ROPE_HALVES]


@pytest.mark.parametrize("style", STYLES)
@pytest.mark.parametrize("pos", [1, 3, 17, 1000, 40000])
def test_first_pair_turns_by_the_position(style, pos):
    # d = 2: a single pair with frequency base^0 = 1, so (1, 0) -> (cos p, sin p).
    y = orc.rope(np.array([1.0, 0.0], np.float32), pos, 10000.0, style)
    assert y[0] == pytest.approx(math.cos(pos), abs=2e-7)
    assert y[1] == pytest.approx(math.sin(pos), abs=2e-7)


def test_second_pair_frequency_and_direction():
    # d = 4, base 100: pair 1 turns by p * 100^(-2/4) = p / 10.
    p = 7
    x = np.array([0.0, 0.0, 2.0, 0.0], np.float32)
    y = orc.rope(x, p, 100.0, orc.ROPE_PAIRS)
    assert np.allclose(y, [0.0, 0.0, 2 * math.cos(0.7), 2 * math.sin(0.7)], atol=1e-6)
    # Halves: pair 1 is (x[1], x[3]).
    x = np.array([0.0, 0.0, 0.0, 3.0], np.float32)
    y = orc.rope(x, p, 100.0, orc.ROPE_HALVES)
    assert np.allclose(y, [0.0, -3 * math.sin(0.7), 0.0, 3 * math.cos(0.7)], atol=1e-6)


@pytest.mark.parametrize("style", STYLES)
def test_position_zero_is_the_identity(style):
    x = np.random.default_rng(1).standard_normal((5, 128)).astype(np.float32)
    assert np.array_equal(orc.rope(x, 0, 1e6, style), x)


@pytest.mark.parametrize("style", STYLES)
def test_pairs_keep_their_norm(style):
    rng = np.random.default_rng(2)
    x = rng.standard_normal((3, 64)).astype(np.float32)
    y = orc.rope(x, 12345, 10000.0, style).astype(np.float64)
    x = x.astype(np.float64)
    if style == orc.ROPE_PAIRS:
        nx = x[:, 0::2] ** 2 + x[:, 1::2] ** 2
        ny = y[:, 0::2] ** 2 + y[:, 1::2] ** 2
    else:
        nx = x[:, :32] ** 2 + x[:, 32:] ** 2
        ny = y[:, :32] ** 2 + y[:, 32:] ** 2
    assert np.allclose(nx, ny, rtol=1e-6, atol=1e-9)


@pytest.mark.parametrize("style", STYLES)
def test_scores_depend_only_on_relative_position(style):
    rng = np.random.default_rng(3)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    base = 1e6
    s = [float(np.dot(orc.rope(q, m + t, base, style).astype(np.float64), orc.rope(k, n + t, base, style)))
         for (m, n, t) in [(9, 4, 0), (9, 4, 100), (9, 4, 31000)]]
    assert s[1] == pytest.approx(s[0], abs=2e-4)
    assert s[2] == pytest.approx(s[0], abs=2e-4)
    # ... and does change with it.
    other = float(np.dot(orc.rope(q, 9, base, style).astype(np.float64), orc.rope(k, 5, base, style)))
    assert abs(other - s[0]) > 1e-3


def test_halves_is_pairs_after_interleaving():
    rng = np.random.default_rng(4)
    d = 128
    x = rng.standard_normal((2, d)).astype(np.float32)
    perm = np.empty(d, np.int64)  # pairs layout index 2j <- j, 2j + 1 <- j + d/2
    perm[0::2] = np.arange(d // 2)
    perm[1::2] = np.arange(d // 2) + d // 2
    for pos in (1, 77, 20000):
        a = orc.rope(x, pos, 500000.0, orc.ROPE_HALVES)
        b = orc.rope(x[:, perm], pos, 500000.0, orc.ROPE_PAIRS)
        assert np.array_equal(a[:, perm], b)


# ---- The runner's optional arguments: ropeDim, invFreqTable, ropeFreqs, mscale
# (PagedTransformerRunner.cs:253-264), orc_rope_ex.  No reference test holds
# vectors for them, so these fix the restatement by closed forms and by
# reduction to the plain rotation above.


@pytest.mark.parametrize("style", STYLES)
@pytest.mark.parametrize("rope_dim", [2, 32, 64, 96])
def test_partial_rotation_is_the_plain_rotation_of_the_first_dims(style, rope_dim):
    # Dims past rope_dim are untouched; the first rope_dim are a plain rotation of
    # a rope_dim-wide head (exponent -2j/rope_dim, HALVES pairs j with j + rope_dim/2).
    rng = np.random.default_rng(rope_dim + style)
    x = rng.standard_normal((3, 128)).astype(np.float32)
    for pos in (5, 4097, 30000):
        y = orc.rope_ex(x, pos, 10000.0, style, rope_dim=rope_dim)
        assert np.array_equal(y[:, rope_dim:], x[:, rope_dim:])
        assert np.array_equal(y[:, :rope_dim], orc.rope(x[:, :rope_dim], pos, 10000.0, style))


def test_full_rope_dim_is_the_plain_rotation():
    x = np.random.default_rng(7).standard_normal((2, 64)).astype(np.float32)
    for style in STYLES:
        assert np.array_equal(orc.rope_ex(x, 321, 1e6, style, rope_dim=64), orc.rope(x, 321, 1e6, style))
        assert np.array_equal(orc.rope_ex(x, 321, 1e6, style), orc.rope(x, 321, 1e6, style))


@pytest.mark.parametrize("style", STYLES)
def test_table_rates_closed_form(style):
    # d = 4 with the table (0.25, 3.0): pair 0 turns by pos/4, pair 1 by 3 pos;
    # the base is ignored.
    pos = 9
    x = np.array([1.0, 0.0, 0.0, 0.0], np.float32)
    y = orc.rope_ex(x, pos, 123.0, style, inv_freq=[0.25, 3.0])
    if style == orc.ROPE_PAIRS:  # pair 0 = (x0, x1)
        assert np.allclose(y, [math.cos(2.25), math.sin(2.25), 0, 0], atol=1e-7)
    else:  # pair 0 = (x0, x2)
        assert np.allclose(y, [math.cos(2.25), 0, math.sin(2.25), 0], atol=1e-7)
    # Pair 1 is (x2, x3) for PAIRS and (x1, x3) for HALVES.
    x = np.array([0.0, 0.0, 2.0, 0.0] if style == orc.ROPE_PAIRS else [0.0, 2.0, 0.0, 0.0], np.float32)
    y = orc.rope_ex(x, pos, 123.0, style, inv_freq=[0.25, 3.0])
    c, s = 2 * math.cos(27.0), 2 * math.sin(27.0)
    want = [0, 0, c, s] if style == orc.ROPE_PAIRS else [0, c, 0, s]
    assert np.allclose(y, want, atol=1e-6)


def test_frequency_factors_divide_the_angle():
    # d = 2, base rate 1: a factor of 4 turns (1, 0) by pos / 4; with a table
    # of 0.5 as well, by pos / 8.
    for pos in (3, 1000):
        y = orc.rope_ex(np.array([1.0, 0.0], np.float32), pos, 10000.0, freq_factors=[4.0])
        assert np.allclose(y, [math.cos(pos / 4), math.sin(pos / 4)], atol=2e-7)
        y = orc.rope_ex(np.array([1.0, 0.0], np.float32), pos, 10000.0, inv_freq=[0.5], freq_factors=[4.0])
        assert np.allclose(y, [math.cos(pos / 8), math.sin(pos / 8)], atol=2e-7)
    # Factors of 1 change nothing; a factor f equals the table base^(-2j/d) / f.
    x = np.random.default_rng(8).standard_normal(64).astype(np.float32)
    assert np.array_equal(orc.rope_ex(x, 777, 1e4, freq_factors=np.ones(32)), orc.rope(x, 777, 1e4))
    f = np.linspace(1.0, 8.0, 32).astype(np.float32)
    rates = (1e4 ** (-2.0 * np.arange(32) / 64) / f.astype(np.float64)).astype(np.float32)
    a = orc.rope_ex(x, 50, 1e4, freq_factors=f)
    b = orc.rope_ex(x, 50, 1e4, inv_freq=rates)
    assert np.allclose(a, b, atol=1e-5)


@pytest.mark.parametrize("style", STYLES)
def test_mscale_scales_the_rotated_dims_only(style):
    rng = np.random.default_rng(9)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    m = 1.3862944
    # Position 0: rotated dims times mscale, the rest untouched.
    y = orc.rope_ex(x, 0, 1e4, style, rope_dim=64, mscale=m)
    assert np.allclose(y[:, :64], m * x[:, :64].astype(np.float64), rtol=1e-7, atol=1e-7)
    assert np.array_equal(y[:, 64:], x[:, 64:])
    # Any position: mscale times the unscaled rotation.
    y = orc.rope_ex(x, 12345, 1e4, style, rope_dim=64, mscale=m)
    z = orc.rope_ex(x, 12345, 1e4, style, rope_dim=64)
    assert np.allclose(y[:, :64], m * z[:, :64].astype(np.float64), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("style", STYLES)
def test_table_rotation_keeps_relative_positions(style):
    # Any rate table keeps q.k a function of the position difference (scaled by mscale^2).
    rng = np.random.default_rng(10)
    q = rng.standard_normal(128).astype(np.float32)
    k = rng.standard_normal(128).astype(np.float32)
    tab = orc.yarn_inv_freq(128, 1e6, 8.0, 32768)
    m = orc.yarn_mscale(8.0)

    def score(a, b):
        qa = orc.rope_ex(q, a, 0.0, style, inv_freq=tab, mscale=m).astype(np.float64)
        return float(np.dot(qa, orc.rope_ex(k, b, 0.0, style, inv_freq=tab, mscale=m)))

    s0 = score(900, 100)
    assert score(900 + 50000, 100 + 50000) == pytest.approx(s0, abs=5e-4)
    plain = float(np.dot(q.astype(np.float64), k))
    assert score(7, 7) == pytest.approx(m * m * plain, rel=1e-5)


def test_yarn_table_shape():
    # The generator used for test tables: fast pairs keep base^(-2j/d), slow pairs
    # are divided by the factor, the rates fall with j, and factor 1 is the identity.
    d, base, s, ctx = 128, 1e6, 4.0, 32768
    theta = base ** (-2.0 * np.arange(d // 2) / d)
    t = orc.yarn_inv_freq(d, base, s, ctx).astype(np.float64)
    assert t[0] == pytest.approx(theta[0], rel=1e-7)
    assert t[-1] == pytest.approx(theta[-1] / s, rel=1e-6)
    assert np.all(np.diff(t) < 0)
    assert np.allclose(orc.yarn_inv_freq(d, base, 1.0, ctx), theta, rtol=1e-6)
    assert orc.yarn_mscale(1.0) == 1.0 and orc.yarn_mscale(math.e) == pytest.approx(1.1)
