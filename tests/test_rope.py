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
