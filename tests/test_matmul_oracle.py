"""The oracle's Q8_0 encoding and projection product, pinned without the reference.

The encoding follows the reference's test builder (PhaseCServeRemediationTests.cs:1587-1622);
these checks fix it by closed forms a wrong rounding mode, scale, byte order or clamp would
break.  QuantKernels.MatMulBatch is closed code, so the product is the definition
y[b][o] = sum_i W[o][i] x[b][i], checked against explicit loops (which pin the orientation).
"""
import struct

import numpy as np
import pytest

import glacier_oracle as orc


def _block(values):
    v = np.zeros(32, np.float32)
    v[: len(values)] = values
    return v


def test_unit_scale_rounds_half_to_even():
    # maxAbs 127 gives d = 1 exactly, so q = Round(v) with ties to even (MathF.Round).
    b = orc.q8_0_encode(_block([127, 2.5, 3.5, -2.5, -3.5, 0.5, -0.5, 1.5, -126.6]))
    assert struct.unpack("<e", b[:2].tobytes())[0] == 1.0
    assert list(b[2:11].view(np.int8)) == [127, 2, 4, -2, -4, 0, 0, 2, -127]


def test_scale_is_fp16_of_max_over_127():
    v = np.linspace(-1.0, 0.75, 32).astype(np.float32)
    b = orc.q8_0_encode(v)
    assert b[:2].tobytes() == np.float16(np.float32(1.0) / np.float32(127.0)).tobytes()  # little-endian fp16
    d = float(np.float16(np.float32(1.0) / np.float32(127.0)))
    inv = np.float32(1.0) / np.float32(d)
    assert np.array_equal(b[2:].view(np.int8), np.rint(v * inv).astype(np.int8))


def test_zero_block_and_clamp():
    z = orc.q8_0_encode(np.zeros(32, np.float32))
    assert not z.any()  # d = 0, invD = 0, q = 0
    # A subnormal fp16 scale rounds far below maxAbs / 127, so maxAbs * invD exceeds 127.5: clamped.
    b = orc.q8_0_encode(_block([1e-4, -5e-5]))
    d = float(np.frombuffer(b[:2].tobytes(), np.float16)[0])
    assert d < 1e-4 / 127 * (127 / 127.5)
    assert b[2:].view(np.int8)[0] == 127


def test_decode_round_trip_bound():
    rng = np.random.default_rng(1)
    v = (rng.standard_normal(32 * 40) * rng.choice([1e-3, 1.0, 300.0], 32 * 40)).astype(np.float32)
    b = orc.q8_0_encode(v)
    w = orc.q8_0_decode(b, 4, 320)
    d = np.frombuffer(b.reshape(-1, 34)[:, :2].tobytes(), np.float16).astype(np.float64)
    err = np.abs(w.reshape(-1, 32) - v.reshape(-1, 32).astype(np.float64))
    assert np.all(err <= d[:, None] * 0.5 * (1 + 1e-3) + 1e-30)


def _loop_product(wm, x):
    out_dim, in_dim = wm.shape
    y = np.zeros((x.shape[0], out_dim))
    for b in range(x.shape[0]):
        for o in range(out_dim):
            s = 0.0
            for i in range(in_dim):
                s += float(wm[o, i]) * float(x[b, i])
            y[b, o] = s
    return y


@pytest.mark.parametrize("w_type", [orc.WTYPE_F32, orc.WTYPE_Q8_0])
def test_product_against_loops(w_type):
    rng = np.random.default_rng(2 + w_type)
    in_dim, out_dim, batch = 64, 5, 3
    w = rng.standard_normal((out_dim, in_dim)).astype(np.float32)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    if w_type == orc.WTYPE_F32:
        data, wm = w, w.astype(np.float64)
    else:
        data = orc.q8_0_encode(w)
        raw = data.reshape(out_dim, 2, 34)
        wm = np.empty((out_dim, in_dim))
        for o in range(out_dim):  # byte-by-byte parse of each block
            for blk in range(2):
                dd = struct.unpack("<e", raw[o, blk, :2].tobytes())[0]
                qs = struct.unpack("<32b", raw[o, blk, 2:].tobytes())
                wm[o, 32 * blk: 32 * blk + 32] = [dd * q for q in qs]
    assert np.allclose(orc.matmul_batch(w_type, data, x, in_dim, out_dim), _loop_product(wm, x), rtol=1e-12,
                       atol=1e-12)
