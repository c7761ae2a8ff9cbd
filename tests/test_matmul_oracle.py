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


# ---- K-quant super-blocks (GGUF Q4_K = 12, Q6_K = 14) ----------------------------------------------
# Blocks are built here field by field from the public GGML layout, written per weight index
# (which byte and which bits hold weight i), the opposite direction of the oracle's decoders.
# Values are chosen so that every product is exact in float32: the decode must equal the closed
# form bit for bit.

def _q4_k_block(d, dmin, sc, mn, q):
    """144 bytes: fp16 d, fp16 dmin, 12 bytes of 6-bit scales/mins, 128 bytes of nibbles."""
    s = [0] * 12
    for j in range(8):
        if j < 4:
            s[j] |= sc[j] & 63
            s[j + 4] |= mn[j] & 63
        else:
            s[j + 4] |= (sc[j] & 0xF) | ((mn[j] & 0xF) << 4)
            s[j - 4] |= (sc[j] >> 4) << 6
            s[j] |= (mn[j] >> 4) << 6
    qs = [0] * 128
    for i in range(256):
        j = i // 32                       # sub-block
        byte = 32 * (j // 2) + i % 32     # sub-blocks 2p and 2p + 1 share quant bytes 32p ..
        qs[byte] |= (q[i] & 0xF) << (4 * (j % 2))
    return (np.float16(d).tobytes() + np.float16(dmin).tobytes() + bytes(s) + bytes(qs))


def _q6_k_block(d, scales, q):
    """210 bytes: 128 low-nibble bytes, 64 high-bit bytes, 16 int8 scales, fp16 d."""
    ql = [0] * 128
    qh = [0] * 64
    for i in range(256):
        n, r = divmod(i, 128)
        c, l = divmod(r, 32)
        ql[64 * n + 32 * (c % 2) + l] |= (q[i] & 0xF) << (4 * (c // 2))
        qh[32 * n + l] |= ((q[i] >> 4) & 3) << (2 * c)
    return bytes(ql) + bytes(qh) + np.array(scales, np.int8).tobytes() + np.float16(d).tobytes()


def _q6_k_scale_index(i):
    n, r = divmod(i, 128)
    c, l = divmod(r, 32)
    return 8 * n + l // 16 + 2 * c


def test_q4_k_closed_form():
    sc = [1, 63, 17, 48, 33, 62, 5, 40]   # high bits set in every j >= 4 packing position
    mn = [0, 63, 31, 32, 50, 1, 62, 21]
    q = [(7 * i + 3) % 16 for i in range(256)]  # every nibble value in every position class
    blk = np.frombuffer(_q4_k_block(0.5, 0.25, sc, mn, q), np.uint8)
    assert blk.size == orc.Q4_K_BYTES
    got = orc.q4_k_decode(blk, 1, 256)[0]
    want = np.array([0.5 * sc[i // 32] * q[i] - 0.25 * mn[i // 32] for i in range(256)])
    assert np.array_equal(got, want)
    assert got[0] == 1.5 and got[32] == 0.5 * 63 * q[32] - 0.25 * 63 and got[255] == 0.5 * 40 * q[255] - 0.25 * 21
    sc_got, mn_got = orc.q4_k_scale_min(blk[4:16])
    assert list(sc_got) == sc and list(mn_got) == mn


def test_q6_k_closed_form():
    scales = [-128, 127, -1, 1, 64, -64, 3, -3, 100, -100, 7, -7, 0, 31, -32, 90]
    q = [(11 * i + 5) % 64 for i in range(256)]  # every 6-bit value: q - 32 covers [-32, 31]
    blk = np.frombuffer(_q6_k_block(0.125, scales, q), np.uint8)
    assert blk.size == orc.Q6_K_BYTES
    got = orc.q6_k_decode(blk, 1, 256)[0]
    want = np.array([0.125 * scales[_q6_k_scale_index(i)] * (q[i] - 32) for i in range(256)])
    assert np.array_equal(got, want)
    assert got[0] == 0.125 * -128 * (5 - 32)
    assert _q6_k_scale_index(255) == 15 and got[255] == 0.125 * 90 * (q[255] - 32)


def test_k_quant_rows_and_blocks_in_order():
    """Rows of several super-blocks: block k of row o holds weights 256 k .. 256 k + 255 of row o."""
    rng = np.random.default_rng(7)
    rows, nb = 3, 4
    b4, b6, w4, w6 = [], [], [], []
    for o in range(rows):
        for k in range(nb):
            d, dmin = float(2.0 ** rng.integers(-4, 2)), float(2.0 ** rng.integers(-6, 0))
            sc, mn = rng.integers(0, 64, 8), rng.integers(0, 64, 8)
            q4 = rng.integers(0, 16, 256)
            b4.append(_q4_k_block(d, dmin, sc, mn, q4))
            w4.append([d * sc[i // 32] * q4[i] - dmin * mn[i // 32] for i in range(256)])
            s6 = rng.integers(-128, 128, 16)
            q6 = rng.integers(0, 64, 256)
            b6.append(_q6_k_block(d, s6, q6))
            w6.append([d * s6[_q6_k_scale_index(i)] * (q6[i] - 32) for i in range(256)])
    got4 = orc.q4_k_decode(np.frombuffer(b"".join(b4), np.uint8), rows, 256 * nb)
    got6 = orc.q6_k_decode(np.frombuffer(b"".join(b6), np.uint8), rows, 256 * nb)
    assert np.array_equal(got4, np.array(w4).reshape(rows, 256 * nb))
    assert np.array_equal(got6, np.array(w6).reshape(rows, 256 * nb))


def test_k_quant_product_is_the_definition():
    rng = np.random.default_rng(8)
    rows, nb, batch = 5, 2, 3
    blocks = [_q4_k_block(0.25, 0.5, rng.integers(0, 64, 8), rng.integers(0, 64, 8), rng.integers(0, 16, 256))
              for _ in range(rows * nb)]
    w = np.frombuffer(b"".join(blocks), np.uint8)
    x = rng.standard_normal((batch, 256 * nb)).astype(np.float32)
    y = orc.matmul_batch(orc.WTYPE_Q4_K, w, x, 256 * nb, rows)
    assert np.allclose(y, _loop_product(orc.q4_k_decode(w, rows, 256 * nb), x), rtol=0, atol=1e-9)
