"""gsp_matmul_batch (QuantKernels.MatMulBatch, PagedTransformerRunner.cs:601-603,659) against the oracle.

y[b][o] = sum_i W[o][i] x[b][i] with F32 or Q8_0 weights.  Every weight is exact in the device's
arithmetic (fp32, or fp16 for Q8_0 values), x is kept to at least ~22 significant bits (fp32, or
a scaled fp16 pair on the Q8_0 fp16 path) and products are summed in fp32, so the bar is fp32
summation error: |y - y64| <= 1e-5 * sum_i |W[o][i] x[b][i]| + 1e-7, against the float64 oracle
on the same encoded weights.  The shapes
cover a single batch row, batches below, at and above one 64-row workgroup tile with ragged
ends, output counts that are not multiples of 16 (or of 4), one K range and several (split K).
"""
import numpy as np
import pytest

import glacier_oracle as orc

pytestmark = pytest.mark.gpu

SHAPES = [
    # (in_dim, out_dim, batch)
    (64, 16, 1),
    (128, 40, 5),
    (896, 1152, 8),
    (3584, 512, 64),
    (256, 96, 100),
    (4096, 48, 17),
    (512, 37, 3),  # out_dim odd: partial weight rows, and the reduce's one-element path
    # batch x out_dim >= 196608: Q8_0 takes the fp16 matrix-core path
    (256, 2048, 100),
    (512, 1600, 128),
    (128, 2049, 97),
    # batch <= 64 and batch x out_dim >= 16384: Q8_0 takes the small-batch fp16 kernel
    # (one, two and four M tiles, ragged batch tiles and weight-row tiles, 1 to 16 K ranges)
    (3584, 1040, 64),
    (1024, 4100, 17),
    (8192, 4160, 16),
    (192, 8192, 9),
    (640, 2050, 33),
]


def _weights(rng, w_type, out_dim, in_dim):
    w = (rng.standard_normal((out_dim, in_dim)) * rng.choice([0.02, 1.0, 30.0], (out_dim, 1))).astype(np.float32)
    if w_type == orc.WTYPE_F32:
        return w, w.astype(np.float64)
    data = orc.q8_0_encode(w)
    return data, orc.q8_0_decode(data, out_dim, in_dim)


def _run(torch, gsp, ctx, w_type, data, x, in_dim, out_dim, fill=np.nan):
    wd = torch.from_numpy(np.ascontiguousarray(data)).cuda()
    xd = torch.from_numpy(np.ascontiguousarray(x)).cuda()
    yd = torch.full((x.shape[0], out_dim), float(fill), device="cuda")
    torch.cuda.synchronize()
    ctx.matmul_batch(w_type, wd.data_ptr(), xd.data_ptr(), yd.data_ptr(), in_dim, out_dim, x.shape[0])
    ctx.sync()
    return yd.cpu().numpy()


@pytest.mark.parametrize("w_type", [orc.WTYPE_F32, orc.WTYPE_Q8_0], ids=["f32", "q8_0"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"in{s[0]}_out{s[1]}_b{s[2]}")
def test_matmul_matches_oracle(torch_mod, gsp, ctx, shape, w_type):
    in_dim, out_dim, batch = shape
    print(f"case matmul {shape} type={w_type}", flush=True)
    rng = np.random.default_rng(in_dim + out_dim + batch + w_type)
    data, wm = _weights(rng, w_type, out_dim, in_dim)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    got = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    ref = orc.matmul_batch(w_type, data, x, in_dim, out_dim)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wm).T
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-7)
    # Deterministic: the split-K partials are added in a fixed order.
    again = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    assert np.array_equal(got, again)


def test_matmul_errors_and_empty(torch_mod, gsp, ctx):
    torch = torch_mod
    w = torch.zeros((16, 96), device="cuda")
    x = torch.zeros((4, 128), device="cuda")
    y = torch.full((4, 16), 7.0, device="cuda")
    torch.cuda.synchronize()
    with pytest.raises(gsp.Unsupported):  # Q4_0 and the other GGUF types are not supported
        ctx.matmul_batch(2, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 16, 4)
    with pytest.raises(gsp.Unsupported):  # in_dim not a multiple of 64
        ctx.matmul_batch(gsp.WTYPE_F32, w.data_ptr(), x.data_ptr(), y.data_ptr(), 96, 16, 4)
    with pytest.raises(gsp.InvalidArgument):  # x not 16-byte aligned
        ctx.matmul_batch(gsp.WTYPE_F32, w.data_ptr(), x.data_ptr() + 4, y.data_ptr(), 64, 16, 2)
    with pytest.raises(gsp.InvalidArgument):
        ctx.matmul_batch(gsp.WTYPE_F32, 0, x.data_ptr(), y.data_ptr(), 64, 16, 4)
    ctx.matmul_batch(gsp.WTYPE_F32, w.data_ptr(), x.data_ptr(), y.data_ptr(), 64, 16, 0)  # batch 0: no work
    ctx.sync()
    assert torch.all(y == 7.0)


def test_matmul_q_projection_then_attention_shapes(torch_mod, gsp, ctx):
    """The Q projection of a Qwen2.5-7B layer (3584 -> 3584) for 64 decode rows, Q8_0 weights:
    the product the reference runs before RoPE and attention (PagedTransformerRunner.cs:601)."""
    rng = np.random.default_rng(11)
    in_dim = out_dim = 3584
    data, wm = _weights(rng, orc.WTYPE_Q8_0, out_dim, in_dim)
    x = rng.standard_normal((64, in_dim)).astype(np.float32)
    got = _run(torch_mod, gsp, ctx, orc.WTYPE_Q8_0, data, x, in_dim, out_dim)
    ref = x.astype(np.float64) @ wm.T
    mag = np.abs(x.astype(np.float64)) @ np.abs(wm).T
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-7)


@pytest.mark.parametrize("batch", [100, 60], ids=["b100", "b60"])
@pytest.mark.parametrize("w_type", [orc.WTYPE_F32, orc.WTYPE_Q8_0, orc.WTYPE_Q4_K, orc.WTYPE_Q6_K],
                         ids=["f32", "q8_0", "q4_k", "q6_k"])
def test_matmul_outlier_channels_and_large_rows(torch_mod, gsp, ctx, w_type, batch):
    """Rows with one channel 1e4 times the rest, rows near 1e30 and rows near 1e-30.  Q8_0 takes an
    fp16 path at both batches (the two-kernel form at 100 rows, the small-batch form at 60, with an
    exponent per K range of each row); Q4_K the two-kernel fp16 form at 100 rows and the small-batch
    form at 60; Q6_K the fp32 form at 100 rows and the small-batch form at 60.
    There x is a scaled fp16 pair whose error is bounded relative to its row's largest |x| (at most
    ~2^-22 of it per element), so the bar adds that term; every finite row stays finite.  The F32
    form keeps x in fp32 and meets the plain fp32 summation bar.  The Q4_K small form sums the
    quant term d1 q x and the min term m1 x separately (|d1 q| <= |w| + m1), so its bar is taken over
    |w| + 2 m1, with m1 the weights the oracle decodes when every quant is zero."""
    in_dim, out_dim = 4096, 2048
    rng = np.random.default_rng(77 + w_type + batch)
    if w_type == orc.WTYPE_Q4_K:
        data, wm = _kquant_weights(rng, w_type, out_dim, in_dim)
        zq = data.reshape(out_dim, in_dim // orc.QK_K, orc.Q4_K_BYTES).copy()
        zq[..., 16:] = 0
        m1 = -orc.q4_k_decode(zq.reshape(-1), out_dim, in_dim)
        assert np.all(m1 >= 0)
        wabs = np.abs(wm) + 2 * m1
    elif w_type == orc.WTYPE_Q6_K:
        data, wm = _kquant_weights(rng, w_type, out_dim, in_dim)
        wabs = np.abs(wm)
    else:
        data, wm = _weights(rng, w_type, out_dim, in_dim)
        wabs = np.abs(wm)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    x[0:30, rng.integers(0, in_dim, 30)] *= 1e4           # one outlier channel per row (some shared)
    x[30:40] *= np.float32(1e30)                          # near the top of the fp32 range
    x[40:50] *= np.float32(3e34)
    x[50:60] *= np.float32(1e-30)                         # tiny rows
    print(f"case matmul outliers type={w_type}", flush=True)
    got = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    ref = orc.matmul_batch(w_type, data, x, in_dim, out_dim)
    x64 = x.astype(np.float64)
    mag = np.abs(x64) @ wabs.T
    bar = 1e-5 * mag + 1e-7 * (np.abs(x64).max(axis=1, keepdims=True) > 1e-20)
    if w_type != orc.WTYPE_F32:
        bar = bar + 2.0 ** -21 * np.abs(x64).max(axis=1, keepdims=True) * wabs.sum(axis=1)[None, :]
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= bar)


# ---- K-quant weights (Q4_K, Q6_K: super-blocks of 256 weights) -------------------------------------
# Random super-blocks are valid encodings: every byte pattern decodes to finite weights once the
# fp16 scales are finite, so the quants, 6-bit scales/mins and high bits are random bytes and only
# d (and dmin) are set.  The fp32 form decodes each weight to the float32 value the oracle's decoder
# gives (pinned by closed forms in tests/test_matmul_oracle.py), so the bar is fp32 summation error;
# the fp16 forms (Q4_K and Q6_K at most 64 rows, Q4_K above with enough outputs) keep the quants
# exact in fp16 and x to ~22 bits as the Q8_0 ones do, within the same bar.

KQ_SHAPES = [
    (256, 16, 1),
    (512, 40, 5),
    (3584, 512, 64),   # Qwen2.5-7B hidden size: 14 super-blocks per row
    (4096, 48, 17),
    (256, 96, 100),
    (512, 37, 3),
    (1024, 4100, 17),
    (3584, 3584, 64),  # the Q projection of a Qwen2.5-7B layer for 64 decode rows
    # the K-quants' small-batch forms (batch <= 64, batch x out_dim >= 16384): one M tile with K ranges of
    # three chunks that start inside a super-block, four M tiles with a ragged batch and a ragged
    # last weight-row tile, one M tile over sixteen K ranges
    (768, 8192, 9),
    (2048, 2100, 40),
    (8192, 4160, 16),
    # more than 64 rows and at least 196608 outputs: Q4_K takes the large fp16 form (x as scaled
    # fp16 pairs per row, block sums for the min term): two batch tiles with a ragged second one,
    # one row in the second tile with a ragged weight-row tile, and four full batch tiles
    (2048, 2048, 100),
    (512, 4100, 65),
    (3584, 3584, 256),
    (18944, 1024, 200),  # rows longer than the pre-pass keeps in registers (Qwen2.5-7B's down projection)
]


def _kquant_weights(rng, w_type, out_dim, in_dim):
    nb = in_dim // orc.QK_K
    if w_type == orc.WTYPE_Q4_K:
        b = rng.integers(0, 256, (out_dim, nb, orc.Q4_K_BYTES), dtype=np.uint8)
        b[..., 0:2] = np.ascontiguousarray((rng.uniform(1e-4, 2e-2, (out_dim, nb, 1))).astype(np.float16)).view(np.uint8)
        b[..., 2:4] = np.ascontiguousarray((rng.uniform(1e-4, 2e-2, (out_dim, nb, 1))).astype(np.float16)).view(np.uint8)
        data = b.reshape(-1)
        return data, orc.q4_k_decode(data, out_dim, in_dim)
    b = rng.integers(0, 256, (out_dim, nb, orc.Q6_K_BYTES), dtype=np.uint8)
    b[..., 208:210] = np.ascontiguousarray((rng.uniform(1e-5, 1e-3, (out_dim, nb, 1))).astype(np.float16)).view(np.uint8)
    data = b.reshape(-1)
    return data, orc.q6_k_decode(data, out_dim, in_dim)


@pytest.mark.parametrize("w_type", [orc.WTYPE_Q4_K, orc.WTYPE_Q6_K], ids=["q4_k", "q6_k"])
@pytest.mark.parametrize("shape", KQ_SHAPES, ids=lambda s: f"in{s[0]}_out{s[1]}_b{s[2]}")
def test_kquant_matmul_matches_oracle(torch_mod, gsp, ctx, shape, w_type):
    in_dim, out_dim, batch = shape
    print(f"case matmul {shape} type={w_type}", flush=True)
    rng = np.random.default_rng(in_dim * 3 + out_dim + batch + w_type)
    data, wm = _kquant_weights(rng, w_type, out_dim, in_dim)
    assert np.all(np.isfinite(wm))
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    got = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    ref = orc.matmul_batch(w_type, data, x, in_dim, out_dim)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wm).T
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-7)
    again = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    assert np.array_equal(got, again)


# Long K and wide outputs on the small-batch form.  When the merge holds too few K ranges for
# ranges of 8 chunks (more than 8 ranges at 33..64 rows, 16 at 17..32, 32 at up to 16), each
# workgroup walks its range in passes of 8 chunks through the same LDS, and the pre-pass takes up to
# four f4 per thread.  Wide outputs run several rounds of workgroups, and from 1024 weight-row tiles
# on 256 CUs with no K split.  The splits below are the library's for a 256-CU device; other CU
# counts give other splits of the same shapes.
LONG_SHAPES = [
    (5120, 1040, 64),   # 8 ranges of 10 chunks: a full pass, then a 2-chunk one; one f4 per pre-pass thread
    (18944, 1040, 64),  # Qwen2.5-7B's FFN down-projection width: 8 ranges of 37 chunks, 5 passes
    (18944, 4100, 17),  # two M tiles, a ragged last weight-row tile
    (6656, 6400, 40),   # 5 ranges of 21 chunks, the last of 20; a ragged batch tile
    (3584, 18944, 64),  # Qwen2.5-7B's gate/up projection: 7 ranges of 296 tiles
    (4096, 16384, 24),  # two M tiles: 8 ranges of 256 tiles
    (512, 65536, 1),    # one range of 1024 tiles, y stored directly
    (1024, 65536, 2),   # 1024 tiles fill the CU slots twice: one range per tile in two passes, no merge
]


@pytest.mark.parametrize("w_type", [orc.WTYPE_Q8_0, orc.WTYPE_Q4_K, orc.WTYPE_Q6_K], ids=["q8_0", "q4_k", "q6_k"])
@pytest.mark.parametrize("shape", LONG_SHAPES, ids=lambda s: f"in{s[0]}_out{s[1]}_b{s[2]}")
def test_small_batch_long_ranges_and_wide_outputs_match_oracle(torch_mod, gsp, ctx, shape, w_type):
    in_dim, out_dim, batch = shape
    print(f"case matmul long {shape} type={w_type}", flush=True)
    rng = np.random.default_rng(in_dim * 5 + out_dim + batch + w_type)
    if w_type in (orc.WTYPE_Q4_K, orc.WTYPE_Q6_K):
        data, wm = _kquant_weights(rng, w_type, out_dim, in_dim)
    else:
        data, wm = _weights(rng, w_type, out_dim, in_dim)
    x = rng.standard_normal((batch, in_dim)).astype(np.float32)
    got = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    ref = orc.matmul_batch(w_type, data, x, in_dim, out_dim)
    mag = np.abs(x.astype(np.float64)) @ np.abs(wm).T
    assert np.all(np.isfinite(got))
    assert np.all(np.abs(got - ref) <= 1e-5 * mag + 1e-7)
    again = _run(torch_mod, gsp, ctx, w_type, data, x, in_dim, out_dim)
    assert np.array_equal(got, again)


def test_kquant_matmul_errors(torch_mod, gsp, ctx):
    torch = torch_mod
    w = torch.zeros(4096, device="cuda")
    x = torch.zeros((4, 512), device="cuda")
    y = torch.zeros((4, 16), device="cuda")
    torch.cuda.synchronize()
    for wt in (gsp.WTYPE_Q4_K, gsp.WTYPE_Q6_K):
        with pytest.raises(gsp.Unsupported):  # in_dim not a multiple of a 256-weight super-block
            ctx.matmul_batch(wt, w.data_ptr(), x.data_ptr(), y.data_ptr(), 128, 16, 4)
    with pytest.raises(gsp.InvalidArgument):  # Q4_K super-blocks are read as 4-byte words
        ctx.matmul_batch(gsp.WTYPE_Q4_K, w.data_ptr() + 2, x.data_ptr(), y.data_ptr(), 256, 16, 4)
    with pytest.raises(gsp.InvalidArgument):  # Q6_K as 2-byte words
        ctx.matmul_batch(gsp.WTYPE_Q6_K, w.data_ptr() + 1, x.data_ptr(), y.data_ptr(), 256, 16, 4)
