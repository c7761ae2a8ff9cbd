"""ctypes wrapper of liboracle.so — TEST INFRASTRUCTURE ONLY.

The oracle is the CPU restatement of the reference's paged-attention path
(PagedAttentionKernel.cs:17-372, PagedBlockPool.cs, BlockTable.cs), plus the
Q8_0 weight encoding and the product of the projection GEMMs around it.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it, as
the checker or the timed CPU baseline; the product never does.
"""
from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path
from typing import Optional

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

ORC_OK, ORC_E_RANGE, ORC_E_UNSUPPORTED = 0, 1, 2
ISA_AUTO, ISA_SCALAR, ISA_AVX2, ISA_AVX512 = -1, 0, 1, 2

i32 = ctypes.c_int32
i32p = ctypes.POINTER(i32)
f32p = ctypes.POINTER(ctypes.c_float)
f64p = ctypes.POINTER(ctypes.c_double)
vp = ctypes.c_void_p


class OrcPool(ctypes.Structure):
    _fields_ = [
        ("k", f32p),
        ("v", f32p),
        ("total_blocks", i32),
        ("layers", i32),
        ("heads_kv", i32),
        ("head_dim", i32),
        ("v_head_dim", i32),
        ("block_size", i32),
    ]


class OrcTable(ctypes.Structure):
    _fields_ = [("ids", i32p), ("n_ids", i32), ("token_count", i32)]


class ArgumentOutOfRange(ValueError):
    """Where the reference throws ArgumentOutOfRangeException."""


_lib = None


def build() -> Path:
    subprocess.run(["make", "-B", "-C", str(HERE)], check=True, capture_output=True, text=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    sig = {
        "orc_host_isa": (ctypes.c_int, []),
        "orc_compute_attention": (
            ctypes.c_int,
            [ctypes.POINTER(OrcPool), ctypes.POINTER(OrcTable), i32, i32, i32, f32p, f32p, i32, i32, i32, i32,
             ctypes.c_float, f32p, i32, f32p, i32, i32],
        ),
        "orc_attention_step": (
            ctypes.c_int,
            [ctypes.POINTER(OrcPool), i32, i32, i32p, i32p, i32p, i32p, i32p, f32p, f32p, i32, ctypes.c_float, i32,
             i32, i32],
        ),
        "orc_attention_fp64": (
            ctypes.c_int,
            [ctypes.POINTER(OrcPool), ctypes.POINTER(OrcTable), i32, i32, f32p, f64p, i32, ctypes.c_double, i32],
        ),
        "orc_alloc_create": (vp, [i32, i32]),
        "orc_alloc_destroy": (None, [vp]),
        "orc_alloc_try_allocate": (ctypes.c_int, [vp, i32p]),
        "orc_alloc_retain": (ctypes.c_int, [vp, i32]),
        "orc_alloc_release": (ctypes.c_int, [vp, i32]),
        "orc_alloc_ref_count": (ctypes.c_int, [vp, i32]),
        "orc_alloc_free_count": (ctypes.c_int, [vp]),
        "orc_alloc_find_prefix": (ctypes.c_int, [vp, ctypes.c_uint64, ctypes.POINTER(i32)]),
        "orc_alloc_bind_prefix": (ctypes.c_int, [vp, ctypes.c_uint64, i32]),
        "orc_rope": (None, [f32p, i32, i32, i32, ctypes.c_double, i32]),
        "orc_rope_ex": (None, [f32p, i32, i32, i32, ctypes.c_double, i32, i32, f32p, f32p, ctypes.c_double]),
        "orc_btab_create": (vp, [vp]),
        "orc_btab_destroy": (None, [vp]),
        "orc_btab_attach_prefix": (None, [vp, i32p, i32, i32]),
        "orc_btab_append_token": (ctypes.c_int, [vp, i32p, i32p]),
        "orc_btab_append_tokens": (ctypes.c_int, [vp, i32]),
        "orc_btab_token_count": (ctypes.c_int, [vp]),
        "orc_btab_ids": (ctypes.c_int, [vp, i32p, i32]),
        "orc_btab_release_all": (None, [vp]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def host_isa() -> int:
    return load().orc_host_isa()


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


ROPE_PAIRS, ROPE_HALVES = 0, 1


def rope(x: np.ndarray, pos: int, freq_base: float, style: int = ROPE_PAIRS) -> np.ndarray:
    """Rotary embedding of the vectors along x's last axis at position `pos` (a rotated copy);
    textbook definition in fp64 (orc_rope)."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    dim = y.shape[-1]
    load().orc_rope(y.ctypes.data_as(f32p), y.size // dim, dim, int(pos), float(freq_base), int(style))
    return y


def rope_ex(x: np.ndarray, pos: int, freq_base: float, style: int = ROPE_PAIRS, rope_dim: int = 0,
            inv_freq=None, freq_factors=None, mscale: float = 1.0) -> np.ndarray:
    """QuantKernels.RoPE with ropeDim, invFreqTable, ropeFreqs and mscale (orc_rope_ex): only the
    first rope_dim dims rotate (0: all), pair j by pos * inv_freq[j] (or freq_base^(-2j/rope_dim))
    divided by freq_factors[j], scaled by mscale; a rotated copy of x."""
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    dim = y.shape[-1]
    rd = int(rope_dim) or dim
    tabs = [None if t is None else _f32(t) for t in (inv_freq, freq_factors)]
    for t in tabs:
        if t is not None and t.size != rd // 2:
            raise ValueError(f"tables hold rope_dim / 2 = {rd // 2} entries (got {t.size})")
    ptrs = [None if t is None else t.ctypes.data_as(f32p) for t in tabs]
    load().orc_rope_ex(y.ctypes.data_as(f32p), y.size // dim, dim, int(pos), float(freq_base), int(style), rd,
                       ptrs[0], ptrs[1], float(mscale))
    return y


def yarn_inv_freq(rope_dim: int, freq_base: float, factor: float, orig_ctx: int, beta_fast: float = 32.0,
                  beta_slow: float = 1.0) -> np.ndarray:
    """A YaRN inverse-frequency table (Peng et al., 2023, "YaRN: Efficient Context Window Extension
    of Large Language Models", NTK-by-parts): pair j's base rate theta_j = base^(-2j/d) completes
    r_j = orig_ctx * theta_j / (2 pi) turns over the original context; rates with r_j above
    beta_fast keep theta_j, below beta_slow become theta_j / factor, and a linear ramp in r_j joins
    them.  Used to make realistic tables for tests: the product takes any table as given, and how
    the reference's closed QuantKernels.PrecomputeYarnFrequencies (PagedTransformerRunner.cs:91-96)
    forms its table is unpinned."""
    j = np.arange(rope_dim // 2, dtype=np.float64)
    theta = float(freq_base) ** (-2.0 * j / rope_dim)
    turns = orig_ctx * theta / (2.0 * np.pi)
    keep = np.clip((turns - beta_slow) / (beta_fast - beta_slow), 0.0, 1.0)
    return (keep * theta + (1.0 - keep) * theta / factor).astype(np.float32)


def yarn_mscale(factor: float) -> float:
    """YaRN's attention factor 0.1 ln(s) + 1 for a context scale s > 1 (1 otherwise), from the same
    paper; a test input, like yarn_inv_freq."""
    return 1.0 if factor <= 1.0 else 0.1 * float(np.log(factor)) + 1.0


# Projection GEMM weights (QuantKernels.MatMulBatch, PagedTransformerRunner.cs:601-603,659).
WTYPE_F32, WTYPE_Q8_0 = 0, 8  # GGUF tensor type ids
Q8_0_BLOCK, Q8_0_BYTES = 32, 34


def q8_0_encode(values) -> np.ndarray:
    """Q8_0 bytes of a float32 array whose length is a multiple of 32, as the reference's test
    builder writes them (PhaseCServeRemediationTests.cs:1587-1622).  Per block of 32 values:
    d = (Half)(maxAbs / 127f) (round to nearest even), invD = 1f / d in float32 (0 when d is 0),
    q = MathF.Round(v * invD) (to nearest even) clamped to [-127, 127]; stored as d's two bytes
    (little-endian) followed by the 32 int8."""
    v = np.ascontiguousarray(values, dtype=np.float32).reshape(-1, Q8_0_BLOCK)
    d16 = (np.abs(v).max(axis=1) / np.float32(127.0)).astype(np.float16)
    d = d16.astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d > 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    q = np.clip(np.rint(v * inv[:, None]), -127, 127).astype(np.int8)
    out = np.empty((v.shape[0], Q8_0_BYTES), np.uint8)
    out[:, :2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.reshape(-1)


def q8_0_decode(data, rows: int, cols: int) -> np.ndarray:
    """Dequantised float64 [rows, cols] of Q8_0 rows (each row cols / 32 blocks): d * q."""
    b = np.ascontiguousarray(data, dtype=np.uint8).reshape(rows, cols // Q8_0_BLOCK, Q8_0_BYTES)
    d = np.ascontiguousarray(b[:, :, :2]).view(np.float16)[..., 0].astype(np.float64)
    q = np.ascontiguousarray(b[:, :, 2:]).view(np.int8).astype(np.float64)
    return (q * d[..., None]).reshape(rows, cols)


# K-quant super-blocks of 256 weights (the GGUF tensor types Q4_K = 12 and Q6_K = 14), decoded as
# the public GGML block layout defines them (block_q4_K / block_q6_K and their dequantisation in
# ggml-quants.c).  The reference runner batches its GEMMs on these types
# (CudaPagedTransformerRunner.cs:470-473) through closed code, so only the layout's arithmetic is
# restated, in float32 in the layout's own order (the weights a dequantising runner would see).
WTYPE_Q4_K, WTYPE_Q6_K = 12, 14
QK_K = 256
Q4_K_BYTES, Q6_K_BYTES = 144, 210


def q4_k_scale_min(scales: np.ndarray):
    """The eight 6-bit (scale, min) pairs of Q4_K super-blocks from their 12 packed bytes
    ([..., 12] uint8 -> two [..., 8] int arrays): sub-block j < 4 keeps its scale in the low 6 bits of
    byte j and its min in those of byte j + 4; j >= 4 keeps the low 4 bits of each in byte j + 4
    (scale low nibble, min high nibble) and the top 2 bits in bits 6-7 of byte j - 4 (scale) and
    byte j (min)."""
    s = scales.astype(np.int32)
    sc = np.empty(s.shape[:-1] + (8,), np.int32)
    mn = np.empty_like(sc)
    sc[..., :4] = s[..., 0:4] & 63
    mn[..., :4] = s[..., 4:8] & 63
    sc[..., 4:] = (s[..., 8:12] & 0xF) | ((s[..., 0:4] >> 6) << 4)
    mn[..., 4:] = (s[..., 8:12] >> 4) | ((s[..., 4:8] >> 6) << 4)
    return sc, mn


def q4_k_decode(data, rows: int, cols: int) -> np.ndarray:
    """Q4_K rows (cols / 256 super-blocks of 144 bytes each: fp16 d, fp16 dmin, 12 bytes of 6-bit
    scales and mins, 128 bytes of 4-bit quants) as float64 [rows, cols].  Weights 64 p .. 64 p + 31
    are the low nibbles of quant bytes 32 p .. 32 p + 31 and weights 64 p + 32 .. 64 p + 63 their high
    nibbles (sub-blocks 2 p and 2 p + 1); weight i of sub-block j is d * sc_j * q_i - dmin * m_j, with
    d * sc_j and dmin * m_j formed in float32 (exact) and one rounding in the difference."""
    b = np.ascontiguousarray(data, dtype=np.uint8).reshape(rows, cols // QK_K, Q4_K_BYTES)
    d = np.ascontiguousarray(b[..., 0:2]).view(np.float16)[..., 0].astype(np.float32)
    dmin = np.ascontiguousarray(b[..., 2:4]).view(np.float16)[..., 0].astype(np.float32)
    sc, mn = q4_k_scale_min(b[..., 4:16])
    qs = b[..., 16:144].astype(np.int32)
    q = np.empty(b.shape[:2] + (QK_K,), np.float32)
    for p in range(4):
        q[..., 64 * p:64 * p + 32] = qs[..., 32 * p:32 * p + 32] & 0xF
        q[..., 64 * p + 32:64 * p + 64] = qs[..., 32 * p:32 * p + 32] >> 4
    d1 = np.repeat(d[..., None] * sc.astype(np.float32), 32, axis=-1)
    m1 = np.repeat(dmin[..., None] * mn.astype(np.float32), 32, axis=-1)
    w = d1 * q - m1  # float32: d1 * q is exact, the difference rounds once
    return w.reshape(rows, cols).astype(np.float64)


def q6_k_decode(data, rows: int, cols: int) -> np.ndarray:
    """Q6_K rows (cols / 256 super-blocks of 210 bytes each: 128 bytes of the quants' low 4 bits,
    64 bytes of their high 2 bits, 16 int8 scales, fp16 d) as float64 [rows, cols].  Half n (weights
    128 n ..) reads low bytes 64 n .., high bytes 32 n .. and scales 8 n ..; its quarter c (weights
    128 n + 32 c + l, l < 32) takes the low (c = 0, 1) or high (c = 2, 3) nibble of low byte
    64 n + 32 (c % 2) + l, bits 2 c .. 2 c + 1 of high byte 32 n + l and scale 8 n + l / 16 + 2 c;
    the quant is those six bits minus 32, the weight (d * scale) * q in float32."""
    b = np.ascontiguousarray(data, dtype=np.uint8).reshape(rows, cols // QK_K, Q6_K_BYTES)
    ql = b[..., 0:128].astype(np.int32)
    qh = b[..., 128:192].astype(np.int32)
    scl = np.ascontiguousarray(b[..., 192:208]).view(np.int8).astype(np.float32)
    d = np.ascontiguousarray(b[..., 208:210]).view(np.float16)[..., 0].astype(np.float32)
    w = np.empty(b.shape[:2] + (QK_K,), np.float32)
    for n in range(2):
        lo = ql[..., 64 * n:64 * n + 64]
        hi = qh[..., 32 * n:32 * n + 32]
        for c in range(4):
            nib = (lo[..., 32 * (c % 2):32 * (c % 2) + 32] >> (4 * (c // 2))) & 0xF
            q = (nib | (((hi >> (2 * c)) & 3) << 4)) - 32
            scale = np.repeat(scl[..., 8 * n + 2 * c:8 * n + 2 * c + 2], 16, axis=-1)
            w[..., 128 * n + 32 * c:128 * n + 32 * c + 32] = (d[..., None] * scale) * q.astype(np.float32)
    return w.reshape(rows, cols).astype(np.float64)


def matmul_batch(w_type: int, w, x, in_dim: int, out_dim: int) -> np.ndarray:
    """y[b][o] = sum_i W[o][i] * x[b][i] in float64: the product MatMulBatch computes (its own
    arithmetic is closed code, so only this definition is restated).  W holds out_dim rows of in_dim
    weights, the GGUF [in, out] layout; x is [batch, in_dim]."""
    if w_type == WTYPE_F32:
        wm = np.asarray(w, dtype=np.float32).reshape(out_dim, in_dim).astype(np.float64)
    elif w_type == WTYPE_Q8_0:
        wm = q8_0_decode(w, out_dim, in_dim)
    elif w_type == WTYPE_Q4_K:
        wm = q4_k_decode(w, out_dim, in_dim)
    elif w_type == WTYPE_Q6_K:
        wm = q6_k_decode(w, out_dim, in_dim)
    else:
        raise ValueError(f"weight type {w_type} is not restated")
    xm = np.asarray(x, dtype=np.float32).reshape(-1, in_dim).astype(np.float64)
    return xm @ wm.T


class HostPool:
    """fp32 K/V arenas in the reference layout [block][layer][hkv][slot][dim]."""

    def __init__(self, k: np.ndarray, v: np.ndarray, block_size: int = 16):
        assert k.ndim == 5 and v.ndim == 5, "arenas are [blocks, layers, heads_kv, block_size, dim]"
        self.k = _f32(k)
        self.v = _f32(v)
        tb, layers, hkv, bs, d = self.k.shape
        assert bs == block_size and self.v.shape[:4] == self.k.shape[:4]
        self.struct = OrcPool(
            self.k.ctypes.data_as(f32p), self.v.ctypes.data_as(f32p), tb, layers, hkv, d, self.v.shape[4], bs
        )

    @property
    def heads_kv(self):
        return self.struct.heads_kv

    @property
    def head_dim(self):
        return self.struct.head_dim

    @property
    def v_head_dim(self):
        return self.struct.v_head_dim


def compute_attention(pool: HostPool, ids, token_count: int, layer: int, pos: int, q: np.ndarray, n_heads: int,
                      attn_scale: float, max_seq_len: int, out: Optional[np.ndarray] = None, n_threads: int = 1,
                      isa: int = ISA_AUTO, n_heads_kv: Optional[int] = None, head_dim: Optional[int] = None,
                      v_head_dim: Optional[int] = None, sink_logit: Optional[float] = None) -> np.ndarray:
    """ComputeAttention for one query token; `out` is left untouched when total == 0."""
    q = _f32(q).reshape(-1)
    if out is None:
        out = np.zeros(n_heads * pool.v_head_dim, np.float32)
    arr = _i32(ids)
    n = len(arr)
    if n == 0:
        arr = np.zeros(1, np.int32)
    tab = OrcTable(arr.ctypes.data_as(i32p), n, int(token_count))
    sink = ctypes.pointer(ctypes.c_float(sink_logit)) if sink_logit is not None else None
    rc = load().orc_compute_attention(
        ctypes.byref(pool.struct), ctypes.byref(tab), layer, layer, pos, q.ctypes.data_as(f32p),
        out.ctypes.data_as(f32p), n_heads, n_heads_kv if n_heads_kv is not None else pool.heads_kv,
        head_dim if head_dim is not None else pool.head_dim, v_head_dim if v_head_dim is not None else pool.v_head_dim,
        attn_scale, None, max_seq_len, sink, n_threads, isa)
    if rc == ORC_E_RANGE:
        raise ArgumentOutOfRange("ComputeAttention argument out of range")
    if rc == ORC_E_UNSUPPORTED:
        raise NotImplementedError("attention sinks are not restated")
    return out


def attention_step(pool: HostPool, layer: int, positions, token_counts, bt_offsets, bt_ids, q: np.ndarray,
                   n_heads: int, attn_scale: float, max_seq_len: int, q_lens=None, out: Optional[np.ndarray] = None,
                   n_threads: int = 1, isa: int = ISA_AUTO) -> np.ndarray:
    pos = _i32(positions)
    tc = _i32(token_counts)
    off = _i32(bt_offsets)
    ids = _i32(bt_ids) if len(bt_ids) else np.zeros(1, np.int32)
    ql = _i32(q_lens) if q_lens is not None else None
    total_q = int(ql.sum()) if ql is not None else len(pos)
    q = _f32(q)
    if out is None:
        out = np.zeros((total_q, n_heads, pool.v_head_dim), np.float32)
    rc = load().orc_attention_step(
        ctypes.byref(pool.struct), layer, len(pos), pos.ctypes.data_as(i32p),
        ql.ctypes.data_as(i32p) if ql is not None else None, tc.ctypes.data_as(i32p), off.ctypes.data_as(i32p),
        ids.ctypes.data_as(i32p), q.ctypes.data_as(f32p), out.ctypes.data_as(f32p), n_heads, attn_scale,
        max_seq_len, n_threads, isa)
    if rc == ORC_E_RANGE:
        raise ArgumentOutOfRange("attention step argument out of range")
    if rc != ORC_OK:
        raise RuntimeError(f"oracle status {rc}")
    return out


def attention_fp64(pool: HostPool, ids, token_count: int, layer: int, pos: int, q: np.ndarray, n_heads: int,
                   attn_scale: float, max_seq_len: int) -> np.ndarray:
    q = _f32(q).reshape(-1)
    out = np.zeros(n_heads * pool.v_head_dim, np.float64)
    arr = _i32(ids)
    n = len(arr)
    if n == 0:
        arr = np.zeros(1, np.int32)
    tab = OrcTable(arr.ctypes.data_as(i32p), n, int(token_count))
    rc = load().orc_attention_fp64(ctypes.byref(pool.struct), ctypes.byref(tab), layer, pos, q.ctypes.data_as(f32p),
                                   out.ctypes.data_as(f64p), n_heads, attn_scale, max_seq_len)
    if rc != ORC_OK:
        raise ArgumentOutOfRange("fp64 attention argument out of range")
    return out


class Alloc:
    """Free stack + refcounts restated from PagedBlockPool.cs:112-121,178-299."""

    def __init__(self, total_blocks: int, block_size: int = 16):
        self._h = load().orc_alloc_create(total_blocks, block_size)
        if not self._h:
            raise ArgumentOutOfRange("totalBlocks and blockSize must be >= 1")

    def __del__(self):
        if getattr(self, "_h", None):
            load().orc_alloc_destroy(self._h)
            self._h = None

    def try_allocate_block(self):
        b = i32()
        ok = load().orc_alloc_try_allocate(self._h, ctypes.byref(b))
        return bool(ok), b.value

    def retain_block(self, bid: int) -> int:
        r = load().orc_alloc_retain(self._h, bid)
        if r < 0:
            raise ArgumentOutOfRange("physicalBlockId")
        return r

    def release_block(self, bid: int) -> int:
        return load().orc_alloc_release(self._h, bid)

    def get_ref_count(self, bid: int) -> int:
        return load().orc_alloc_ref_count(self._h, bid)

    @property
    def free_blocks_count(self) -> int:
        return load().orc_alloc_free_count(self._h)

    def try_find_prefix_block(self, prefix_hash: int):
        b = i32()
        ok = load().orc_alloc_find_prefix(self._h, prefix_hash, ctypes.byref(b))
        return bool(ok), b.value

    def bind_prefix_block(self, prefix_hash: int, bid: int) -> None:
        if load().orc_alloc_bind_prefix(self._h, prefix_hash, bid) < 0:
            raise ArgumentOutOfRange("physicalBlockId or prefixHash")


class BTab:
    """BlockTable restated from BlockTable.cs:13-117 (metadata only)."""

    def __init__(self, alloc: Alloc):
        self._alloc = alloc
        self._h = load().orc_btab_create(alloc._h)

    def __del__(self):
        if getattr(self, "_h", None):
            load().orc_btab_destroy(self._h)
            self._h = None

    def attach_prefix_blocks(self, ids, token_count: int) -> None:
        a = _i32(ids) if len(ids) else np.zeros(1, np.int32)
        load().orc_btab_attach_prefix(self._h, a.ctypes.data_as(i32p), len(ids), token_count)

    def append_token(self):
        b, o = i32(), i32()
        ok = load().orc_btab_append_token(self._h, ctypes.byref(b), ctypes.byref(o))
        return bool(ok), b.value, o.value

    def append_tokens(self, n: int) -> int:
        return load().orc_btab_append_tokens(self._h, n)

    @property
    def token_count(self) -> int:
        return load().orc_btab_token_count(self._h)

    def as_span(self) -> np.ndarray:
        n = load().orc_btab_ids(self._h, None, 0)
        out = np.zeros(max(1, n), np.int32)
        load().orc_btab_ids(self._h, out.ctypes.data_as(i32p), n)
        return out[:n]

    def release_all(self) -> None:
        load().orc_btab_release_all(self._h)
