"""Python binding of libglacier_paged.so (ctypes over the C ABI in
include/glacier_paged.h).

Names follow the reference's C# API so that callers read like the reference:
``BlockAllocator`` / ``BlockTable`` mirror the block-id half of
``PagedBlockPool`` and ``BlockTable`` (PagedBlockPool.cs:178-299,
BlockTable.cs:13-117); ``Context.compute_attention`` mirrors
``PagedAttentionKernel.ComputeAttention`` (PagedAttentionKernel.cs:17-32);
``Context.pack_step`` + ``Context.attention_step`` are the batched step the
engine tick issues (ContinuousBatchEngine.cs:426-468).  Status codes become
exceptions the way the reference throws: ``InvalidArgument`` is a
``ValueError`` (ArgumentOutOfRangeException), ``OutOfMemory`` is pool/HBM
exhaustion, ``Unsupported`` is a shape the GPU path rejects.

Device pointers (q, out, k, v) are plain integers, e.g. ``tensor.data_ptr()``.
There is no CPU fallback: if the library is missing this module raises.
"""
from __future__ import annotations

import ctypes
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

try:  # torch, when present, must own the process's HIP runtime: it ships its
    # own libamdhip64 under another file name, and loading ours first would put
    # two HIP runtimes into one process.
    import torch  # noqa: F401
except Exception:  # pragma: no cover - torch is optional for host-only use
    torch = None

LIB_PATH = Path(__file__).resolve().with_name("libglacier_paged.so")

GSP_OK = 0
GSP_E_INVALID_ARG = 1
GSP_E_OOM = 2
GSP_E_UNSUPPORTED = 3
GSP_E_HIP = 4
GSP_E_STATE = 5

KV_F32 = 0
KV_F16 = 1

DECODE_AUTO = 0
DECODE_DPP = 1
DECODE_MFMA = 2
PREFILL_AUTO = 0
PREFILL_TILES = 1
PREFILL_PER_TOKEN = 2
SPLIT_RECORDS = 0
SPLIT_IN_TILE = 1
ROPE_PAIRS = 0
ROPE_HALVES = 1
WTYPE_F32, WTYPE_Q8_0, WTYPE_Q4_K, WTYPE_Q6_K = 0, 8, 12, 14  # GGUF tensor type ids (gsp_matmul_batch)
BLOCK_SIZE = 16
NOALLOC_SCRATCH_BYTES = 16 << 20  # GSP_NOALLOC_SCRATCH_BYTES: fixed scratch of attention_step_noalloc per GPU
NOALLOC_COUNTERS = 65536          # GSP_NOALLOC_COUNTERS: its leading int32 counters


class GspError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[{code}] {message}")
        self.code = code


class InvalidArgument(GspError, ValueError):
    pass


class OutOfMemory(GspError, MemoryError):
    pass


class Unsupported(GspError):
    pass


class HipError(GspError):
    pass


class StateError(GspError):
    pass


_EXC = {
    GSP_E_INVALID_ARG: InvalidArgument,
    GSP_E_OOM: OutOfMemory,
    GSP_E_UNSUPPORTED: Unsupported,
    GSP_E_HIP: HipError,
    GSP_E_STATE: StateError,
}

i32 = ctypes.c_int32
i32p = ctypes.POINTER(ctypes.c_int32)
vp = ctypes.c_void_p
fp = ctypes.POINTER(ctypes.c_float)


class PoolDesc(ctypes.Structure):
    _fields_ = [
        ("total_blocks", i32),
        ("layers", i32),
        ("heads_kv", i32),
        ("head_dim", i32),
        ("v_head_dim", i32),
        ("block_size", i32),
        ("kv_dtype", i32),
    ]


class StepDesc(ctypes.Structure):
    _fields_ = [
        ("num_rows", i32),
        ("max_seq_len", i32),
        ("positions", i32p),
        ("q_lens", i32p),
        ("token_counts", i32p),
        ("bt_offsets", i32p),
        ("bt_ids", i32p),
        ("n_bt_ids", i32),
    ]


class StepInfo(ctypes.Structure):
    _fields_ = [
        ("num_rows", i32),
        ("total_q", i32),
        ("packed_pages", i32),
        ("heads_kv", i32),
        ("decode_units", i32),
        ("split_pairs", i32),
        ("partial_slots", i32),
        ("pages_per_split", i32),
        ("kv_tokens", ctypes.c_int64),
        ("staging_bytes", ctypes.c_int64),
        ("prefill_tiles", i32),
        ("prefill_queries", i32),
        ("prefill_pairs", ctypes.c_int64),
        ("decode_bins", i32),
        ("split_records", i32),
        ("pack_host_ns", ctypes.c_int64),
        ("pack_wait_ns", ctypes.c_int64),
    ]


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
        ("compute_units", i32),
        ("wavefront_size", i32),
        ("clock_khz", i32),
        ("memory_clock_khz", i32),
        ("memory_bus_width_bits", i32),
        ("total_global_mem", ctypes.c_int64),
        ("lds_per_block", ctypes.c_int64),
    ]


class RopeSpec(ctypes.Structure):
    """gsp_rope_spec: QuantKernels.RoPE's freqBase, pairing, ropeDim, mscale, invFreqTable and
    ropeFreqs (host tables of rope_dim / 2 floats, or NULL)."""
    _fields_ = [
        ("freq_base", ctypes.c_float),
        ("style", i32),
        ("rope_dim", i32),
        ("mscale", ctypes.c_float),
        ("inv_freq", ctypes.POINTER(ctypes.c_float)),
        ("freq_factors", ctypes.POINTER(ctypes.c_float)),
    ]


# name -> (restype, argtypes); every symbol declared in include/glacier_paged.h.
_SIGNATURES = {
    "gsp_last_error": (ctypes.c_char_p, []),
    "gsp_abi_version": (ctypes.c_int, []),
    "gsp_device_info_get": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(DeviceInfo)]),
    "gsp_init": (ctypes.c_int, [ctypes.c_int, ctypes.POINTER(vp)]),
    "gsp_shutdown": (None, [vp]),
    "gsp_set_stream": (ctypes.c_int, [vp, vp]),
    "gsp_get_stream": (vp, [vp]),
    "gsp_sync": (ctypes.c_int, [vp]),
    "gsp_pool_create": (ctypes.c_int, [vp, ctypes.POINTER(PoolDesc), ctypes.POINTER(vp)]),
    "gsp_pool_wrap": (ctypes.c_int, [vp, ctypes.POINTER(PoolDesc), vp, vp, ctypes.POINTER(vp)]),
    "gsp_pool_destroy": (None, [vp]),
    "gsp_pool_arenas": (
        ctypes.c_int,
        [vp, ctypes.POINTER(vp), ctypes.POINTER(vp), ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_size_t)],
    ),
    "gsp_pool_write_tokens": (ctypes.c_int, [vp, vp, i32, i32, i32p, i32p, vp, vp]),
    "gsp_rope_write_tokens": (ctypes.c_int, [vp, vp, i32, i32, i32p, i32p, i32p, i32, ctypes.c_float, i32, vp, vp, vp]),
    "gsp_matmul_batch": (ctypes.c_int, [vp, i32, vp, vp, vp, i32, i32, i32]),
    "gsp_pool_write_step": (ctypes.c_int, [vp, vp, i32, vp, vp]),
    "gsp_rope_write_step": (ctypes.c_int, [vp, vp, i32, i32, ctypes.c_float, i32, vp, vp, vp]),
    "gsp_rope_write_tokens_ex": (
        ctypes.c_int,
        [vp, vp, i32, i32, i32p, i32p, i32p, i32, ctypes.POINTER(RopeSpec), vp, vp, vp],
    ),
    "gsp_rope_write_step_ex": (ctypes.c_int, [vp, vp, i32, i32, ctypes.POINTER(RopeSpec), vp, vp, vp]),
    "gsp_pool_copy_block": (ctypes.c_int, [vp, vp, i32, i32, i32]),
    "gsp_pool_upload": (ctypes.c_int, [vp, vp, i32, ctypes.c_size_t, vp, ctypes.c_size_t]),
    "gsp_pool_download": (ctypes.c_int, [vp, vp, i32, ctypes.c_size_t, vp, ctypes.c_size_t]),
    "gsp_step_pack": (ctypes.c_int, [vp, vp, ctypes.POINTER(StepDesc)]),
    "gsp_step_get_info": (ctypes.c_int, [vp, ctypes.POINTER(StepInfo)]),
    "gsp_step_download": (ctypes.c_int, [vp, i32p, i32p, i32p]),
    "gsp_set_split_pages": (ctypes.c_int, [vp, i32]),
    "gsp_set_decode_path": (ctypes.c_int, [vp, i32]),
    "gsp_set_prefill_path": (ctypes.c_int, [vp, i32]),
    "gsp_set_prefill_split": (ctypes.c_int, [vp, i32]),
    "gsp_set_decode_bins": (ctypes.c_int, [vp, i32]),
    "gsp_attention_step": (ctypes.c_int, [vp, vp, i32, i32, vp, vp, ctypes.c_float, fp]),
    "gsp_attention_step_noalloc": (ctypes.c_int, [vp, vp, i32, i32, vp, vp, ctypes.c_float, fp]),
    "gsp_compute_attention": (
        ctypes.c_int,
        [vp, vp, i32, i32, i32, vp, vp, i32p, i32, i32, i32, i32, i32, i32, ctypes.c_float, fp, i32, fp],
    ),
    "gsp_block_allocator_create": (ctypes.c_int, [i32, i32, ctypes.POINTER(vp)]),
    "gsp_block_allocator_destroy": (None, [vp]),
    "gsp_block_allocator_attach_pool": (ctypes.c_int, [vp, vp, vp]),
    "gsp_block_allocator_try_allocate": (ctypes.c_int, [vp, i32p]),
    "gsp_block_allocator_retain": (ctypes.c_int, [vp, i32]),
    "gsp_block_allocator_release": (ctypes.c_int, [vp, i32]),
    "gsp_block_allocator_ref_count": (ctypes.c_int, [vp, i32]),
    "gsp_block_allocator_free_count": (ctypes.c_int, [vp]),
    "gsp_block_allocator_total": (ctypes.c_int, [vp]),
    "gsp_prefix_hash": (ctypes.c_uint64, [ctypes.c_uint64, i32p, i32]),
    "gsp_prefix_hash_chain": (ctypes.c_int, [ctypes.c_uint64, i32p, i32, i32, ctypes.POINTER(ctypes.c_uint64)]),
    "gsp_block_allocator_find_prefix": (ctypes.c_int, [vp, ctypes.c_uint64, i32p]),
    "gsp_block_allocator_bind_prefix": (ctypes.c_int, [vp, ctypes.c_uint64, i32]),
    "gsp_block_table_create": (ctypes.c_int, [vp, ctypes.POINTER(vp)]),
    "gsp_block_table_destroy": (None, [vp]),
    "gsp_block_table_attach_prefix": (ctypes.c_int, [vp, i32p, i32, i32]),
    "gsp_block_table_append_token": (ctypes.c_int, [vp, i32p, i32p]),
    "gsp_block_table_append_tokens": (ctypes.c_int, [vp, i32]),
    "gsp_block_table_token_location": (ctypes.c_int, [vp, i32, i32p, i32p]),
    "gsp_block_table_block_id": (ctypes.c_int, [vp, i32]),
    "gsp_block_table_token_count": (ctypes.c_int, [vp]),
    "gsp_block_table_block_count": (ctypes.c_int, [vp]),
    "gsp_block_table_ids": (ctypes.c_int, [vp, i32p, i32]),
    "gsp_block_table_release_all": (None, [vp]),
}

_lib: Optional[ctypes.CDLL] = None


def load() -> ctypes.CDLL:
    """Loads libglacier_paged.so; raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python glacier.serve_amd/build.py` "
            "(there is no CPU fallback for the paged-attention step)"
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def _check(rc: int) -> None:
    if rc != GSP_OK:
        msg = load().gsp_last_error().decode(errors="replace")
        raise _EXC.get(rc, GspError)(rc, msg)


def _i32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.int32))


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(i32p)


def device_info(device: int = 0) -> DeviceInfo:
    info = DeviceInfo()
    _check(load().gsp_device_info_get(device, ctypes.byref(info)))
    return info


class Context:
    """One device context (GpuContext + the runner's device state)."""

    def __init__(self, device: int = 0):
        lib = load()
        h = vp()
        _check(lib.gsp_init(device, ctypes.byref(h)))
        self._h = h
        self._lib = lib
        self._keep = []

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            self._lib.gsp_shutdown(self._h)
            self._h = vp()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def set_stream(self, hip_stream: Optional[int]) -> None:
        _check(self._lib.gsp_set_stream(self._h, vp(hip_stream or 0)))

    def sync(self) -> None:
        _check(self._lib.gsp_sync(self._h))

    def matmul_batch(self, w_type: int, w_ptr: int, x_ptr: int, y_ptr: int, in_dim: int, out_dim: int,
                     batch: int) -> None:
        """QuantKernels.MatMulBatch (PagedTransformerRunner.cs:601-603,659) on device pointers:
        y[b][o] = sum_i W[o][i] x[b][i], W as F32, Q8_0, Q4_K or Q6_K rows (WTYPE_*)."""
        _check(self._lib.gsp_matmul_batch(self._h, int(w_type), vp(w_ptr), vp(x_ptr), vp(y_ptr), int(in_dim),
                                          int(out_dim), int(batch)))

    def set_split_pages(self, pages: int) -> None:
        """Largest split-KV unit in pages for the next pack (0: sized from the step and device)."""
        _check(self._lib.gsp_set_split_pages(self._h, int(pages)))

    def set_decode_path(self, path: int) -> None:
        _check(self._lib.gsp_set_decode_path(self._h, int(path)))

    def set_decode_bins(self, bins: int) -> None:
        """Most decode workgroups for the next pack_step (0: two per CU)."""
        _check(self._lib.gsp_set_decode_bins(self._h, int(bins)))

    def set_prefill_path(self, path: int) -> None:
        """Route prefill rows for the next pack_step (PREFILL_AUTO / TILES / PER_TOKEN)."""
        _check(self._lib.gsp_set_prefill_path(self._h, int(path)))

    def set_prefill_split(self, mode: int) -> None:
        """How fp32 prefill tiles of the next pack_step get their pages' hi/lo split:
        SPLIT_RECORDS (once per step and layer, the default) or SPLIT_IN_TILE."""
        _check(self._lib.gsp_set_prefill_split(self._h, int(mode)))

    # ---- step packing -------------------------------------------------
    def pack_step(
        self,
        pool: "Pool",
        positions: Sequence[int],
        token_counts: Sequence[int],
        bt_offsets: Sequence[int],
        bt_ids: Sequence[int],
        max_seq_len: int,
        q_lens: Optional[Sequence[int]] = None,
        n_bt_ids: Optional[int] = None,
        want_info: bool = True,
    ) -> Optional[StepInfo]:
        """Packs one engine step (gsp_step_pack).  n_bt_ids defaults to len(bt_ids); the library
        checks the CSR offsets against it."""
        pos = _i32(positions)
        tc = _i32(token_counts)
        off = _i32(bt_offsets)
        ids = _i32(bt_ids) if len(bt_ids) else np.zeros(1, np.int32)
        ql = _i32(q_lens) if q_lens is not None else None
        d = StepDesc()
        d.num_rows = len(pos)
        d.max_seq_len = int(max_seq_len)
        d.positions = _ptr(pos)
        d.q_lens = _ptr(ql) if ql is not None else ctypes.cast(None, i32p)
        d.token_counts = _ptr(tc)
        d.bt_offsets = _ptr(off)
        d.bt_ids = _ptr(ids)
        d.n_bt_ids = len(bt_ids) if n_bt_ids is None else int(n_bt_ids)
        _check(self._lib.gsp_step_pack(self._h, pool.handle, ctypes.byref(d)))
        return self.step_info() if want_info else None

    def step_info(self) -> StepInfo:
        info = StepInfo()
        _check(self._lib.gsp_step_get_info(self._h, ctypes.byref(info)))
        return info

    def download_step(self):
        info = self.step_info()
        rows = np.zeros(info.num_rows + 1, np.int32)
        ids = np.zeros(max(1, info.packed_pages), np.int32)
        ctxl = np.zeros(max(1, info.total_q), np.int32)
        _check(self._lib.gsp_step_download(self._h, _ptr(rows), _ptr(ids), _ptr(ctxl)))
        return rows, ids[: info.packed_pages], ctxl[: info.total_q]

    # ---- attention ------------------------------------------------------
    def attention_step(
        self, pool: "Pool", layer: int, n_heads: int, q_ptr: int, out_ptr: int, attn_scale: float, sink_logit=None
    ) -> None:
        sink = None
        if sink_logit is not None:
            sink = ctypes.pointer(ctypes.c_float(sink_logit))
        _check(
            self._lib.gsp_attention_step(
                self._h, pool.handle, int(layer), int(n_heads), vp(q_ptr), vp(out_ptr), float(attn_scale), sink
            )
        )

    def attention_step_noalloc(
        self, pool: "Pool", layer: int, n_heads: int, q_ptr: int, out_ptr: int, attn_scale: float, sink_logit=None
    ) -> None:
        """attention_step with the split-KV workspace in the library's fixed per-GPU scratch array:
        allocates nothing (for graph capture and tight loops); calls that overlap on one GPU race."""
        sink = None
        if sink_logit is not None:
            sink = ctypes.pointer(ctypes.c_float(sink_logit))
        _check(
            self._lib.gsp_attention_step_noalloc(
                self._h, pool.handle, int(layer), int(n_heads), vp(q_ptr), vp(out_ptr), float(attn_scale), sink
            )
        )

    def compute_attention(
        self,
        stage_layer: int,
        model_layer: int,
        pos: int,
        q_ptr: int,
        out_ptr: int,
        block_table: "BlockTable | Sequence[int]",
        pool: "Pool",
        n_heads: int,
        n_heads_kv: int,
        head_dim: int,
        v_head_dim: int,
        attn_scale: float,
        max_seq_len: int,
        token_count: Optional[int] = None,
        sink_logit=None,
    ) -> None:
        """PagedAttentionKernel.ComputeAttention (PagedAttentionKernel.cs:17-32) on the GPU."""
        if isinstance(block_table, BlockTable):
            ids = block_table.as_span()
            tc = block_table.token_count
        else:
            ids = _i32(block_table)
            tc = int(token_count)
        n = len(ids)
        arr = ids if n else np.zeros(1, np.int32)
        sink = ctypes.pointer(ctypes.c_float(sink_logit)) if sink_logit is not None else None
        _check(
            self._lib.gsp_compute_attention(
                self._h, pool.handle, int(stage_layer), int(model_layer), int(pos), vp(q_ptr), vp(out_ptr),
                _ptr(arr), n, int(tc), int(n_heads), int(n_heads_kv), int(head_dim), int(v_head_dim),
                float(attn_scale), None, int(max_seq_len), sink,
            )
        )


class Pool:
    """Device K/V arenas in the reference PagedBlockPool layout."""

    def __init__(self, ctx: Context, handle: vp, desc: PoolDesc):
        self._ctx = ctx
        self._h = handle
        self.desc = desc

    @classmethod
    def create(cls, ctx: Context, total_blocks: int, layers: int, heads_kv: int, head_dim: int,
               kv_dtype: int = KV_F32, v_head_dim: int = -1, block_size: int = BLOCK_SIZE) -> "Pool":
        d = PoolDesc(total_blocks, layers, heads_kv, head_dim, v_head_dim, block_size, kv_dtype)
        h = vp()
        _check(load().gsp_pool_create(ctx.handle, ctypes.byref(d), ctypes.byref(h)))
        d2 = PoolDesc.from_buffer_copy(d)
        if d2.v_head_dim <= 0:
            d2.v_head_dim = d2.head_dim
        return cls(ctx, h, d2)

    @classmethod
    def wrap(cls, ctx: Context, k_ptr: int, v_ptr: int, total_blocks: int, layers: int, heads_kv: int,
             head_dim: int, kv_dtype: int = KV_F32, v_head_dim: int = -1, block_size: int = BLOCK_SIZE) -> "Pool":
        d = PoolDesc(total_blocks, layers, heads_kv, head_dim, v_head_dim, block_size, kv_dtype)
        h = vp()
        _check(load().gsp_pool_wrap(ctx.handle, ctypes.byref(d), vp(k_ptr), vp(v_ptr), ctypes.byref(h)))
        d2 = PoolDesc.from_buffer_copy(d)
        if d2.v_head_dim <= 0:
            d2.v_head_dim = d2.head_dim
        return cls(ctx, h, d2)

    @property
    def handle(self):
        return self._h

    def destroy(self) -> None:
        if self._h:
            load().gsp_pool_destroy(self._h)
            self._h = vp()

    def arenas(self):
        k, v = vp(), vp()
        kb, vb = ctypes.c_size_t(), ctypes.c_size_t()
        _check(load().gsp_pool_arenas(self._h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(kb), ctypes.byref(vb)))
        return k.value, v.value, kb.value, vb.value

    def upload(self, which: int, data: np.ndarray, offset_bytes: int = 0) -> None:
        data = np.ascontiguousarray(data)
        _check(load().gsp_pool_upload(self._ctx.handle, self._h, which, offset_bytes, data.ctypes.data, data.nbytes))

    def download(self, which: int, nbytes: int, offset_bytes: int = 0) -> np.ndarray:
        buf = np.empty(nbytes, np.uint8)
        _check(load().gsp_pool_download(self._ctx.handle, self._h, which, offset_bytes, buf.ctypes.data, nbytes))
        return buf

    def write_tokens(self, layer: int, block_ids, slots, k_ptr: int, v_ptr: int) -> None:
        """PagedBlockPool.Store (PagedBlockPool.cs:151-161) for a batch of tokens."""
        b = _i32(block_ids)
        s = _i32(slots)
        if len(b) != len(s):
            raise ValueError("block_ids and slots differ in length")
        _check(load().gsp_pool_write_tokens(self._ctx.handle, self._h, int(layer), len(b), _ptr(b), _ptr(s),
                                            vp(k_ptr), vp(v_ptr)))

    def rope_write_tokens(self, layer: int, positions, block_ids, slots, n_heads: int, freq_base: float,
                          style: int, q_ptr: int, k_ptr: int, v_ptr: int) -> None:
        """QuantKernels.RoPE then PagedBlockPool.Store for a batch of tokens
        (PagedTransformerRunner.cs:253-267): Q rotated in place, K rotated into the pool, V stored."""
        p = _i32(positions)
        b = _i32(block_ids)
        s = _i32(slots)
        if not (len(p) == len(b) == len(s)):
            raise ValueError("positions, block_ids and slots differ in length")
        _check(load().gsp_rope_write_tokens(self._ctx.handle, self._h, int(layer), len(b), _ptr(p), _ptr(b), _ptr(s),
                                            int(n_heads), float(freq_base), int(style), vp(q_ptr), vp(k_ptr),
                                            vp(v_ptr)))

    def rope_write_tokens_ex(self, layer: int, positions, block_ids, slots, n_heads: int, rope: "Rope",
                             q_ptr: int, k_ptr: int, v_ptr: int) -> None:
        """rope_write_tokens with the runner's optional RoPE arguments (gsp_rope_write_tokens_ex)."""
        p = _i32(positions)
        b = _i32(block_ids)
        s = _i32(slots)
        if not (len(p) == len(b) == len(s)):
            raise ValueError("positions, block_ids and slots differ in length")
        spec = rope.spec(self.desc.head_dim)
        _check(load().gsp_rope_write_tokens_ex(self._ctx.handle, self._h, int(layer), len(b), _ptr(p), _ptr(b),
                                               _ptr(s), int(n_heads), ctypes.byref(spec), vp(q_ptr), vp(k_ptr),
                                               vp(v_ptr)))

    def rope_write_step_ex(self, layer: int, n_heads: int, rope: "Rope", q_ptr: int, k_ptr: int, v_ptr: int) -> None:
        """rope_write_step with the runner's optional RoPE arguments (gsp_rope_write_step_ex)."""
        spec = rope.spec(self.desc.head_dim)
        _check(load().gsp_rope_write_step_ex(self._ctx.handle, self._h, int(layer), int(n_heads), ctypes.byref(spec),
                                             vp(q_ptr), vp(k_ptr), vp(v_ptr)))

    def write_step(self, layer: int, k_ptr: int, v_ptr: int) -> None:
        """Store of the packed step's own tokens (gsp_pool_write_step): query token i's K/V into the
        slot of its position, from the step's device copy (no host arrays, no upload)."""
        _check(load().gsp_pool_write_step(self._ctx.handle, self._h, int(layer), vp(k_ptr), vp(v_ptr)))

    def rope_write_step(self, layer: int, n_heads: int, freq_base: float, style: int, q_ptr: int, k_ptr: int,
                        v_ptr: int) -> None:
        """RoPE then Store of the packed step's own tokens at their positions (gsp_rope_write_step)."""
        _check(load().gsp_rope_write_step(self._ctx.handle, self._h, int(layer), int(n_heads), float(freq_base),
                                          int(style), vp(q_ptr), vp(k_ptr), vp(v_ptr)))

    def copy_block_data(self, src: int, dst: int, valid_tokens: int) -> None:
        """PagedBlockPool.CopyBlockData (PagedBlockPool.cs:304-327) on the device."""
        _check(load().gsp_pool_copy_block(self._ctx.handle, self._h, int(src), int(dst), int(valid_tokens)))


class Rope:
    """The rotation QuantKernels.RoPE applies (PagedTransformerRunner.cs:253-264): freqBase, the
    pairing (ROPE_PAIRS / ROPE_HALVES), ropeDim (0: the whole head), invFreqTable (YaRN), ropeFreqs
    (frequency factors) and mscale (0: 1).  Holds its tables for the calls that use it."""

    def __init__(self, freq_base: float, style: int = 0, rope_dim: int = 0, inv_freq=None, freq_factors=None,
                 mscale: float = 0.0):
        self.freq_base = float(freq_base)
        self.style = int(style)
        self.rope_dim = int(rope_dim)
        self.mscale = float(mscale)
        self.inv_freq = None if inv_freq is None else np.ascontiguousarray(inv_freq, dtype=np.float32)
        self.freq_factors = None if freq_factors is None else np.ascontiguousarray(freq_factors, dtype=np.float32)

    def spec(self, head_dim: int) -> RopeSpec:
        """The C struct for a pool of `head_dim`; the tables must hold rope_dim / 2 entries, the
        count the library reads."""
        half = (self.rope_dim or head_dim) // 2
        for name, t in (("inv_freq", self.inv_freq), ("freq_factors", self.freq_factors)):
            if t is not None and t.size != half:
                raise ValueError(f"{name} holds {t.size} entries; rope_dim / 2 = {half}")
        fp32 = ctypes.POINTER(ctypes.c_float)
        tab = lambda t: fp32() if t is None else t.ctypes.data_as(fp32)
        return RopeSpec(self.freq_base, self.style, self.rope_dim, self.mscale, tab(self.inv_freq),
                        tab(self.freq_factors))


def prefix_hash(parent_hash: int, tokens) -> int:
    """PagedBlockPool.ComputePrefixHash (PagedBlockPool.cs:168-172): XXH3-64 of the
    token ids' little-endian bytes, seeded with the parent block's hash."""
    t = _i32(tokens)
    h = load().gsp_prefix_hash(int(parent_hash) & 0xFFFFFFFFFFFFFFFF, _ptr(t) if len(t) else None, len(t))
    if h == 0:
        err = load().gsp_last_error()
        if err:
            _check(GSP_E_INVALID_ARG)
    return h


def prefix_hash_chain(parent_hash: int, tokens, block_size: int = BLOCK_SIZE) -> np.ndarray:
    """The hash of every full block of `tokens`, each seeded with the previous one (uint64 array)."""
    t = _i32(tokens)
    n = len(t) // block_size
    out = np.zeros(max(1, n), np.uint64)
    _check(load().gsp_prefix_hash_chain(int(parent_hash) & 0xFFFFFFFFFFFFFFFF, _ptr(t) if len(t) else None, n,
                                        int(block_size), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint64))))
    return out[:n]


class BlockAllocator:
    """Block-id half of PagedBlockPool: LIFO free stack with refcounts."""

    def __init__(self, total_blocks: int, block_size: int = BLOCK_SIZE):
        h = vp()
        _check(load().gsp_block_allocator_create(int(total_blocks), int(block_size), ctypes.byref(h)))
        self._h = h
        self.block_size = block_size

    @property
    def handle(self):
        return self._h

    def close(self) -> None:
        if self._h:
            load().gsp_block_allocator_destroy(self._h)
            self._h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attach_pool(self, ctx: Optional[Context], pool: Optional[Pool]) -> None:
        _check(load().gsp_block_allocator_attach_pool(self._h, ctx.handle if ctx else None,
                                                      pool.handle if pool else None))

    def try_allocate_block(self):
        bid = i32()
        ok = load().gsp_block_allocator_try_allocate(self._h, ctypes.byref(bid))
        return bool(ok), bid.value

    def retain_block(self, block_id: int) -> int:
        r = load().gsp_block_allocator_retain(self._h, int(block_id))
        if r < 0:
            _check(GSP_E_INVALID_ARG)
        return r

    def release_block(self, block_id: int) -> int:
        return load().gsp_block_allocator_release(self._h, int(block_id))

    free_block = release_block

    def free_blocks(self, ids) -> None:
        for b in ids:
            self.release_block(int(b))

    def get_ref_count(self, block_id: int) -> int:
        return load().gsp_block_allocator_ref_count(self._h, int(block_id))

    @property
    def total_blocks(self) -> int:
        return load().gsp_block_allocator_total(self._h)

    @property
    def free_blocks_count(self) -> int:
        return load().gsp_block_allocator_free_count(self._h)

    def try_find_prefix_block(self, prefix_hash: int):
        """TryFindPrefixBlock (PagedBlockPool.cs:194-220): (found, block id); a hit holds one more reference."""
        b = i32()
        ok = load().gsp_block_allocator_find_prefix(self._h, int(prefix_hash), ctypes.byref(b))
        return bool(ok), b.value

    def bind_prefix_block(self, prefix_hash: int, block_id: int) -> None:
        """BindPrefixBlock (PagedBlockPool.cs:225-234)."""
        _check(load().gsp_block_allocator_bind_prefix(self._h, int(prefix_hash), int(block_id)))

    @property
    def allocated_blocks_count(self) -> int:
        return self.total_blocks - self.free_blocks_count


class BlockTable:
    """Per-sequence logical -> physical page table (BlockTable.cs:13-117)."""

    def __init__(self, allocator: BlockAllocator):
        h = vp()
        _check(load().gsp_block_table_create(allocator.handle, ctypes.byref(h)))
        self._h = h
        self._alloc = allocator  # keeps the allocator alive

    def close(self) -> None:
        if self._h:
            load().gsp_block_table_destroy(self._h)
            self._h = vp()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def attach_prefix_blocks(self, ids, token_count: int) -> None:
        a = _i32(ids)
        _check(load().gsp_block_table_attach_prefix(self._h, _ptr(a) if len(a) else None, len(a), int(token_count)))

    def append_token(self):
        b, o = i32(), i32()
        ok = load().gsp_block_table_append_token(self._h, ctypes.byref(b), ctypes.byref(o))
        if ok < 0:
            _check(GSP_E_INVALID_ARG)
        return bool(ok), b.value, o.value

    def append_tokens(self, n: int) -> int:
        """AppendToken n times; returns how many succeeded."""
        return load().gsp_block_table_append_tokens(self._h, int(n))

    def get_token_location(self, token: int):
        b, o = i32(), i32()
        _check(load().gsp_block_table_token_location(self._h, int(token), ctypes.byref(b), ctypes.byref(o)))
        return b.value, o.value

    def get_block_id(self, index: int) -> int:
        r = load().gsp_block_table_block_id(self._h, int(index))
        if r < 0:
            _check(GSP_E_INVALID_ARG)
        return r

    @property
    def token_count(self) -> int:
        return load().gsp_block_table_token_count(self._h)

    @property
    def block_count(self) -> int:
        return load().gsp_block_table_block_count(self._h)

    def as_span(self) -> np.ndarray:
        n = self.block_count
        out = np.zeros(max(1, n), np.int32)
        load().gsp_block_table_ids(self._h, _ptr(out), n)
        return out[:n]

    def release_all(self) -> None:
        load().gsp_block_table_release_all(self._h)
