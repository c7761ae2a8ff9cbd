"""The host step packer under AddressSanitizer + UndefinedBehaviorSanitizer.

gsp_step_pack validates caller CSR tables, plans the split-KV units, the decode
bins and the prefill tiles, and writes the step image (gsp_step_plan.cpp, plain
C++ with no HIP).  tests/native/step_plan_fuzz.cpp drives that code, built from
the library's own source with the sanitizers, on:
- the five measured shapes and smaller steps of general shapes (pages of 4, 8,
  17, 24 and 32 tokens, head_dim 32 with v_head_dim 64, prefill chunks, empty
  rows), each
  planned with several split sizes, bin counts and prefill routes and its image
  checked (packed tables, unit coverage, split slots, bins, tiles, write slots);
- seeded malformed copies of them (offsets out of order or out of range, short
  tables, block ids outside the pool, positions and token counts outside
  [0, maxSeqLen), negative or huge query lengths, NULL arrays), each of which
  must be refused with GSP_E_INVALID_ARG (PagedAttentionKernel.cs:34-39 and the
  table bounds);
- random steps over wide value ranges, refused or planned into a checked image.
The test passes when the driver reports no failure and the sanitizers none.
"""
import struct
import subprocess
from pathlib import Path

import numpy as np
import pytest

import workloads

NATIVE = Path(__file__).resolve().parent / "native"


@pytest.fixture(scope="module")
def plan_builds():
    subprocess.run(["make", "-C", str(NATIVE), "-j2", "_build/step_plan_fuzz", "_build/step_plan_fuzz_asan"],
                   check=True, capture_output=True, text=True)
    return NATIVE / "_build"


def _steps():
    steps = [workloads.CONFIGS[c]() for c in (1, 2, 3, 4, 5)]
    steps.append(workloads.refmodel_decode())
    steps.append(workloads.small_step(seed=1, rows=9, n_heads=4, n_kv=2, head_dim=32, ctx_lo=0, ctx_hi=300,
                                      total_blocks=512, block_size=4, v_head_dim=64))
    steps.append(workloads.small_step(seed=2, rows=7, n_heads=28, n_kv=4, head_dim=128, ctx_lo=0, ctx_hi=400,
                                      total_blocks=512, q_lens=np.array([1, 40, 0, 17, 1, 3, 1])))
    steps.append(workloads.small_step(seed=3, rows=5, n_heads=8, n_kv=8, head_dim=64, kv_dtype="f16", ctx_lo=0,
                                      ctx_hi=50, total_blocks=64, block_size=8))
    # Pool pages above 16 tokens (read as kernel pages of 16, 12 and 1 tokens).
    steps.append(workloads.small_step(seed=4, rows=8, n_heads=28, n_kv=4, head_dim=128, ctx_lo=0, ctx_hi=900,
                                      total_blocks=256, block_size=32, q_lens=np.array([1, 33, 1, 1, 17, 0, 1, 2])))
    steps.append(workloads.small_step(seed=5, rows=6, n_heads=8, n_kv=2, head_dim=64, ctx_lo=1, ctx_hi=400,
                                      total_blocks=128, block_size=24))
    steps.append(workloads.small_step(seed=6, rows=4, n_heads=4, n_kv=2, head_dim=32, ctx_lo=1, ctx_hi=100,
                                      total_blocks=64, block_size=17))
    return steps


def _write(path: Path, steps) -> None:
    with open(path, "wb") as f:
        f.write(struct.pack("<ii", 0x53505347, len(steps)))
        for s in steps:
            has_q = s.q_lens is not None
            f.write(struct.pack("<11i", s.total_blocks, s.n_kv, s.head_dim, s.dv, s.block_size,
                                1 if s.kv_dtype == "f16" else 0, s.num_rows, s.max_seq_len, int(has_q),
                                len(s.bt_ids), 4))
            arrays = [s.positions] + ([s.q_lens] if has_q else []) + [s.token_counts, s.bt_offsets, s.bt_ids]
            for a in arrays:
                f.write(np.ascontiguousarray(a, dtype="<i4").tobytes())


@pytest.mark.parametrize("variant", ["step_plan_fuzz", "step_plan_fuzz_asan"])
def test_step_packer_under_sanitizers(plan_builds, tmp_path, variant):
    path = tmp_path / "steps.bin"
    _write(path, _steps())
    res = subprocess.run([str(plan_builds / variant), str(path), "3000"], capture_output=True, text=True, timeout=600)
    report = res.stdout + res.stderr
    assert res.returncode == 0, report
    assert "ok" in res.stdout.splitlines()[-1], report
    for marker in ("ERROR: AddressSanitizer", "runtime error:", "FAIL "):
        assert marker not in report, report
