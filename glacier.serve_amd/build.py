"""Builds libglacier_paged.so (gfx950 kernels + host runtime + C ABI) in-tree, and
libglacier_probe.so, the streaming-read probe that bench.py times beside it.

    python glacier.serve_amd/build.py

Every call recompiles.  hipcc cross-compiles for gfx950 without a GPU.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB = PKG / "libglacier_paged.so"
PROBE_LIB = PKG / "libglacier_probe.so"
PROBE_SOURCES = [CSRC / "gsp_stream_probe.hip"]

SOURCES = [
    CSRC / "gsp_decode.hip",
    CSRC / "gsp_decode_mfma.hip",
    CSRC / "gsp_prefill_mfma.hip",
    CSRC / "gsp_pool_ops.hip",
    CSRC / "gsp_matmul.hip",
    CSRC / "gsp_noalloc.hip",
    CSRC / "gsp_runtime.cpp",
    CSRC / "gsp_step_plan.cpp",
    CSRC / "gsp_host_meta.cpp",
    CSRC / "gsp_status.cpp",
]

ARCH = "gfx950"

# Packed FP32 (v_pk_*_f32) is switched off for all device code.
# The atomic optimizer is off too: it turns the decode kernels' one-lane queue
# ticket into a wave-wide scan whose result is waited for at once, which
# drains every page load in flight.  Without it the wait lands where the
# ticket is used, as a count that leaves the prefetched pages in flight.
DEVICE_FLAGS = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
                "-mllvm", "-amdgpu-atomic-optimizer-strategy=None"]


def hipcc() -> str:
    cand = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(cand).exists():
        raise RuntimeError("hipcc not found: the HIP toolchain is required to build libglacier_paged.so")
    return cand


def build(verbose: bool = False) -> Path:
    _compile(SOURCES, LIB, verbose)
    _compile(PROBE_SOURCES, PROBE_LIB, verbose)
    return LIB


def _compile(sources, lib: Path, verbose: bool) -> None:
    tmp = lib.with_suffix(".so.tmp")
    cmd = [
        hipcc(),
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        "-shared",
        "-Wall",
        "-Wno-unused-result",
        "-fvisibility=hidden",
        "-fvisibility-inlines-hidden",
        f"-I{ROOT / 'include'}",
        *DEVICE_FLAGS,
        "-x",
        "hip",
        *[str(s) for s in sources],
        "-o",
        str(tmp),
    ]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, cwd=str(ROOT), capture_output=True, text=True)
    if res.returncode != 0:
        sys.stderr.write(res.stdout + res.stderr)
        raise RuntimeError(f"hipcc failed with exit code {res.returncode}")
    if verbose and res.stderr.strip():
        # hipcc's host pass warns about the device-only target feature; keep the rest visible.
        lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if lines:
            print("\n".join(lines))
    os.replace(tmp, lib)


if __name__ == "__main__":
    print(build(verbose=True))
