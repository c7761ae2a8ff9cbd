"""The split-KV handoff's instructions on gfx950, pinned at build time.

A split piece publishes its partial with agent-scope relaxed atomic stores,
waits for every store of the wave to complete (s_waitcnt vmcnt(0)), meets the
workgroup barrier and bumps the pair's counter with an agent-scope relaxed
atomic add; the last piece reads the partials with agent-scope relaxed atomic
loads (gsp_epilogue.h).  Relaxed atomics order nothing in the HIP/C++ memory
model, so the protocol's correctness rests on how gfx950 lowers them: the
stores and loads carry sc1 (they go to and come from the coherence point that
all XCDs share instead of one XCD's L2), and the explicit wait completes the
stores before the counter moves.  This test compiles a probe kernel made of
exactly those helpers with the library's own flags and checks that lowering
in the resulting gfx950 assembly, so that a compiler that lowered them
differently fails here, on the CPU, rather than silently in a GPU soak.
"""
import shutil
import subprocess
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT / "glacier.serve_amd"))

PROBE = r"""
#include "gsp_epilogue.h"

extern "C" __global__ void handoff_probe(float* part, int* counter, const float* other, float* out, int* last) {
    gsp::coherent_store(part + threadIdx.x, (float)threadIdx.x);  // publish
    gsp::wait_vm_complete();                                       // the stores are complete
    __syncthreads();
    if (threadIdx.x == 0)
        *last = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);  // count
    __syncthreads();
    out[threadIdx.x] = gsp::coherent_load(other + threadIdx.x);    // merge reads another piece
}
"""


def _kernel_asm(tmp_path: Path) -> list:
    import build

    hipcc = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(hipcc).exists():
        pytest.skip("hipcc is not installed")
    src = tmp_path / "probe.hip"
    src.write_text(PROBE)
    out = tmp_path / "probe.s"
    cmd = [hipcc, f"--offload-arch={build.ARCH}", "-O3", "-std=c++17", f"-I{ROOT / 'include'}",
           f"-I{ROOT / 'glacier.serve_amd' / 'csrc'}", *build.DEVICE_FLAGS, "-x", "hip", "--cuda-device-only",
           "-S", str(src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    lines, inside = [], False
    for ln in out.read_text().splitlines():
        if ln.startswith("handoff_probe:"):
            inside = True
        elif inside and "s_endpgm" in ln:
            break
        elif inside:
            ln = ln.split(";")[0].strip()
            if ln and not ln.startswith("."):
                lines.append(ln)
    assert lines, "probe kernel not found in the assembly"
    return lines


def test_handoff_lowering(tmp_path):
    asm = _kernel_asm(tmp_path)
    ops = [ln.split()[0] for ln in asm]
    stores = [ln for ln in asm if ln.startswith(("global_store", "buffer_store", "flat_store"))]
    loads_sc1 = [ln for ln in asm if ln.startswith(("global_load", "buffer_load", "flat_load")) and "sc1" in ln]
    atomics = [i for i, ln in enumerate(asm) if ln.startswith(("global_atomic_add", "flat_atomic_add",
                                                                "buffer_atomic_add"))]
    # No cache writeback or invalidation: the protocol does not rely on fences.
    assert not any(op.startswith(("buffer_wbl2", "buffer_inv", "buffer_wbinvl1")) for op in ops), asm
    # The partial store goes to the shared coherence point (sc1) ...
    assert stores and all("sc1" in ln for ln in stores[:1]), stores
    # ... and is complete (vmcnt(0)) before the counter's atomic add.
    assert len(atomics) == 1, asm
    first_store = asm.index(stores[0])
    between = asm[first_store + 1:atomics[0]]
    assert any(ln.startswith("s_waitcnt") and "vmcnt(0)" in ln for ln in between), between
    # The last piece reads other pieces' partials from the same point.
    assert loads_sc1, asm
