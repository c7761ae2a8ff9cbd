"""The C-ABI library loads and exports every entry point include/glacier_paged.h declares.

No compute is issued: these run without a GPU.
"""
import ctypes
import re
import subprocess
from pathlib import Path

import glacier_paged as gp

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "glacier_paged.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gsp_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared_functions()
    for must in ("gsp_init", "gsp_pool_create", "gsp_step_pack", "gsp_attention_step", "gsp_compute_attention",
                 "gsp_pool_write_tokens", "gsp_block_table_append_token", "gsp_last_error"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = ctypes.CDLL(str(gp.LIB_PATH))
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_covers_every_declared_symbol():
    assert set(declared_functions()) <= set(gp._SIGNATURES)


def test_no_unexpected_exports():
    out = subprocess.run(["nm", "-D", "--defined-only", str(gp.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    ours = {n for n in exported if n.startswith("gsp_")}
    assert ours == set(declared_functions())


def test_abi_version_and_error_string():
    lib = gp.load()
    assert lib.gsp_abi_version() == 9
    # A host-only call that fails sets the thread-local message.
    h = ctypes.c_void_p()
    rc = lib.gsp_block_allocator_create(0, 16, ctypes.byref(h))
    assert rc == gp.GSP_E_INVALID_ARG
    assert b"totalBlocks" in lib.gsp_last_error()


def test_probe_library_exports_only_the_stream_probe():
    """libglacier_probe.so (bench.py's streaming-read ceiling) is separate from the boundary."""
    probe = Path(gp.LIB_PATH).with_name("libglacier_probe.so")
    out = subprocess.run(["nm", "-D", "--defined-only", str(probe)], capture_output=True, text=True,
                         check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    assert {n for n in exported if n.startswith("gsp_")} == {"gsp_probe_stream_read"}
    assert "gsp_probe_stream_read" not in declared_functions()
