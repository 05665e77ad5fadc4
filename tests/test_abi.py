"""The C-ABI library loads and exports every symbol include/llrs.h declares (CPU only)."""
from __future__ import annotations

import re
import subprocess

import pytest

from conftest import ROOT


def declared(header) -> set:
    text = re.sub(r"/\*.*?\*/", "", header.read_text(), flags=re.S)
    return set(re.findall(r"\b(llrs_[a-z0-9_]+)\s*\(", text)) | \
        set(re.findall(r"\b(oq_[a-z0-9_]+)\s*\(", text))


def exported(lib) -> set:
    out = subprocess.run(["nm", "-D", "--defined-only", str(lib)], capture_output=True, text=True,
                         check=True).stdout
    return {l.split()[-1] for l in out.splitlines() if " T " in l}


def test_library_exports_every_declared_symbol(llrs):
    names = declared(ROOT / "include" / "llrs.h")
    assert len(names) >= 30
    missing = names - exported(llrs.LIB_PATH)
    assert not missing, missing
    llrs.lib()  # loads, and binds every signature


def test_python_bindings_cover_the_header(llrs):
    bound = {name for name, _, _ in llrs.SIGNATURES}
    assert bound == declared(ROOT / "include" / "llrs.h")


def test_oracle_exports_its_header(oracle):
    from oracle_ffi import LIB
    names = declared(ROOT / "oracle" / "oracle.h")
    assert not names - exported(LIB)


def test_no_cpu_fallback_without_a_gpu(llrs):
    """Without a GPU the backend refuses to start instead of falling back to CPU."""
    import os
    if os.path.exists("/dev/kfd"):
        pytest.skip("a GPU is present")
    with pytest.raises(llrs.LlrsError):
        llrs.HipBackend(0)


def test_error_text_is_thread_local_and_set(llrs):
    import ctypes as C
    rc = llrs.lib().llrs_quantize(99, None, 0, 0, None, 0, None, None)
    assert rc == -2
    assert b"supports" in llrs.lib().llrs_last_error()
    del C
