"""The C ABI without a GPU: the library loads, exports every function
include/titania_hip.h declares, and reports errors instead of crashing."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from titania_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "titania_hip.h"


def declared() -> list[str]:
    text = HEADER.read_text()
    return sorted(set(re.findall(r"^TH_API\s+[\w\s\*]*?\b(th_\w+)\s*\(", text, re.M)))


def test_header_declares_the_trait():
    names = declared()
    # One entry point per method of model/device.rs:9-89.
    for m in ["upload", "alloc", "resize", "read", "write", "copy", "embed", "matmul", "add", "rmsnorm", "rope",
              "attention", "silu_mul"]:
        assert f"th_{m}" in names


def test_library_exports_every_declared_symbol():
    lib = C.CDLL(str(_lib.LIB_PATH))
    missing = [n for n in declared() if not hasattr(lib, n)]
    assert not missing, missing


def test_binding_matches_header():
    assert sorted(_lib.SIGNATURES) == declared()


def test_errors_without_gpu_are_reported():
    lib = _lib.lib()
    rc = lib.th_resize(None, None, 1)
    assert rc == _lib.TH_ERR_INVALID
    assert b"null" in lib.th_last_error()
    rc = lib.th_model_create(None, None, None, 0, None)
    assert rc == _lib.TH_ERR_INVALID
    assert lib.th_buffer_len(None) == 0


@pytest.mark.skipif(Path("/dev/kfd").exists(), reason="a GPU is present")
def test_device_create_fails_cleanly_without_gpu():
    lib = _lib.lib()
    h = C.c_void_p()
    rc = lib.th_device_create(0, C.byref(h))
    assert rc in (_lib.TH_ERR_HIP, _lib.TH_ERR_INVALID)
    assert lib.th_last_error()
