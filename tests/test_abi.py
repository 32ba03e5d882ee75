"""The C ABI without a GPU: the library loads, exports every function
include/titania_hip.h declares, and reports errors instead of crashing."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

import cabi
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


def test_ctypes_argtypes_match_header():
    """Every ctypes restype and argtype against the header's declaration: the
    same number of arguments, each of the same kind (pointer, size_t, int,
    float, fixed-width integer)."""
    header = cabi.header_signatures()
    bound = cabi.ctypes_signatures(_lib.SIGNATURES)
    bad = {n: (cabi.as_ctypes_kinds(header[n]), bound[n]) for n in header
           if cabi.as_ctypes_kinds(header[n]) != bound[n]}
    assert not bad, bad


def test_test_entry_points_exported_and_bound():
    """The test-only entry points of include/titania_hip_test.h: exported,
    and bound by tests/test_fused_kernels.py with the header's kinds."""
    import test_fused_kernels as fk

    header = cabi.header_signatures(cabi.TEST_HEADER)
    assert len(header) == 10 and sorted(header) == sorted(fk.TEST_SIGNATURES)
    lib = C.CDLL(str(_lib.LIB_PATH))
    assert all(hasattr(lib, n) for n in header)
    bound = cabi.ctypes_signatures({n: (C.c_int, a) for n, a in fk.TEST_SIGNATURES.items()})
    bad = {n: (cabi.as_ctypes_kinds(header[n]), bound[n]) for n in header if cabi.as_ctypes_kinds(header[n]) != bound[n]}
    assert not bad, bad


def test_rust_sys_crate_matches_header():
    """The Rust FFI crate's extern block (titania_amd/rust/hip-sys/lib.rs,
    not compiled here) declares every header function with the same argument
    count and kinds and the same return kind."""
    header = cabi.header_signatures()
    rust = cabi.rust_signatures()
    assert sorted(rust) == sorted(header)
    bad = {n: (header[n], rust[n]) for n in header if header[n] != rust[n]}
    assert not bad, bad


def test_signature_parsers_see_a_planted_mismatch(tmp_path):
    """The checks above can fail: a copy of the crate with one argument
    dropped and one changed from usize to i32 is caught."""
    text = cabi.RUST_SYS.read_text()
    text = text.replace("pub fn th_buffer_len(buf: *const th_buffer) -> usize;", "pub fn th_buffer_len() -> usize;")
    text = text.replace("pub fn th_resize(dev: *mut th_device, buf: *mut th_buffer, len: usize)",
                        "pub fn th_resize(dev: *mut th_device, buf: *mut th_buffer, len: i32)")
    p = tmp_path / "lib.rs"
    p.write_text(text)
    rust = cabi.rust_signatures(p)
    header = cabi.header_signatures()
    assert rust["th_buffer_len"] != header["th_buffer_len"]
    assert rust["th_resize"] != header["th_resize"]
    assert rust["th_read"] == header["th_read"]


# The methods of model/device.rs:9-89 `trait Device`.
TRAIT_METHODS = ["upload", "alloc", "resize", "read", "write", "copy", "embed", "matmul", "add", "rmsnorm", "rope",
                 "attention", "silu_mul"]


def test_rust_device_impl_covers_the_trait():
    """titania_amd/rust/model/hip.rs implements every trait method, each
    through the header function of the same name, and calls only functions
    the header declares."""
    text = (cabi.ROOT / "titania_amd" / "rust" / "model" / "hip.rs").read_text()
    impl = text[text.index("impl Device for Hip"):]
    for m in TRAIT_METHODS:
        assert re.search(rf"\bfn {m}\(", impl), m
        assert f"sys::th_{m}(" in impl, m
    called = set(re.findall(r"sys::(th_\w+)\(", text))
    assert called <= set(cabi.header_signatures()), called - set(cabi.header_signatures())


# The trait extension (titania_amd/rust/patches/model-device.rs.patch): each
# default method, and the header function hip.rs overrides it with.
EXTENSION_METHODS = {"add_rmsnorm": "th_add_rmsnorm", "qkv_rope_append": "th_qkv_rope_append",
                     "gate_up_silu": "th_gate_up_silu", "argmax": "th_argmax"}
PATCHES = cabi.ROOT / "titania_amd" / "rust" / "patches"
PATCHED_FILES = ["model/device.rs", "model/model.rs", "model/lib.rs", "model/Cargo.toml", "cli/opts.rs", "cli/run.rs"]


def _added_lines(name: str) -> str:
    text = (PATCHES / name).read_text()
    return "\n".join(line[1:] for line in text.splitlines() if line.startswith("+") and not line.startswith("+++"))


def test_rust_device_impl_overrides_the_extension():
    """Every default method the trait-extension patch adds is overridden in
    hip.rs through its fused header function, and the patched forward_batch
    calls each of them."""
    device = _added_lines("model-device.rs.patch")
    model = _added_lines("model-model.rs.patch")
    text = (cabi.ROOT / "titania_amd" / "rust" / "model" / "hip.rs").read_text()
    impl = text[text.index("impl Device for Hip"):text.index("pub struct HipModel")]
    header = cabi.header_signatures()
    for m, fn in EXTENSION_METHODS.items():
        assert re.search(rf"\bfn {m}\(", device), f"default method {m}"
        body = impl[impl.index(f"fn {m}("):]
        body = body[:body.index("\n    }\n")]
        assert f"sys::{fn}(" in body, (m, fn)
        assert fn in header
        assert re.search(rf"\.{m}\(", model), f"forward_batch calls {m}"
    assert len(re.findall(r"\bfn \w+\(", device)) == len(EXTENSION_METHODS)


def test_patches_apply_to_the_reference(tmp_path):
    """The reference-side patches apply cleanly to copies of the reference's
    files (the reference itself is not touched) and give the `hip` device,
    its CLI name and the extension calls."""
    import shutil
    import subprocess

    ref_root = Path("/root/reference")
    if not (ref_root / "model" / "device.rs").exists():
        pytest.skip("the reference sources are not in this container")
    for f in PATCHED_FILES:
        (tmp_path / f).parent.mkdir(parents=True, exist_ok=True)
        shutil.copy(ref_root / f, tmp_path / f)
    for f in PATCHED_FILES:
        patch = PATCHES / (f.replace("/", "-") + ".patch")
        r = subprocess.run(["patch", "-p1", "--no-backup-if-mismatch", "-i", str(patch)], cwd=tmp_path,
                           capture_output=True, text=True)
        assert r.returncode == 0, (f, r.stdout, r.stderr)
    opts = (tmp_path / "cli/opts.rs").read_text()
    assert '"hip" => Ok(Device::Hip)' in opts
    run = (tmp_path / "cli/run.rs").read_text()
    assert "Device::Hip => serve(dir, Hip::new(0)" in run and run.count("Device::Hip =>") == 3
    lib_rs = (tmp_path / "model/lib.rs").read_text()
    assert "mod hip;" in lib_rs and "pub use hip::{Hip, HipModel};" in lib_rs
    assert "titania-hip-sys" in (tmp_path / "model/Cargo.toml").read_text()
    model = (tmp_path / "model/model.rs").read_text()
    body = model[model.index("fn run_batch("):model.index("pub struct State")]
    # The per-layer copies and norms now go through the extension.
    assert "d.copy(&mut s.xb, 0, &s.x, 0" not in body
    for m in EXTENSION_METHODS:
        if m != "argmax":
            assert f"d.{m}(" in body, m
    assert "self.device.argmax(&state.logits)" in model


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
