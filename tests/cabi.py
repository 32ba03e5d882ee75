"""Signatures of the C ABI as the header, the ctypes binding and the Rust FFI
crate state them, reduced to comparable kinds (ptr, size, i32, i64, u32, u64,
f32, void), for tests/test_abi.py."""

from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "titania_hip.h"
TEST_HEADER = ROOT / "include" / "titania_hip_test.h"
RUST_SYS = ROOT / "titania_amd" / "rust" / "hip-sys" / "lib.rs"

_C_SCALARS = {"int": "i32", "size_t": "size", "float": "f32", "uint32_t": "u32", "uint64_t": "u64",
              "int64_t": "i64", "void": "void"}
_RUST_SCALARS = {"i32": "i32", "c_int": "i32", "usize": "size", "f32": "f32", "u32": "u32", "u64": "u64",
                 "i64": "i64"}


def _c_kind(decl: str) -> str:
    decl = decl.strip()
    if "*" in decl:
        return "ptr"
    words = [w for w in re.split(r"\s+", decl) if w and w not in ("const", "TH_API")]
    # Last word is the parameter name when there are two or more.
    base = words[0] if len(words) == 1 else words[-2]
    return _C_SCALARS[base]


def header_signatures(path: Path = HEADER) -> dict[str, tuple[str, list[str]]]:
    """name -> (return kind, [argument kinds]) of every TH_API declaration."""
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    out = {}
    for m in re.finditer(r"^TH_API\s+([^;]*?)\b(th_\w+)\s*\(([^)]*)\)\s*;", text, re.M | re.S):
        ret, name, args = m.group(1), m.group(2), m.group(3).strip()
        kinds = [] if args in ("", "void") else [_c_kind(a) for a in args.split(",")]
        out[name] = (_c_kind(ret + " x"), kinds)
    return out


def _ctype_kind(t) -> str:
    if t is None:
        return "void"
    if t in (C.c_void_p, C.c_char_p) or (isinstance(t, type) and issubclass(t, C._Pointer)):
        return "ptr"
    return {C.c_int: "i32", C.c_size_t: "size", C.c_float: "f32", C.c_uint32: "u32", C.c_uint64: "u64",
            C.c_int64: "i64"}[t]


def ctypes_signatures(table: dict) -> dict[str, tuple[str, list[str]]]:
    """The ctypes table's signatures. On this platform ctypes.c_size_t is
    ctypes.c_uint64 itself, so both read as "u64"; compare them with
    as_ctypes_kinds() applied to the header's."""
    return {name: (_ctype_kind(res), [_ctype_kind(a) for a in args]) for name, (res, args) in table.items()}


def as_ctypes_kinds(sig: tuple[str, list[str]]) -> tuple[str, list[str]]:
    """A header signature with size_t folded into u64 where ctypes cannot tell
    them apart (LP64: both are 64-bit unsigned)."""
    fold = (lambda k: "u64" if k == "size" else k) if C.c_size_t is C.c_uint64 else (lambda k: k)
    return fold(sig[0]), [fold(k) for k in sig[1]]


def _rust_kind(t: str) -> str:
    t = t.strip()
    if t.startswith("*"):
        return "ptr"
    return _RUST_SCALARS[t]


def rust_signatures(path: Path = RUST_SYS) -> dict[str, tuple[str, list[str]]]:
    """name -> (return kind, [argument kinds]) of the functions in the crate's
    `extern "C"` block."""
    text = path.read_text()
    block = re.search(r'extern\s+"C"\s*\{(.*?)\n\}', text, re.S).group(1)
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for m in re.finditer(r"pub\s+fn\s+(th_\w+)\s*\(([^)]*)\)\s*(->\s*([^;]+))?;", block, re.S):
        name, args, ret = m.group(1), m.group(2).strip(), m.group(4)
        kinds = []
        if args:
            for a in args.split(","):
                if a.strip():
                    kinds.append(_rust_kind(a.split(":", 1)[1]))
        out[name] = ("void" if ret is None else _rust_kind(ret), kinds)
    return out
