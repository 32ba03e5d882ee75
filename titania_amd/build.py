"""Build recipe for the hip device: compiles every HIP source under csrc/ for
gfx950 with hipcc and links them into titania_amd/libtitania_hip.so.

Run as `python -m titania_amd.build` or through __graft_entry__.build().
"""

from __future__ import annotations

import concurrent.futures as cf
import os
import re
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
OUT = PKG / "libtitania_hip.so"
OBJ = PKG / "_build"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-fvisibility=hidden",
    "-fvisibility-inlines-hidden",
    # Packed FP32 instructions stay off: hipcc would otherwise form them from
    # ordinary float code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Kernel arguments that lead a kernel's parameter list (scalars and
    # pointers, up to 16 dwords) arrive preloaded in SGPRs, so a kernel's first
    # loads need not wait on a fetch of its arguments.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-result",
    # Per-kernel resource remarks, read by _compile: no kernel here may use
    # scratch memory (a spill, or a local table the compiler failed to keep in
    # registers, turns a kernel's loads into slow, serialized ones).
    "-Rpass-analysis=kernel-resource-usage",
]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> tuple[Path, str]:
    obj = OBJ / (src.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(src), "-o", str(obj)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{r.stdout}\n{r.stderr}")
    scratch, kernel, notes, remark = [], None, [], False
    for line in r.stderr.splitlines():
        if "[-Rpass-analysis=kernel-resource-usage]" not in line:
            # A remark's source excerpt and caret follow it.
            if not (remark and re.match(r"\s*\d*\s*\|", line)):
                notes.append(line)
                remark = False
            continue
        remark = True
        if (m := re.search(r"Function Name: (\S+)", line)):
            kernel = m.group(1)
        elif (m := re.search(r"ScratchSize \[bytes/lane\]: (\d+)", line)) and int(m.group(1)):
            scratch.append(f"{kernel}: {m.group(1)} bytes a lane")
    if scratch:
        raise RuntimeError(f"kernels of {src.name} use scratch memory:\n" + "\n".join(scratch))
    return obj, "\n".join(notes)


SYNTH_SRC = PKG / "synth.c"
SYNTH_OUT = PKG / "libtitania_synth.so"


def build_synth() -> Path:
    """The host-side synthetic-weight generator (plain C, OpenMP)."""
    tmp = SYNTH_OUT.with_suffix(".so.tmp")
    cmd = ["gcc", "-O3", "-fPIC", "-shared", "-fopenmp", "-fvisibility=hidden", "-Wall",
           "-o", str(tmp), str(SYNTH_SRC), "-lm"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"gcc failed on synth.c:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, SYNTH_OUT)
    return SYNTH_OUT


def build(verbose: bool = False) -> Path:
    """Compiles all sources (always, as the build check expects) and links the library."""
    build_synth()
    OBJ.mkdir(exist_ok=True)
    srcs = sources()
    jobs = min(len(srcs), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4)), 16)
    with cf.ThreadPoolExecutor(max_workers=max(jobs, 1)) as ex:
        results = list(ex.map(_compile, srcs))
    objs = [o for o, _ in results]
    if verbose:
        for _, err in results:
            # hipcc's host pass does not know the packed-fp32 feature flag; that note is noise.
            lines = [l for l in err.splitlines() if l.strip() and "packed-fp32-ops" not in l]
            if lines:
                print("\n".join(lines), file=sys.stderr)
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(tmp, OUT)
    return OUT


if __name__ == "__main__":
    print(build(verbose=True))
