"""Build ``libavattn.so`` (the C-ABI HIP library) in-tree with hipcc for gfx950.

Usage: ``python -m avgen_amd.build`` (or ``__graft_entry__.build()``).  Each
``csrc/*.hip`` is compiled to an object under ``avgen_amd/_build/`` in
parallel, then linked into ``avgen_amd/libavattn.so``.  Always recompiles.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
INCLUDE = ROOT / "include"
BUILD = PKG / "_build"
LIB = PKG / "libavattn.so"
ARCH = "gfx950"

# Packed-fp32 VALU forms stay disabled (plain scalar fp32 code only).
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    """Return the hipcc executable (ROCm install or PATH)."""
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the avattn HIP library cannot be built")


def _compile(src: Path, extra: list[str]) -> Path:
    obj = BUILD / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature name; drop that
    # one harmless warning line and surface everything else.
    noise = "is not a recognized feature for this target"
    msg = "\n".join(line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{msg}")
    if msg.strip():
        print(msg, file=sys.stderr)
    return obj


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every kernel source and link the shared library; return its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    extra = list(extra_flags or [])
    if verbose:
        extra += ["-Rpass-analysis=kernel-resource-usage"]
    with ThreadPoolExecutor(max_workers=min(8, len(sources))) as pool:
        objs = list(pool.map(lambda s: _compile(s, extra), sources))
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}{proc.stderr}")
    # A kernel whose host-side launch stub was not emitted links fine but
    # fails at load time; refuse such a library here.
    nm = subprocess.run(["nm", "-D", "--undefined-only", str(tmp)], capture_output=True, text=True)
    missing = [line.split()[-1] for line in nm.stdout.splitlines() if "__device_stub__" in line]
    if missing:
        raise RuntimeError(f"link produced undefined kernel stubs (compiler host-pass issue): {missing[:4]}")
    os.replace(tmp, LIB)
    return LIB


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv)
    print(path)
