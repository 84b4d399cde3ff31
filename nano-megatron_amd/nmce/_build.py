"""Compile ``libnmce.so`` (the gfx950 HIP kernels and their C ABI) in-tree.

    python -m nmce._build          # from nano-megatron_amd/, or
    python -c "import __graft_entry__ as g; g.build()"   # from the repo root

Every source is compiled to an object in parallel with ``hipcc`` for gfx950,
then linked into ``nmce/libnmce.so``. No GPU is needed: hipcc cross-compiles.
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys

PKG_DIR = pathlib.Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent  # nano-megatron_amd/
REPO_DIR = PROJECT_DIR.parent
CSRC_DIR = PROJECT_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PROJECT_DIR / "_build"
LIB_PATH = PKG_DIR / "libnmce.so"

SOURCES = ["nmce_ce.hip", "nmce_lmhead.hip"]

ARCH = "gfx950"

# -packed-fp32-ops off: no v_pk_{add,mul,fma}_f32 in the device code.
# Code object v5 loads under every ROCm runtime this library may meet (the
# torch wheel bundles its own HIP runtime).
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
    f"-I{INCLUDE_DIR}",
    f"-I{CSRC_DIR}",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found; a ROCm toolchain is required to build libnmce")
    return path


def _run(cmd: list[str], verbose: bool) -> subprocess.Popen:
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def _noise(line: str) -> bool:
    # hipcc forwards -target-feature to the host pass, which does not know it.
    return "packed-fp32-ops" in line and "not a recognized feature" in line


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every source and link ``libnmce.so``; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objects = []
    for src in SOURCES:
        obj = BUILD_DIR / (pathlib.Path(src).stem + ".o")
        objects.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(CSRC_DIR / src), "-o", str(obj)]
        procs.append((src, _run(cmd, verbose)))
    failed = []
    for src, proc in procs:
        out, _ = proc.communicate()
        text = "\n".join(l for l in out.splitlines() if not _noise(l))
        if text.strip() and (verbose or proc.returncode):
            print(text, file=sys.stderr)
        if proc.returncode:
            failed.append(src)
    if failed:
        raise RuntimeError(f"hipcc failed for {failed}")
    tmp = LIB_PATH.with_suffix(".so.tmp")
    link = [cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = _run(link, verbose)
    out, _ = proc.communicate()
    if proc.returncode:
        print(out, file=sys.stderr)
        raise RuntimeError("linking libnmce.so failed")
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
