"""Compile ``libnmce.so`` (the gfx950 HIP kernels and their C ABI) and the
``_nmce_autograd`` extension (the one-pass loss's autograd node, host C++ over
that ABI) in-tree.

    python -m nmce._build          # from nano-megatron_amd/, or
    python -c "import __graft_entry__ as g; g.build()"   # from the repo root

Every source is compiled to an object in parallel with ``hipcc`` (gfx950 for
the kernels), then the kernels are linked into ``nmce/libnmce.so`` and the
extension into ``nmce/_nmce_autograd<EXT_SUFFIX>`` against it and torch. No
GPU is needed: hipcc cross-compiles.
"""

from __future__ import annotations

import os
import pathlib
import shutil
import subprocess
import sys
import sysconfig

PKG_DIR = pathlib.Path(__file__).resolve().parent
PROJECT_DIR = PKG_DIR.parent  # nano-megatron_amd/
REPO_DIR = PROJECT_DIR.parent
CSRC_DIR = PROJECT_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = PROJECT_DIR / "_build"
LIB_PATH = PKG_DIR / "libnmce.so"

SOURCES = ["nmce_ce.hip", "nmce_lmhead.hip"]
EXT_SOURCE = "nmce_autograd.cpp"
EXT_NAME = "_nmce_autograd"
EXT_PATH = PKG_DIR / (EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))

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


def _ext_flags() -> tuple[list[str], list[str]]:
    """Compile and link flags of the autograd extension: torch's and Python's
    headers, torch's libraries, libnmce.so found next to the extension."""
    from torch.utils import cpp_extension
    import torch
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], str(INCLUDE_DIR)]
    cflags = ["-O2", "-std=c++17", "-fPIC", "-Wall", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
              f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
              *[f"-I{p}" for p in incs]]
    lflags = [*[f"-L{p}" for p in cpp_extension.library_paths()], f"-L{PKG_DIR}", "-lnmce",
              "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_python",
              "-Wl,-rpath,$ORIGIN"]
    return cflags, lflags


def build(verbose: bool = False) -> pathlib.Path:
    """Compile every source, link ``libnmce.so`` and the autograd extension;
    returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    cc = hipcc()
    procs = []
    objects = []
    for src in SOURCES:
        obj = BUILD_DIR / (pathlib.Path(src).stem + ".o")
        objects.append(obj)
        cmd = [cc, *HIPCC_FLAGS, "-c", str(CSRC_DIR / src), "-o", str(obj)]
        procs.append((src, _run(cmd, verbose)))
    ext_cflags, ext_lflags = _ext_flags()
    ext_obj = BUILD_DIR / (pathlib.Path(EXT_SOURCE).stem + ".o")
    procs.append((EXT_SOURCE, _run([cc, *ext_cflags, "-c", str(CSRC_DIR / EXT_SOURCE), "-o",
                                    str(ext_obj)], verbose)))
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
    tmp = EXT_PATH.with_name(EXT_PATH.name + ".tmp")
    proc = _run([cc, "-shared", "-fPIC", "-o", str(tmp), str(ext_obj), *ext_lflags], verbose)
    out, _ = proc.communicate()
    if proc.returncode:
        print(out, file=sys.stderr)
        raise RuntimeError(f"linking {EXT_PATH.name} failed")
    os.replace(tmp, EXT_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
