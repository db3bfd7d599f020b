"""Build the MI355X hot-path libraries in-tree.

  soinfer/libsoinfer_hip.so   hipcc --offload-arch=gfx950: every HIP kernel and
                              the C ABI declared in include/soinfer_amd.h
  soinfer/_C<ext>.so          the torch binding (csrc/bindings.cpp), compiled
                              with the host C++ compiler against torch's
                              headers and linked to libsoinfer_hip.so

Both land inside the package so they travel with the source tree. Objects are
rebuilt only when a source or header is newer (force=True rebuilds all).
Run: python sparse-offload-infer_amd/build.py [--force]
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
CSRC = PKG_ROOT / "csrc"
SOINFER = PKG_ROOT / "soinfer"
REPO = PKG_ROOT.parent
INCLUDE = REPO / "include"
BUILD = PKG_ROOT / "_build"

ARCH = os.environ.get("SOINFER_HIP_ARCH", "gfx950")
HIP_SOURCES = ["decoder.hip", "capi.hip", "gemv_int4.hip", "gemv_int8.hip", "topk_select.hip", "dip_descriptors.hip",
               "sparse_down.hip", "decode_attention.hip", "dip_dense_down.hip", "grid_sync.hip"]
HIP_LIB = SOINFER / "libsoinfer_hip.so"
EXT_LIB = SOINFER / ("_C" + sysconfig.get_config_var("EXT_SUFFIX"))

# Packed-fp32 VALU forms are disabled for all device code (the compiler
# otherwise forms them from ordinary float code).
HIPCC_FLAGS = [f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Xclang", "-target-feature", "-Xclang",
               "-packed-fp32-ops", "-munsafe-fp-atomics", "-Wall", "-Wno-unused-function"]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the soinfer HIP library cannot be built")


def _headers() -> list[Path]:
    return sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def _stale(target: Path, deps: list[Path]) -> bool:
    if not target.exists():
        return True
    t = target.stat().st_mtime
    return any(d.stat().st_mtime > t for d in deps)


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(" ".join(cmd) + "\n" + r.stdout + r.stderr)
        raise RuntimeError(f"build step failed: {cmd[0]} ... {cmd[-1]}")


def build_hip(force: bool = False, jobs: int = 8) -> Path:
    BUILD.mkdir(exist_ok=True)
    hipcc = _hipcc()
    headers = _headers()
    objs = []
    todo = []
    for src in HIP_SOURCES:
        s = CSRC / src
        o = BUILD / (src + ".o")
        objs.append(o)
        if force or _stale(o, [s, *headers, Path(__file__)]):
            todo.append([hipcc, *HIPCC_FLAGS, "-c", str(s), "-o", str(o)])
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, todo))
    if force or todo or _stale(HIP_LIB, objs):
        tmp = HIP_LIB.with_suffix(".so.tmp")
        _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs),
              "-Wl,-soname,libsoinfer_hip.so"])
        os.replace(tmp, HIP_LIB)
    return HIP_LIB


def build_ext(force: bool = False) -> Path:
    import torch
    from torch.utils import cpp_extension

    BUILD.mkdir(exist_ok=True)
    src = CSRC / "bindings.cpp"
    if not (force or _stale(EXT_LIB, [src, *_headers(), HIP_LIB, Path(__file__)])):
        return EXT_LIB
    incs = [*cpp_extension.include_paths(), sysconfig.get_paths()["include"], "/opt/rocm/include"]
    libdirs = cpp_extension.library_paths()
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cxx = os.environ.get("CXX", "g++")
    tmp = EXT_LIB.with_suffix(".tmp.so")
    cmd = [cxx, "-O2", "-std=c++17", "-fPIC", "-shared", "-w", str(src), "-o", str(tmp),
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1", "-DHIPBLAS_V2", "-DTORCH_EXTENSION_NAME=_C",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           *[f"-I{p}" for p in incs], *[f"-L{p}" for p in libdirs], f"-L{SOINFER}",
           "-lsoinfer_hip", "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
           "-Wl,-rpath,$ORIGIN", *[f"-Wl,-rpath,{p}" for p in libdirs]]
    _run(cmd)
    os.replace(tmp, EXT_LIB)
    return EXT_LIB


def build(force: bool = False) -> tuple[Path, Path]:
    hip = build_hip(force)
    ext = build_ext(force)
    return hip, ext


if __name__ == "__main__":
    force = "--force" in sys.argv
    for p in build(force):
        print(p)
