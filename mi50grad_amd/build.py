"""Build recipe for libkvattn.so (gfx950) — run ``python -m mi50grad_amd.build``.

hipcc compiles the kernels (``csrc/k_*.hip``) for gfx950 only; g++ compiles the
host side (``csrc/kva_host.cpp``) against the HIP runtime API; hipcc links the
shared library in-tree (``mi50grad_amd/libkvattn.so``) so it travels with the
source tree.  The build always recompiles: it is the "does it build" check.

``--sanitize`` builds ``libkvattn_san.so`` instead: the same kernels, the host
side under AddressSanitizer and UndefinedBehaviorSanitizer (g++ only; no GPU
code is instrumented).  The CPU suite runs against it with

    ASAN_OPTIONS=detect_leaks=0 LD_PRELOAD=$(gcc -print-file-name=libasan.so) \
        KVA_LIB=mi50grad_amd/libkvattn_san.so python -m pytest tests -m "not gpu"
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
ROOT = PKG.parent
INCLUDE = ROOT / "include"
OUT = PKG / "libkvattn.so"
OUT_SAN = PKG / "libkvattn_san.so"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = "gfx950"

# Packed-FP32 VALU ops stay disabled (hand-written or compiler-made).
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC", "-Wall",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", f"-I{INCLUDE}", f"-I{CSRC}",
]
HOST_FLAGS = [
    "-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
    "-D__HIP_PLATFORM_AMD__", f"-I{ROCM / 'include'}", f"-I{INCLUDE}", f"-I{CSRC}",
]
SAN_FLAGS = ["-fsanitize=address,undefined", "-fno-sanitize-recover=undefined", "-fno-omit-frame-pointer", "-g"]


def _run(cmd: list[str]) -> None:
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"build step failed: {' '.join(cmd)}\n{res.stdout}\n{res.stderr}")


def build(verbose: bool = False, sanitize: bool = False) -> Path:
    """Compile every kernel and the host side, link libkvattn.so (sanitize:
    libkvattn_san.so, host side instrumented); return its path."""
    objdir = PKG / ("_build_san" if sanitize else "_build")
    out = OUT_SAN if sanitize else OUT
    if objdir.exists():
        shutil.rmtree(objdir)
    objdir.mkdir()
    jobs = []
    for src in sorted(CSRC.glob("k_*.hip")):
        jobs.append([HIPCC, *HIP_FLAGS, "-c", str(src), "-o", str(objdir / (src.stem + ".o"))])
    jobs.append(["g++", *HOST_FLAGS, *(SAN_FLAGS if sanitize else []), "-c", str(CSRC / "kva_host.cpp"),
                 "-o", str(objdir / "kva_host.o")])
    with cf.ThreadPoolExecutor(max_workers=min(8, len(jobs))) as ex:
        for cmd, fut in zip(jobs, [ex.submit(_run, j) for j in jobs]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    objs = sorted(str(p) for p in objdir.glob("*.o"))
    tmp = out.with_suffix(".so.tmp")
    if sanitize:  # the instrumented host object needs the sanitizer runtimes: link with g++
        _run(["g++", "-shared", *SAN_FLAGS, "-o", str(tmp), *objs,
              f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    else:
        _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *objs,
              f"-L{ROCM / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{ROCM / 'lib'}"])
    os.replace(tmp, out)
    shutil.rmtree(objdir)
    return out


if __name__ == "__main__":
    path = build(verbose="-v" in sys.argv, sanitize="--sanitize" in sys.argv)
    print(f"built {path}")
