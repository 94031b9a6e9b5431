"""Build the gfx950 kernel layer in-tree with hipcc (no hipify, no JIT cache):

  libespalier_hip.so   the HIP kernels and the C ABI of include/espalier.h (dense.hip, dense_multi.hip, dense_tile.hip,
                       moe.hip, step.hip, abi.cpp)
  espalier_ext*.so     the torch extension module (binding.cpp, host code only), linked to libespalier_hip.so
  libespalier_probe.so bench.py --probes' measurement kernels (probe.hip), apart from the kernel layer

All land in the vllm_espalier package directory. Usage: python build.py [--jobs N] [--only lib|ext|probe]

--phase-trace builds, instead, a timing copy of the package under csrc/_phase/vllm_espalier (its Python files and both
libraries, compiled with ESP_PHASE_TRACE): esp_dense's and esp_dense_tile's workgroups record when each phase of the
launch starts (dense.hpp, dense_tile.hip), which bench.py --phase-trace reads. The product package is left as it is.
"""
from __future__ import annotations

import argparse
import os
import shutil
import subprocess
import sys
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

CSRC = Path(__file__).resolve().parent
PKG = CSRC.parent
REPO = PKG.parent.parent
BUILD = CSRC / "_build"
PHASE = CSRC / "_phase"
ARCH = os.environ.get("ESPALIER_OFFLOAD_ARCH", "gfx950")
LIB = PKG / "libespalier_hip.so"

HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
             "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-Wall", "-Wno-unused-function", "-Wno-unused-variable"]


def hipcc() -> str:
    for c in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if c and Path(c).exists():
            return c
    raise RuntimeError("hipcc not found: the gfx950 kernels need ROCm's hipcc")


def run(cmd: list[str]) -> None:
    p = subprocess.run(cmd, capture_output=True, text=True)
    # the host pass does not know the packed-fp32 feature; that warning is expected
    noise = "is not a recognized feature for this target"
    err = "\n".join(l for l in (p.stderr or "").splitlines() if noise not in l)
    if p.returncode != 0:
        raise RuntimeError(f"command failed ({p.returncode}): {' '.join(cmd)}\n{err}")
    if err.strip():
        print(err, file=sys.stderr)


def ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build_lib(jobs: int, incremental: bool = False, pkg: Path = PKG, build_dir: Path = BUILD,
              defines: tuple = ()) -> Path:
    build_dir.mkdir(parents=True, exist_ok=True)
    lib = pkg / "libespalier_hip.so"
    cc = hipcc()
    srcs = [CSRC / "dense.hip", CSRC / "dense_multi.hip", CSRC / "dense_tile.hip", CSRC / "moe.hip", CSRC / "step.hip", CSRC / "abi.cpp"]
    objs = [build_dir / (s.stem + ".o") for s in srcs]
    headers = [*CSRC.glob("*.hpp"), REPO / "include" / "espalier.h"]
    newest_header = max(h.stat().st_mtime for h in headers)

    def compile_one(pair):
        s, o = pair
        if incremental and o.exists() and o.stat().st_mtime > max(s.stat().st_mtime, newest_header):
            return                                       # object newer than its source and every header
        lang = ["-x", "hip"] if s.suffix == ".hip" else []
        run([cc, *HIP_FLAGS, *defines, *lang, "-c", str(s), "-o", str(o)])

    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(compile_one, zip(srcs, objs)))
    tmp = lib.with_suffix(".so.tmp")
    run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)])
    os.replace(tmp, lib)
    return lib


def build_probe() -> Path:
    BUILD.mkdir(exist_ok=True)
    cc = hipcc()
    out = PKG / "libespalier_probe.so"
    run([cc, *HIP_FLAGS, "-x", "hip", "-shared", str(CSRC / "probe.hip"), "-o", str(out) + ".tmp"])
    os.replace(str(out) + ".tmp", out)
    return out


def build_ext(pkg: Path = PKG) -> Path:
    import torch.utils.cpp_extension as ce
    import torch
    cc = hipcc()
    out = pkg / ("espalier_ext" + ext_suffix())
    inc = [f"-I{p}" for p in ce.include_paths()] + [f"-I{sysconfig.get_paths()['include']}"]
    libdirs = [f"-L{p}" for p in ce.library_paths()]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [cc, "-O2", "-std=c++17", "-fPIC", "-shared", str(CSRC / "binding.cpp"), *inc,
           "-DTORCH_EXTENSION_NAME=espalier_ext", "-DTORCH_API_INCLUDE_EXTENSION_H", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", "-Wno-unused-result", "-Wno-deprecated-declarations",
           *libdirs, f"-L{pkg}", "-lespalier_hip", "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu", "-ltorch_hip",
           "-ltorch_python", "-Wl,-rpath,$ORIGIN", "-o", str(out) + ".tmp"]
    run(cmd)
    os.replace(str(out) + ".tmp", out)
    return out


def build(jobs: int = 4, only: str | None = None, incremental: bool = False) -> None:
    if only in (None, "lib"):
        build_lib(jobs, incremental)
    if only in (None, "ext"):
        build_ext()
    if only in (None, "probe"):
        build_probe()


def build_phase(jobs: int = 4) -> Path:
    """The timing copy of the package (csrc/_phase/vllm_espalier), built with ESP_PHASE_TRACE."""
    dst = PHASE / "vllm_espalier"
    if dst.exists():
        shutil.rmtree(dst)
    dst.mkdir(parents=True)
    for f in PKG.glob("*.py"):
        shutil.copy2(f, dst / f.name)
    build_lib(jobs, pkg=dst, build_dir=PHASE / "_build", defines=("-DESP_PHASE_TRACE",))
    build_ext(pkg=dst)
    return dst


if __name__ == "__main__":
    ap = argparse.ArgumentParser()
    ap.add_argument("--jobs", type=int, default=4)
    ap.add_argument("--only", choices=["lib", "ext", "probe"])
    ap.add_argument("--incremental", action="store_true", help="skip objects newer than their source and every header")
    ap.add_argument("--phase-trace", action="store_true", help="build the timing copy of the package instead")
    a = ap.parse_args()
    if a.phase_trace:
        build_phase(a.jobs)
    else:
        build(a.jobs, a.only, a.incremental)
