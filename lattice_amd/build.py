"""Build recipe for libkcmm.so (gfx950) and the host-only check library.

    python -m lattice_amd.build            # build everything
    python -m lattice_amd.build --jobs 8

libkcmm.so: the C++ host runtime (pool_core.cpp, tiering.cpp, ffi.cpp; g++) plus the HIP
kernels (kernels/*.hip; hipcc --offload-arch=gfx950), linked with hipcc.
libkcmm_hostcheck.so: the same host runtime over a host-memory page backing
(tests/hostcheck), so CPU tests exercise the product's bookkeeping code.
Objects go to lattice_amd/_build/; the libraries are written in-tree.
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
BUILD = PKG / "_build"
LIB = PKG / "libkcmm.so"
HOSTCHECK_DIR = ROOT / "tests" / "hostcheck"
HOSTCHECK_LIB = HOSTCHECK_DIR / "libkcmm_hostcheck.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")
CXX = os.environ.get("CXX", "g++")

# -packed-fp32-ops: no v_pk_*_f32 in generated code.
HIP_FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-fPIC", "-std=c++17",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]
CXX_FLAGS = ["-O2", "-fPIC", "-std=c++17", "-Wall", "-Wextra", "-Wno-unused-parameter"]

HOST_SOURCES = ["pool_core.cpp", "tiering.cpp", "ffi.cpp", "tunables.cpp"]
HIP_SOURCES = ["kernels/backing.hip", "kernels/attn_decode.hip", "kernels/attn_prefill.hip",
               "kernels/kv_write.hip",
               "kernels/page_copy.hip", "kernels/gemm.hip", "kernels/gemm_tiled.hip",
               "kernels/glue.hip",
               "kernels/tier_copy.hip"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(l for l in proc.stdout.splitlines()
                    if "packed-fp32-ops' is not a recognized feature" not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out)


def _obj(src: str, tag: str) -> Path:
    return BUILD / tag / (src.replace("/", "_") + ".o")


def build_kcmm(jobs: int = 8) -> Path:
    """Compile and link lattice_amd/libkcmm.so."""
    (BUILD / "kcmm").mkdir(parents=True, exist_ok=True)
    cmds = []
    objs = []
    for s in HOST_SOURCES:
        o = _obj(s, "kcmm")
        cmds.append([CXX, *CXX_FLAGS, "-c", str(CSRC / s), "-o", str(o)])
        objs.append(o)
    for s in HIP_SOURCES:
        o = _obj(s, "kcmm")
        cmds.append([HIPCC, *HIP_FLAGS, "-c", str(CSRC / s), "-o", str(o)])
        objs.append(o)
    with cf.ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        list(ex.map(_run, cmds))
    tmp = LIB.with_suffix(".so.tmp")
    _run([HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
          *map(str, objs), "-Wl,--no-undefined"])
    os.replace(tmp, LIB)
    return LIB


def build_hostcheck() -> Path:
    """Host-only build of the pool runtime for the CPU test tier."""
    (BUILD / "hostcheck").mkdir(parents=True, exist_ok=True)
    srcs = [CSRC / s for s in HOST_SOURCES] + [HOSTCHECK_DIR / "host_device.cpp"]
    tmp = HOSTCHECK_LIB.with_suffix(".so.tmp")
    _run([CXX, *CXX_FLAGS, "-shared", "-o", str(tmp), *map(str, srcs), "-Wl,--no-undefined"])
    os.replace(tmp, HOSTCHECK_LIB)
    return HOSTCHECK_LIB


def build_all(jobs: int = 8) -> None:
    build_hostcheck()
    build_kcmm(jobs)


def main() -> None:
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("--clean", action="store_true")
    a = ap.parse_args()
    if a.clean and BUILD.exists():
        shutil.rmtree(BUILD)
    build_all(a.jobs)
    print(f"built {LIB} and {HOSTCHECK_LIB}")


if __name__ == "__main__":
    main()
