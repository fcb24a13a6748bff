"""Builds the native parts of chimera_amd in-tree.

  chimera_amd/libchimera_hip.so   gfx950 HIP kernels + the C ABI (include/chimera_hip.h)
  chimera_amd/libchimera_core.so  host C++: codec, index files, CPU index build,
                                  Chimera::chimera_index (include/chimera/chimera_index.hpp)
  chimera_amd/chimera*.so         pybind11 module `chimera` (ChimeraIndex)
  chimera_amd/chimera_search      the search command (gpu_search's flags and report lines)

Compilers are driven directly (hipcc, g++); every call rebuilds.
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
INC = ROOT / "include"
HIP_SRC = PKG / "csrc" / "hip"
HOST_SRC = PKG / "csrc" / "host"
PY_SRC = PKG / "csrc" / "python"
APP_SRC = PKG / "csrc" / "apps"
OBJ = PKG / "_obj"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
CXX = os.environ.get("CXX", "g++")
ARCH = os.environ.get("CHIMERA_OFFLOAD_ARCH", "gfx950")

HIP_FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed FP32 instructions are disabled for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics", "-ffp-contract=off",
    # matrix-core accumulators in ordinary VGPRs: the epilogues read them
    # without v_accvgpr_read copies
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    f"-I{INC}", f"-I{HIP_SRC}",
]
HOST_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-march=x86-64-v3", "-ffp-contract=off", "-fopenmp", f"-I{INC}", f"-I{HOST_SRC}"]


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines()
                    if "packed-fp32-ops" not in line and "not a recognized feature" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"build command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")


def _hip_objects(jobs: int) -> list[Path]:
    OBJ.mkdir(exist_ok=True)
    srcs = sorted(HIP_SRC.glob("*.hip"))
    objs = [OBJ / (s.stem + ".o") for s in srcs]
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_run, [HIPCC, *HIP_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in zip(srcs, objs)]
        for f in futs:
            f.result()
    return objs


def ext_suffix() -> str:
    return sysconfig.get_config_var("EXT_SUFFIX") or ".so"


def build(jobs: int | None = None, verbose: bool = False) -> None:
    jobs = jobs or min(16, os.cpu_count() or 4)
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    objs = _hip_objects(jobs)
    hip_so = PKG / "libchimera_hip.so"
    _run([HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *map(str, objs), "-o", str(hip_so)])

    core_so = PKG / "libchimera_core.so"
    host_srcs = sorted(HOST_SRC.glob("*.cpp"))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        host_objs = [OBJ / (s.stem + ".host.o") for s in host_srcs]
        futs = [ex.submit(_run, [CXX, *HOST_FLAGS, "-c", str(s), "-o", str(o)]) for s, o in zip(host_srcs, host_objs)]
        for f in futs:
            f.result()
    _run([CXX, "-shared", "-fopenmp", *map(str, host_objs), "-o", str(core_so), f"-L{PKG}", "-lchimera_hip",
          "-Wl,-rpath,$ORIGIN", "-L/opt/rocm/lib", "-lamdhip64", "-Wl,-rpath,/opt/rocm/lib"])

    # the search command (chimera_search), linked against both libraries
    _run([CXX, *HOST_FLAGS, str(APP_SRC / "chimera_search.cpp"), "-o", str(PKG / "chimera_search"), f"-L{PKG}",
          "-lchimera_core", "-lchimera_hip", "-Wl,-rpath,$ORIGIN"])

    import pybind11  # noqa: WPS433

    py_inc = sysconfig.get_paths()["include"]
    mod = PKG / ("chimera" + ext_suffix())
    _run([CXX, *HOST_FLAGS, "-shared", f"-I{pybind11.get_include()}", f"-I{py_inc}", str(PY_SRC / "bindings.cpp"),
          "-o", str(mod), f"-L{PKG}", "-lchimera_core", "-lchimera_hip", "-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {hip_so.name}, {core_so.name}, chimera_search, {mod.name}")


def build_oracle() -> None:
    """Builds oracle/liboracle.so and, where the reference tree exists, oracle/_ref."""
    _run(["make", "-s", "-B", "-C", str(ROOT / "oracle"), "all"])


if __name__ == "__main__":
    build(verbose=True)
    if "--oracle" in sys.argv:
        build_oracle()
