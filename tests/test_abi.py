"""The shared libraries load without a GPU and export every entry point their
headers declare: the C ABI (include/chimera_hip.h, include/chimera_workload.h)
from libchimera_hip.so and the C++ class Chimera::chimera_index (include/chimera/chimera_index.hpp)
from libchimera_core.so. No compute call is made."""
import ctypes
import re
import shutil
import subprocess
from pathlib import Path

import pytest

from chimera_amd import CORE_LIB, HIP_LIB, capi

ROOT = Path(__file__).resolve().parents[1]


def header_functions() -> list[str]:
    names = set()
    for h in sorted((ROOT / "include").glob("*.h")):
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        names.update(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][\w\s\*]*?\b(chimera_\w+)\s*\(", text, flags=re.M))
    return sorted(names)


def test_header_declares_the_expected_entry_points():
    names = header_functions()
    assert "chimera_search" in names and "chimera_build_index_device" in names
    assert "chimera_exact_maxsim_device" in names
    assert sorted(capi.EXPORTED) == names


def test_hip_library_exports_every_declared_function():
    lib = ctypes.CDLL(str(HIP_LIB))
    missing = [n for n in header_functions() if not hasattr(lib, n)]
    assert not missing, missing


def test_last_error_is_callable_without_a_device():
    lib = ctypes.CDLL(str(HIP_LIB))
    lib.chimera_last_error.restype = ctypes.c_char_p
    assert isinstance(lib.chimera_last_error(), bytes)


@pytest.mark.skipif(shutil.which("nm") is None, reason="binutils nm is not installed")
def test_core_library_exports_the_cpp_class():
    out = subprocess.run(["nm", "-DC", "--defined-only", str(CORE_LIB)], capture_output=True, text=True,
                         check=True).stdout
    for sym in ["Chimera::chimera_index::chimera_index()", "Chimera::chimera_index::~chimera_index()",
                "Chimera::chimera_index::build(", "Chimera::chimera_index::search(std::vector<float",
                "Chimera::chimera_index::search(float const*", "Chimera::chimera_index::search_batch(",
                "Chimera::chimera_index::save(", "Chimera::chimera_index::load("]:
        assert sym in out, sym
