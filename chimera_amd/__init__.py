"""Chimera for MI355X: late-interaction (multi-vector) retrieval with the
reference's C++/Python API and index files, scored by gfx950 HIP kernels.

Native parts (built in-tree by chimera_amd.build):
  libchimera_hip.so   kernels + C ABI (include/chimera_hip.h)
  libchimera_core.so  host C++ (index files, codec, CPU build, chimera_index)
  chimera*.so         pybind11 module `chimera` (ChimeraIndex)
"""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
HIP_LIB = PKG_DIR / "libchimera_hip.so"
CORE_LIB = PKG_DIR / "libchimera_core.so"


def load_module():
    """Imports the pybind11 module `chimera` from this package directory.

    Raises ImportError when the native build is missing; there is no
    pure-Python fallback.
    """
    if str(PKG_DIR) not in sys.path:
        sys.path.insert(0, str(PKG_DIR))
    return importlib.import_module("chimera")


def __getattr__(name):
    if name == "ChimeraIndex":
        return load_module().ChimeraIndex
    raise AttributeError(name)
