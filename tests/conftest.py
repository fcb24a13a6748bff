import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "chimera_amd"))
GOLDEN = ROOT / "tests" / "golden"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def _ensure_built():
    from chimera_amd import CORE_LIB, HIP_LIB, PKG_DIR

    mods = list(PKG_DIR.glob("chimera*.so"))
    if not (HIP_LIB.exists() and CORE_LIB.exists() and mods):
        from chimera_amd import build

        build.build()
    from oracle import oracle as orc

    orc.ensure_built()


_ensure_built()


@pytest.fixture(scope="session")
def chimera_mod():
    from chimera_amd import load_module

    return load_module()


@pytest.fixture(scope="session")
def golden():
    return dict(np.load(GOLDEN / "reference_host.npz"))


@pytest.fixture(scope="session")
def small_workload():
    """2,000 docs (~175k tokens), 512-centre mixture, 16 queries."""
    from chimera_amd import synthetic

    return synthetic.generate(num_docs=2000, num_centres=512, sigma=0.15, nq=16, seed=11)


@pytest.fixture(scope="session")
def small_index(chimera_mod, small_workload):
    w = small_workload
    return chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 1024, 4)


@pytest.fixture(scope="session")
def tiny_workload():
    """120 docs of 1..24 tokens: small enough for pure-Python brute force."""
    from chimera_amd import synthetic

    rng = np.random.default_rng(5)
    centres = synthetic.unit_centres(rng, 16, 128)
    lens = rng.integers(1, 25, size=120).astype(np.int32)
    emb = synthetic.mixture_tokens(rng, centres, int(lens.sum()), 0.15)
    q, t = synthetic.make_queries(rng, emb, lens, 4)
    return synthetic.Workload(emb, lens, q, t)


@pytest.fixture(scope="session")
def tiny_index(chimera_mod, tiny_workload):
    w = tiny_workload
    return chimera_mod._build_index(w.embeddings, w.doc_lens.tolist(), 48, 3)


def gpu_available() -> bool:
    if os.environ.get("CHIMERA_FORCE_NO_GPU"):
        return False
    try:
        from chimera_amd import capi

        return capi.lib().chimera_device_count() > 0
    except Exception:
        return False
