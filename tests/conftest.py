import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)
GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def pytest_collection_modifyitems(config, items):
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:  # pragma: no cover
        has_gpu = False
    if has_gpu:
        return
    skip = pytest.mark.skip(reason="no GPU in this container")
    for it in items:
        if "gpu" in it.keywords:
            it.add_marker(skip)


@pytest.fixture(scope="session")
def R():
    from oracle import hif8_ref
    hif8_ref.build_lib()
    return hif8_ref


@pytest.fixture(scope="session")
def pkg():
    from __graft_entry__ import load_package
    return load_package()


@pytest.fixture(scope="session")
def golden():
    ex = np.load(os.path.join(GOLDEN, "hif8_bf16_exhaustive.npz"))
    sc = np.load(os.path.join(GOLDEN, "hif8_scale_bf16.npz"))
    c1 = np.load(os.path.join(GOLDEN, "c1_samples.npz"))
    import json
    with open(os.path.join(GOLDEN, "c1_digest.json")) as f:
        meta = json.load(f)
    return {"ex": ex, "scale": sc, "c1": c1, "c1_meta": meta}
