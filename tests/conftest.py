import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
GOLDEN = Path(__file__).resolve().parent / "golden"
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


def load_forward_cases():
    """Cases of tests/golden/forward_small.npz as dicts."""
    data = np.load(GOLDEN / "forward_small.npz", allow_pickle=False)
    names = sorted({k.split("/")[0] for k in data.files})
    cases = []
    for name in names:
        M, K, N, nb, with_bias = (int(v) for v in data[f"{name}/meta"])
        branches = []
        for i in range(nb):
            b = {key: data[f"{name}/b{i}/{key}"] for key in ("v_sign", "u_sign", "g", "l", "h")}
            b["R"] = int(b["v_sign"].shape[0])
            branches.append(b)
        cases.append({
            "name": name, "M": M, "K": K, "N": N, "x": data[f"{name}/x"], "branches": branches,
            "bias": data[f"{name}/bias"] if with_bias else None, "y": data[f"{name}/y"],
        })
    return cases


@pytest.fixture(scope="session")
def forward_cases():
    return load_forward_cases()


@pytest.fixture(scope="session")
def gpu():
    """The GPU device; skips when no GPU is visible."""
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    import littlebit_amd._lib as L
    L.load()  # raises if the HIP library was not built
    return torch.device("cuda:0")
