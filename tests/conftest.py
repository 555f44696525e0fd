import json
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "qwendecisioncore.jl_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def ramp(fn, shape, scale=1.0):
    """Closed-form inputs of the reference's op tests: fn(1), fn(2), ... in fp32."""
    n = int(np.prod(shape))
    return (fn(np.arange(1, n + 1, dtype=np.float32)) * np.float32(scale)).astype(np.float32).reshape(shape)


def normwise(a, b):
    """Relative error in the sense of Julia's isapprox on arrays:
    norm(a-b) / max(norm(a), norm(b))."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = max(np.linalg.norm(a), np.linalg.norm(b))
    return 0.0 if den == 0 else float(np.linalg.norm(a - b) / den)


def isapprox(a, b, atol, rtol):
    """Julia ``isapprox(a, b; atol, rtol)`` on arrays (normwise)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return np.linalg.norm(a - b) <= max(atol, rtol * max(np.linalg.norm(a), np.linalg.norm(b)))


@pytest.fixture(scope="session")
def native_fixture():
    d = np.load(os.path.join(GOLDEN, "native_fixture.npz"), allow_pickle=False)
    from oracle import forward
    cfg = forward.config_from_text_config(json.loads(str(d["config_json"]))["text_config"])
    weights = {k[2:]: d[k] for k in d.files if k.startswith("w/")}
    cases = []
    for name in d["case_names"]:
        label = str(name).split(":")[0]
        cases.append((str(name), d[f"case/{label}/ids"], d[f"case/{label}/mask"],
                      d[f"case/{label}/logits"]))
    return {"cfg": cfg, "weights": weights, "readout": d["readout"], "cases": cases}


@pytest.fixture(scope="session")
def transformers_golden():
    return dict(np.load(os.path.join(GOLDEN, "transformers_golden.npz"), allow_pickle=False))
