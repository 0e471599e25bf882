import json
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) to run")


@pytest.fixture(scope="session")
def kat():
    with open(os.path.join(GOLDEN, "reference_kat.json")) as f:
        return json.load(f)


@pytest.fixture(scope="session")
def hip_device():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test selected but no HIP device is visible")
    return torch.device("cuda:0")


def seeded_kv(shape, seed, kind, outlier_axis=-1):
    """Seeded synthetic K/V with the benchmark outlier pattern, made on the CPU.

    kind="key":   N(0,1), 4 fixed channels (last axis) scaled x10.
    kind="value": N(0,1), round(2% of the token axis) scaled x8.
    Generated with a CPU torch.Generator so CPU and GPU see identical bits.
    """
    import torch
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g, dtype=torch.float32)
    if kind == "key":
        D = shape[-1]
        ch = torch.randperm(D, generator=g)[:min(4, D)]
        x[..., ch] *= 10.0
    elif kind == "value":
        T = shape[-2]
        n = max(1, round(0.02 * T))
        tok = torch.randperm(T, generator=g)[:n]
        x[..., tok, :] *= 8.0
    return x
