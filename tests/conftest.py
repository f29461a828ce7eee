import os
import sys

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


# Shapes of the reference test-suite (tests/test_dropkv_triton.py:80-83).
LLAMA_CFG = dict(B=1, Hq=32, Hkv=8, D=128)
QWEN_CFG = dict(B=1, Hq=14, Hkv=2, D=64)
BATCH2_CFG = dict(B=2, Hq=32, Hkv=8, D=128)
MHA_CFG = dict(B=1, Hq=8, Hkv=8, D=128)


def make_qkv(cfg, Lq, Lk=None, dtype=torch.bfloat16, seed=0, device="cpu", k_scale=None):
    """Seeded N(0,1) Q/K/V drawn on the CPU (so CPU and GPU see the same bytes)."""
    Lk = Lq if Lk is None else Lk
    g = torch.Generator().manual_seed(seed)
    B, Hq, Hkv, D = cfg["B"], cfg["Hq"], cfg["Hkv"], cfg["D"]
    Q = torch.randn(B, Hq, Lq, D, generator=g)
    K = torch.randn(B, Hkv, Lk, D, generator=g)
    V = torch.randn(B, Hkv, Lk, D, generator=g)
    if k_scale == "lognormal":
        s = torch.exp(torch.randn(B, Hkv, 1, D, generator=g))
        K = K * s
    return Q.to(dtype).to(device), K.to(dtype).to(device), V.to(dtype).to(device)


@pytest.fixture(scope="session")
def gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from dropkv_amd import _lib
    _lib.load()
    return torch.device("cuda:0")
