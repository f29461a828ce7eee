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


# ---------------------------------------------------------------------------
# Golden fixtures (tests/golden/dropkv_golden.npz, written by make_golden.py)
# ---------------------------------------------------------------------------
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "dropkv_golden.npz")


def _bf16_from_bits(u):
    import numpy as np
    return torch.from_numpy((u.astype(np.uint32) << 16).view(np.float32).copy()).to(torch.bfloat16)


def golden_names():
    import numpy as np
    with np.load(GOLDEN) as z:
        return sorted({k.split("/")[0] for k in z.files})


def golden_case(name):
    """Inputs as bf16 tensors (q is the stored query tail) and float64 /
    float32 / int64 expectations of one golden case."""
    import numpy as np
    with np.load(GOLDEN) as z:
        d = {k.split("/", 1)[1]: z[k] for k in z.files if k.startswith(name + "/")}
    out = {"meta": [int(x) for x in d["meta"]], "ratio": float(d["ratio"])}
    out["q"], out["k"], out["v"] = (_bf16_from_bits(d[x]) for x in ("q_tail", "k", "v"))
    for key in ("exact", "bf16p", "deployed"):
        if key in d:
            out[key] = torch.from_numpy(d[key].copy())
    if "bf16p" in d:
        out["bf16p_np"] = d["bf16p"]
    for key in ("pooled_bf16p", "pooled_deployed"):
        if key in d:
            out[key] = torch.from_numpy(d[key].copy())
    for key in ("keep_idx_bf16p", "keep_idx_deployed"):
        if key in d:
            out[key] = torch.from_numpy(d[key].copy())
    return out
