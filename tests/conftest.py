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


# ---------------------------------------------------------------------------
# Score bars that bind at full size
# ---------------------------------------------------------------------------
def binding_keys(ref, pooled_ref, keep, frac=0.1):
    """Keys whose reference score is at least ``frac`` times the row's keep
    threshold (the keep-th largest pooled, protected reference value): the
    keys whose scores can move the selection.  At full size almost every
    other key scores far below any absolute tolerance (scores scale like
    p^2 with p ~ 1/Lk), so a bar over all keys binds on almost nothing."""
    T = torch.topk(pooled_ref.double(), keep, dim=-1).values[..., -1:]
    return ref.double() >= frac * T


def assert_binding_scores(got, ref, pooled_ref, keep, Qt, K, V, W, p_round, max_rel, rel_bar, frac_above,
                          frac=0.1, excuse_sinks=True, max_arbitrated=4096, bracket=None):
    """Relative bars on the binding keys: every one within ``max_rel`` and
    fewer than ``frac_above`` of them beyond ``rel_bar``.

    A key beyond ``rel_bar`` against the float32 reference is arbitrated in
    float64.  With p rounded (``p_round``), by the oracle's
    ``dropkv_score_bracket``: the interval of values a float32 evaluation of
    the formula can return (p off by its float32 error before the rounding,
    which can flip it to the neighbouring bf16 value; y and the expansion
    off by their float32 rounding); its error is its distance to that
    interval, relative to the float64 score.  Keys within ``max_rel`` of
    their bracket but of neither the float32 reference nor the float64
    score (attention sinks, p ~ 1: no float32 evaluation determines them)
    are counted as sinks and must stay under 1e-3 of the row, and need
    ``excuse_sinks``.  Without p
    rounding the arbiter is the float64 score alone (``dropkv_scores_fp64``).
    ``bracket`` may hold precomputed (score, lo, hi) [B, Hkv, Lk] float64.
    Returns (binding keys, worst relative error after arbitration, keys
    beyond rel_bar, sink-excused keys)."""
    from oracle import dropkv_ref as R
    got, ref = got.double().cpu(), ref.double().cpu()
    sel = binding_keys(ref, pooled_ref.cpu(), keep, frac)
    rel = torch.where(sel, (got - ref).abs() / ref.abs().clamp_min(1e-300), torch.zeros_like(ref))
    B, Hkv, Lk = ref.shape
    g = Qt.shape[1] // Hkv
    worst, n_above, n_excused = 0.0, 0, 0
    for b in range(B):
        for h in range(Hkv):
            r = rel[b, h]
            keys = torch.nonzero(r > rel_bar).flatten()
            assert keys.numel() <= max_arbitrated, ((b, h), keys.numel(), float(r.max()))
            best = r.clone()
            if keys.numel():
                gk = got[b, h, keys]
                qh = Qt[b:b + 1, h * g:(h + 1) * g].cpu()
                kh, vh = K[b:b + 1, h:h + 1].cpu(), V[b:b + 1, h:h + 1].cpu()
                if p_round is None:
                    s64 = R.dropkv_scores_fp64(qh, kh, vh, W, keys=keys)[0, 0]
                    lo = hi = s64
                elif bracket is not None:
                    s64, lo, hi = (x[b, h, keys] for x in bracket)
                else:
                    s64, lo, hi = (x[0, 0] for x in R.dropkv_score_bracket(qh, kh, vh, W, p_round=p_round,
                                                                             keys=keys))
                scale = s64.abs().clamp_min(1e-300)
                dist = torch.where(gk < lo, lo - gk, torch.where(gk > hi, gk - hi, torch.zeros_like(gk))) / scale
                e64 = (gk - s64).abs() / scale
                best[keys] = torch.minimum(r[keys], dist)
                # within max_rel of its bracket but of neither evaluation: a
                # score the float32 formula does not determine (a sink)
                sink = (best[keys] <= max_rel) & (torch.minimum(r[keys], e64) > max_rel)
                row_sinks = int(sink.sum())
                if row_sinks:
                    assert excuse_sinks, ((b, h), keys[sink][:8].tolist())
                assert row_sinks <= 1e-3 * Lk, ((b, h), row_sinks)
                n_excused += row_sinks
            worst = max(worst, float(best.max()))
            above = torch.nonzero(best > rel_bar).flatten()
            n_above += int(above.numel())
            for key in above[:8].tolist():
                print(f"  beyond {rel_bar:g}: (b={b}, h={h}) key {key}: got {float(got[b, h, key]):.6e} "
                      f"ref32 {float(ref[b, h, key]):.6e} rel32 {float(r[key]):.2e} best {float(best[key]):.2e}")
    n_sel = int(sel.sum())
    assert n_above < frac_above * max(n_sel, 1), (n_above, n_sel)
    assert worst <= max_rel, worst
    return n_sel, worst, n_above, n_excused
