"""The layer-call's selection finished in the scoring kernel's tail
(dkv_tail_dev.h: pooling, threshold, ordered emit and K/V gather in the
pass-2 launch, with two barriers among each row's workgroups) against the same
selection run as two further kernels (dropkv_set_tail_select(0)), and against
the oracle's selection rule.

* The tail is the path taken: a timed call launches three kernels (pass 1,
  merge, pass 2 with the tail) instead of five.
* Bit-identical scores, kept indices and gathered K/V with the tail on and
  off, on shapes that take it: the Llama-8B head shape, a partial last split,
  a last split shorter than the pooling half-width, batch 2 in fp16 with
  padding rows, the Qwen2 head shape at the C4 length (many short splits),
  D = 32, and keep = window.
* The kept indices equal the oracle's rule (pool, protect, stable top-k,
  ascending) applied to the GPU's own scores, bit for bit.
* V = 0 makes every score 0: all unprotected keys tie at the threshold, the
  candidates overflow the tail's LDS list and each workgroup sweeps the
  pooled row instead; the lowest indices must win, as in the oracle.
* Lone finish: with a spin limit of 0 at barrier A every workgroup but a
  row's last one leaves there, and the last one finishes the row from
  memory; with a limit of 0 at barrier B every workgroup that does not find
  the whole row arrived gives up there and finishes the whole row alone
  (concurrently with the others, writing the same outputs); with both at 0,
  both happen.  In every case every kernel exits and the bits must not
  change.
* Repeated calls, and HIP graph replays with eager calls in between, give
  the same bits (the barrier words are cleared by the merge kernel of every
  call).
* Edge cases of the pooling and protection geometry: a 33-wide pooling
  window, no pooling (kernel 1), a protected tail longer than a split,
  keep = Lk - 1, keep = 1 with nothing protected, and one KV head split 128
  ways; each against the oracle's rule, the gather and the separate kernels.
"""

import ctypes

import pytest
import torch

from conftest import LLAMA_CFG, QWEN_CFG, make_qkv
from oracle import dropkv_ref as R

pytestmark = pytest.mark.gpu

SPIN_A, SPIN_B = 1 << 16, 1 << 22  # the library's default poll limits at barriers A and B

CASES = [
    # (cfg, Lq, Lk, W, dtype, keep_ratio)
    (LLAMA_CFG, 8192, 8192, 8, torch.bfloat16, 0.1),                       # 32 splits of 256 keys
    (dict(B=1, Hq=16, Hkv=4, D=128), 6000, 6000, 8, torch.bfloat16, 0.1),  # partial last split
    (LLAMA_CFG, 8931, 8931, 8, torch.bfloat16, 0.1),                       # last split of 3 keys (< h)
    (dict(B=2, Hq=8, Hkv=2, D=128), 4096, 4096, 7, torch.float16, 0.1),    # g*W = 28: padding rows
    (QWEN_CFG, 16384, 16384, 8, torch.bfloat16, 0.1),                      # 64 splits of 256 keys, two row-chunks
    (dict(B=1, Hq=8, Hkv=2, D=32), 3000, 3000, 8, torch.bfloat16, 0.1),    # D = 32
    (LLAMA_CFG, 4096, 4096, 8, torch.bfloat16, 0.0),                       # keep = window
]


@pytest.fixture
def tail():
    """The tail on (the library default) for the test and afterwards."""
    from dropkv_amd import ops
    ops.set_tail_select(True, SPIN_A, SPIN_B)
    yield ops
    ops.set_tail_select(True, SPIN_A, SPIN_B)


def _run(ops, Q, K, V, W, ks, keep, plan=None):
    if plan is None:
        plan = ops.EvictPlan(Q, K, W, ks, keep, keep_scores=True)
    idx, ko, vo = plan(Q, K, V)
    torch.cuda.synchronize()
    return plan, (idx.clone(), ko.clone(), vo.clone(), plan.scores.clone())


def _kernels_of(fn):
    """Number of kernels one library call launched (dropkv_timing_*)."""
    from dropkv_amd import _lib
    lib = _lib.load()
    buf = (ctypes.c_double * 16)()
    _lib.check(lib.dropkv_timing_enable(1), "dropkv_timing_enable")
    try:
        fn()
        n = lib.dropkv_timing_read(buf, 16)
    finally:
        lib.dropkv_timing_enable(0)
    assert n >= 0
    return n


def _inputs(case, gpu, seed):
    cfg, Lq, Lk, W, dtype, ratio = CASES[case]
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=dtype, seed=seed, k_scale="lognormal")
    keep = R.keep_length(ratio, Lk, W)
    return (Q, K, V), (Q.to(gpu), K.to(gpu), V.to(gpu)), W, keep


def _assert_oracle_rule(out, K, V, ks, W, keep):
    idx, ko, vo, s = out
    pooled = R.pool_protect(s.cpu().clone(), ks, W)
    assert torch.equal(idx.cpu(), R.topk_sorted(pooled, keep))
    rk, rv = R.gather_compressed(K, V, idx.cpu())
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_tail_equals_separate_kernels(gpu, tail, case):
    (Q, K, V), (Qg, Kg, Vg), W, keep = _inputs(case, gpu, 60 + case)
    ks = 11
    print(f"[tail] case {case} shape {tuple(K.shape)} keep {keep}", flush=True)
    plan, a = _run(tail, Qg, Kg, Vg, W, ks, keep)
    assert _kernels_of(lambda: plan(Qg, Kg, Vg)) == 3, "the selection did not run in the scoring tail"
    _assert_oracle_rule(a, K, V, ks, W, keep)
    tail.set_tail_select(False)
    plan_b, b = _run(tail, Qg, Kg, Vg, W, ks, keep)
    assert _kernels_of(lambda: plan_b(Qg, Kg, Vg)) == 5
    tail.set_tail_select(True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_tail_all_ties_sweeps_the_row(gpu, tail):
    """V = 0: every score is 0, so every unprotected key sits at the
    threshold and the lowest indices are kept."""
    (Q, K, V), (Qg, Kg, Vg), W, keep = _inputs(0, gpu, 70)
    V = torch.zeros_like(V)
    Vg = V.to(gpu)
    ks = 11
    print("[tail] all ties", flush=True)
    plan, a = _run(tail, Qg, Kg, Vg, W, ks, keep)
    assert _kernels_of(lambda: plan(Qg, Kg, Vg)) == 3
    assert not a[3].any()
    _assert_oracle_rule(a, K, V, ks, W, keep)
    Lk = K.shape[2]
    expect = torch.cat([torch.arange(keep - W), torch.arange(Lk - W, Lk)])
    assert torch.equal(a[0].cpu(), expect.expand_as(a[0].cpu()))


@pytest.mark.parametrize("limits", [(0, SPIN_B), (SPIN_A, 0), (0, 0)], ids=["A", "B", "AB"])
@pytest.mark.parametrize("case", [0, 4])
def test_tail_lone_finish_is_bit_identical(gpu, tail, case, limits):
    (Q, K, V), (Qg, Kg, Vg), W, keep = _inputs(case, gpu, 80 + case)
    ks = 11
    print(f"[tail lone] case {case} poll limits {limits}", flush=True)
    plan, a = _run(tail, Qg, Kg, Vg, W, ks, keep)
    tail.set_tail_select(True, *limits)
    try:
        plan_b, b = _run(tail, Qg, Kg, Vg, W, ks, keep)
    finally:
        tail.set_tail_select(True, SPIN_A, SPIN_B)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    # the workspace serves a normal call again afterwards
    _, c = _run(tail, Qg, Kg, Vg, W, ks, keep, plan=plan_b)
    for x, y in zip(a, c):
        assert torch.equal(x, y)


def test_tail_repeats_and_graph_replays(gpu, tail):
    (Q, K, V), (Qg, Kg, Vg), W, keep = _inputs(0, gpu, 90)
    ks = 11
    # a second input set on the same plan, alternating with the first
    Q2, K2, V2 = make_qkv(LLAMA_CFG, 8192, 8192, seed=91, k_scale="lognormal")
    Q2g, K2g, V2g = Q2.to(gpu), K2.to(gpu), V2.to(gpu)
    print("[tail] repeats and graph replays", flush=True)
    plan, a = _run(tail, Qg, Kg, Vg, W, ks, keep)
    _, b = _run(tail, Q2g, K2g, V2g, W, ks, keep, plan=plan)
    _assert_oracle_rule(b, K2, V2, ks, W, keep)
    for _ in range(3):
        _, x = _run(tail, Qg, Kg, Vg, W, ks, keep, plan=plan)
        assert all(torch.equal(u, v) for u, v in zip(a, x))
        _, y = _run(tail, Q2g, K2g, V2g, W, ks, keep, plan=plan)
        assert all(torch.equal(u, v) for u, v in zip(b, y))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        plan(Qg, Kg, Vg)
    for _ in range(3):
        plan.keep_idx.fill_(-1)
        plan.k_out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        got = (plan.keep_idx.clone(), plan.k_out.clone(), plan.v_out.clone(), plan.scores.clone())
        assert all(torch.equal(u, v) for u, v in zip(a, got))
        _, y = _run(tail, Q2g, K2g, V2g, W, ks, keep, plan=plan)
        assert all(torch.equal(u, v) for u, v in zip(b, y))


EDGE_CASES = [
    # (cfg, Lk, W, kernel_size, protect_window, keep)
    (LLAMA_CFG, 8192, 8, 33, 8, 819),                      # wide pooling: 4h = 64 raw scores per boundary
    (LLAMA_CFG, 8192, 8, 1, 8, 819),                       # no pooling (h = 0): no boundary keys
    (LLAMA_CFG, 8192, 8, 11, 600, 819),                    # protected tail longer than a 256-key split
    (LLAMA_CFG, 4096, 8, 11, 8, 4095),                     # almost every key kept
    (LLAMA_CFG, 4096, 8, 11, 0, 1),                        # one key, nothing protected
    (dict(B=1, Hq=8, Hkv=1, D=128), 32768, 8, 11, 8, 3276),  # one row in 128 splits
]


@pytest.mark.parametrize("case", range(len(EDGE_CASES)))
def test_tail_edge_cases(gpu, tail, case):
    cfg, Lk, W, ks, pw, keep = EDGE_CASES[case]
    Q, K, V = make_qkv(cfg, Lk, Lk, seed=110 + case, k_scale="lognormal")
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    print(f"[tail edge] case {case} Lk {Lk} ks {ks} protect {pw} keep {keep}", flush=True)

    def run():
        plan = tail.EvictPlan(Qg, Kg, W, ks, keep, protect_window=pw, keep_scores=True)
        idx, ko, vo = plan(Qg, Kg, Vg)
        torch.cuda.synchronize()
        return plan, (idx.clone(), ko.clone(), vo.clone(), plan.scores.clone())

    plan, a = run()
    assert _kernels_of(lambda: plan(Qg, Kg, Vg)) == 3
    pooled = R.pool_protect(a[3].cpu().clone(), ks, pw)
    assert torch.equal(a[0].cpu(), R.topk_sorted(pooled, keep))
    rk, rv = R.gather_compressed(K, V, a[0].cpu())
    assert torch.equal(a[1].cpu(), rk) and torch.equal(a[2].cpu(), rv)
    tail.set_tail_select(False)
    _, b = run()
    tail.set_tail_select(True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
