"""The resident layer-call (pass 1, merge and pass 2 in one kernel that keeps
V and the logits on chip, dkv_resident.hip) against the oracle and against
itself.

* Parity: shapes that take the resident kernel (D = 128, g*W <= 32,
  B*Hkv*ceil(Lk/1024) <= CUs), including a partial last 1024-key split,
  padding rows (g*W < 32) and fp16, against the float32 reference with the
  binding-key bars of the full-size tests (max relative error 2e-2, fewer
  than 1e-3 of the binding keys beyond 1e-3) and the tie-aware overlap of
  the kept sets; gathers bit-exact.
* The lone-finish path: with a spin limit of 0 every workgroup but a head's
  last one leaves at the first barrier and the last one finishes the head
  from memory; scores, kept indices and gathered rows must equal the
  resident run's bit for bit (same instructions on the same operands).
* State: the barrier counters are zero after every call; repeated calls and
  HIP graph replays (with eager calls in between) give the same bits.
* Against the streaming passes (dropkv_set_resident(0)): the same
  selection up to keys at the threshold, scores within 1e-4 relative on the
  binding keys with p unrounded (the two differ only in the split-K
  summation order).
"""

import pytest
import torch

from conftest import assert_binding_scores, binding_keys, make_qkv
from oracle import dropkv_ref as R

pytestmark = pytest.mark.gpu

SHAPES = [
    # (cfg, Lq, Lk, W, dtype): S = ceil(Lk/1024) workgroups per head
    (dict(B=1, Hq=16, Hkv=4, D=128), 6000, 6000, 8, torch.bfloat16),    # partial last split
    (dict(B=2, Hq=8, Hkv=2, D=128), 4096, 4096, 7, torch.float16),      # g*W = 28: padding rows
    (dict(B=1, Hq=32, Hkv=8, D=128), 9000, 9000, 8, torch.bfloat16),    # Llama-8B heads
    (dict(B=1, Hq=8, Hkv=8, D=128), 700, 700, 4, torch.bfloat16),       # one split per head
]


@pytest.fixture
def resident():
    """The resident kernel on for the test, the library default afterwards."""
    from dropkv_amd import ops
    ops.set_resident(True, 1 << 16)
    yield ops
    ops.set_resident(False, 1 << 16)


def _run(ops, Q, K, V, W, ks, keep, p_round=True):
    plan = ops.EvictPlan(Q, K, W, ks, keep, keep_scores=True, p_round=p_round)
    idx, ko, vo = plan(Q, K, V)
    torch.cuda.synchronize()
    return plan, idx.clone(), ko.clone(), vo.clone(), plan.scores.clone()


def _counters_zero(plan):
    from dropkv_amd import _lib
    return not bool(plan.ws[: _lib.SYNC_BYTES].any().item())


@pytest.mark.parametrize("case", range(len(SHAPES)))
def test_resident_parity(gpu, resident, case):
    cfg, Lq, Lk, W, dtype = SHAPES[case]
    ks, ratio = 11, 0.1
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=dtype, seed=40 + case, k_scale="lognormal")
    keep = R.keep_length(ratio, Lk, W)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    print(f"[resident parity] case {case} cfg {cfg} Lk {Lk} W {W} {dtype}", flush=True)
    plan, idx, ko, vo, s = _run(resident, Qg, Kg, Vg, W, ks, keep)
    assert _counters_zero(plan)
    Qt = Q[:, :, -W:].contiguous()
    ref = R.dropkv_scores_reference(Qt, K, V, W, match_pytorch_precision=True)
    ref_idx, pooled = R.compute_keep_indices(Qt, K, V, ratio, W, ks, scores=ref)
    stats = assert_binding_scores(s, ref, pooled, keep, Qt, K, V, W, dtype, 2e-2, 1e-3, 1e-3)
    print(f"[resident parity] binding {stats[0]}, worst rel {stats[1]:.2e}, beyond 1e-3 {stats[2]}", flush=True)
    worst, unexcused = R.index_overlap(idx.cpu(), ref_idx, pooled)
    assert worst >= 0.999, (worst, unexcused)
    rk, rv = R.gather_compressed(K, V, idx.cpu())
    assert torch.equal(ko.cpu(), rk) and torch.equal(vo.cpu(), rv)


@pytest.mark.parametrize("case", [0, 1])
def test_lone_finish_is_bit_identical(gpu, resident, case):
    cfg, Lq, Lk, W, dtype = SHAPES[case]
    ks = 11
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=dtype, seed=50 + case, k_scale="lognormal")
    keep = R.keep_length(0.1, Lk, W)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    print(f"[resident lone] case {case}", flush=True)
    plan_a, *a = _run(resident, Qg, Kg, Vg, W, ks, keep)
    resident.set_resident(True, 0)
    plan_b, *b = _run(resident, Qg, Kg, Vg, W, ks, keep)
    assert _counters_zero(plan_b)
    resident.set_resident(True, 1 << 16)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    # and the workspace serves a normal call again afterwards
    idx, ko, vo = plan_b(Qg, Kg, Vg)
    assert torch.equal(idx, a[0]) and torch.equal(ko, a[1]) and _counters_zero(plan_b)


def test_repeat_and_graph_replays(gpu, resident):
    cfg, Lq, Lk, W, dtype = SHAPES[2]
    ks = 11
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=dtype, seed=60, k_scale="lognormal")
    keep = R.keep_length(0.1, Lk, W)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    print("[resident graph] eager", flush=True)
    plan, idx0, ko0, vo0, s0 = _run(resident, Qg, Kg, Vg, W, ks, keep)
    for _ in range(3):
        idx, ko, vo = plan(Qg, Kg, Vg)
        assert torch.equal(idx, idx0) and torch.equal(ko, ko0) and torch.equal(plan.scores, s0)
    gplan = resident.EvictPlan(Qg, Kg, W, ks, keep, keep_scores=True)
    gplan(Qg, Kg, Vg)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gplan(Qg, Kg, Vg)
    print("[resident graph] replays", flush=True)
    for _ in range(3):
        gplan.keep_idx.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gplan.keep_idx, idx0) and torch.equal(gplan.k_out, ko0)
        assert torch.equal(gplan.v_out, vo0) and torch.equal(gplan.scores, s0)
        assert _counters_zero(gplan)
        plan(Qg, Kg, Vg)  # eager work between replays
        torch.cuda.synchronize()


def test_resident_against_streaming(gpu, resident):
    cfg, Lq, Lk, W, dtype = SHAPES[2]
    ks, ratio = 11, 0.1
    Q, K, V = make_qkv(cfg, Lq, Lk, dtype=dtype, seed=70, k_scale="lognormal")
    keep = R.keep_length(ratio, Lk, W)
    Qg, Kg, Vg = Q.to(gpu), K.to(gpu), V.to(gpu)
    print("[resident vs streaming]", flush=True)
    # p unrounded (fp32 mode), so that the two differ only by summation order
    _, idx_r, _, _, s_r = _run(resident, Qg, Kg, Vg, W, ks, keep, p_round=False)
    resident.set_resident(False)
    try:
        _, idx_s, _, _, s_s = _run(resident, Qg, Kg, Vg, W, ks, keep, p_round=False)
    finally:
        resident.set_resident(True)
    pooled = R.pool_protect(s_s.cpu().clone(), ks, W)
    sel = binding_keys(s_s.cpu(), pooled, keep)
    rel = ((s_r.cpu().double() - s_s.cpu().double()).abs() / s_s.cpu().double().abs().clamp_min(1e-300))[sel]
    print(f"[resident vs streaming] binding keys {int(sel.sum())}, max rel {rel.max().item():.2e}", flush=True)
    assert rel.max().item() <= 1e-4
    worst, unexcused = R.index_overlap(idx_r.cpu(), idx_s.cpu(), pooled)
    assert worst >= 0.999, (worst, unexcused)


def test_new_inputs_on_a_used_workspace(gpu, resident):
    """A plan's workspace still holds the previous call's partials and merged
    rows: a call on other inputs must read only what its own workgroups
    published (scores equal to a fresh streaming run's up to summation order,
    p unrounded), in both orders of two input sets."""
    cfg, Lq, Lk, W, dtype = SHAPES[2]
    ks = 11
    keep = R.keep_length(0.1, Lk, W)
    sets = [tuple(t.to(gpu) for t in make_qkv(cfg, Lq, Lk, dtype=dtype, seed=s, k_scale="lognormal"))
            for s in (80, 81)]
    ref = []
    resident.set_resident(False)
    try:
        for Q, K, V in sets:
            plan = resident.EvictPlan(Q, K, W, ks, keep, keep_scores=True, p_round=False)
            plan(Q, K, V)
            ref.append(plan.scores.clone())
    finally:
        resident.set_resident(True)
    plan = resident.EvictPlan(sets[0][0], sets[0][1], W, ks, keep, keep_scores=True, p_round=False)
    for order in ((0, 1), (1, 0), (0, 1)):
        for i in order:
            print(f"[resident reuse] inputs {i}", flush=True)
            plan(*sets[i])
            torch.cuda.synchronize()
            got, exp = plan.scores.double(), ref[i].double()
            rel = ((got - exp).abs() / exp.abs().clamp_min(1e-30)).max().item()
            assert rel <= 1e-4, (i, rel)
