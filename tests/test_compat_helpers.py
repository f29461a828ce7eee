"""The reference's launch-geometry helpers kept in ``dropkv_triton`` for
callers that import them (dropkv_triton.py:618-640; reference tests
:1336-1362).  The HIP path sizes its own grids and never calls them, so they
are checked here against hand-computed values of the formula, on the CPU
with the device's CU count stubbed."""

import types

import pytest
import torch

from dropkv_amd.dropkv_triton import _compute_num_splits, _next_power_of_2


@pytest.mark.parametrize("n,expect", [(1, 16), (5, 16), (16, 16), (17, 32), (32, 32), (56, 64), (64, 64),
                                      (65, 128), (256, 256)])
def test_next_power_of_2(n, expect):
    """BLOCK_M = max(16, next_pow2(M)): Qwen2's M = 7*8 = 56 pads to 64."""
    assert _next_power_of_2(n) == expect


def _with_cus(monkeypatch, n):
    monkeypatch.setattr(torch.cuda, "get_device_properties",
                        lambda device=None: types.SimpleNamespace(multi_processor_count=n))


# (cus, B, Hkv, L, BLOCK_N) -> splits, each worked out by hand:
# target = 2*cus; base = B*Hkv; 1 if base >= target, else
# min(ceil(target/base), max(1, ceil(L/BLOCK_N)//4), 64)
CASES = [
    ((256, 1, 8, 32768, 64), 64),    # wanted 64, max_by_work 128
    ((256, 1, 2, 32768, 64), 64),    # wanted 256 -> capped at 64
    ((132, 1, 8, 32768, 64), 33),    # wanted ceil(264/8) = 33
    ((132, 1, 2, 32768, 64), 64),    # wanted 132 -> 64
    ((256, 1, 8, 8, 64), 1),         # one tile
    ((256, 32, 8, 4096, 64), 2),     # 256 programs < 512: wanted 2
    ((132, 32, 8, 4096, 64), 2),     # 256 programs < 264: wanted ceil(264/256) = 2
    ((100, 32, 8, 4096, 64), 1),     # 256 programs >= 200: no split
    ((256, 1, 8, 256, 64), 1),       # 4 tiles -> max_by_work 1
    ((256, 4, 8, 131072, 64), 16),   # wanted ceil(512/32) = 16
    ((256, 1, 8, 1000, 64), 4),      # 16 tiles -> max_by_work 4
]


@pytest.mark.parametrize("args,expect", CASES)
def test_compute_num_splits_table(monkeypatch, args, expect):
    cus, B, Hkv, L, BN = args
    _with_cus(monkeypatch, cus)
    target, base = 2 * cus, B * Hkv
    tiles = -(-L // BN)
    closed = 1 if base >= target else max(1, min(-(-target // base), max(1, tiles // 4), 64))
    got = _compute_num_splits(B, Hkv, L, BN, "cuda")
    assert got == closed == expect


def test_compute_num_splits_reference_properties(monkeypatch):
    """The properties the reference's test asserts (tests:1336-1362) hold
    on a 108-SM part.  On MI355X (256 CUs) two of them do not: Llama and
    Qwen2 both reach the 64-split cap, and B=32, Hkv=8 (256 programs) stays
    below 2*256 programs and still splits in two."""
    for cus in (108, 256):
        _with_cus(monkeypatch, cus)
        ns = _compute_num_splits(1, 8, 32768, 64, "cuda")
        assert 1 < ns and ns * 8 <= 2 * cus + 8
        ns_qwen = _compute_num_splits(1, 2, 32768, 64, "cuda")
        assert (ns_qwen > ns) == (cus == 108)
        assert _compute_num_splits(1, 8, 8, 64, "cuda") == 1
        assert _compute_num_splits(1, 8, 256, 64, "cuda") == 1
        assert _compute_num_splits(32, 8, 4096, 64, "cuda") == (1 if cus == 108 else 2)
