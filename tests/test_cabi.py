"""The C-ABI library loads and exports every entry point that
include/dropkv_amd.h declares; host-side argument checks and workspace
queries behave as documented.  No GPU work is launched (CPU suite)."""

import ctypes
import os
import re

import pytest

from dropkv_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dropkv_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[a-z_0-9]+\s*\*?\s*(dropkv_[a-z_0-9]+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        from dropkv_amd import _build
        _build.build()
    return _lib.load()


def test_header_declares_entry_points():
    names = _declared_functions()
    assert "dropkv_scores" in names and "dropkv_evict" in names and len(names) >= 10


def test_every_declared_symbol_is_exported(lib):
    raw = ctypes.CDLL(_lib.LIB_PATH)
    missing = [n for n in _declared_functions() if not hasattr(raw, n)]
    assert not missing, f"not exported: {missing}"


def test_binding_table_matches_header():
    """The ctypes signature table covers exactly the declared functions."""
    assert sorted(_lib._SIGNATURES) == _declared_functions()


def test_version_and_head_dims(lib):
    assert lib.dropkv_version() >= 100
    assert _lib.supported_head_dims() == (32, 64, 128)


def test_workspace_queries(lib):
    # invalid shapes report 0 bytes
    assert lib.dropkv_scores_workspace_bytes(1, 7, 2, 100, 64, 8, 0) == 0
    assert lib.dropkv_select_workspace_bytes(0, 100) == 0
    a = lib.dropkv_scores_workspace_bytes(1, 32, 8, 32768, 128, 8, 0)
    b = lib.dropkv_select_workspace_bytes(8, 32768)
    c = lib.dropkv_evict_workspace_bytes(1, 32, 8, 32768, 128, 8, 0)
    assert a > 0 and b > 0 and c >= a + b + 8 * 32768 * 4


@pytest.mark.parametrize("args,code,msg", [
    # (q, k, v) null
    (dict(q=None), 1, "null q/k/v"),
    (dict(dtype=4), 1, "bf16, fp16 or fp32"),
    (dict(Hq=30), 1, "divisible"),
    (dict(W=0), 1, "window must be positive"),
    (dict(Lq=4), 1, "must be >= window_size"),
    (dict(Lq=200), 1, "must be <= Lk"),
    (dict(D=0), 1, "head dim must be positive"),
    (dict(D=8192), 2, "head dim 8192 above 4096"),
    (dict(B=1 << 20, Lk=1 << 12), 2, "B*Hq*W or B*Hkv*Lk above"),     # 2^35 keys
    (dict(Hq=1 << 22, Hkv=1 << 10, W=1 << 10, Lq=1 << 10, Lk=1 << 10), 2, "B*Hq*W or B*Hkv*Lk above"),  # 2^32 rows
])
def test_score_argument_checks(lib, args, code, msg):
    """Checks happen on the host before anything is enqueued."""
    fake = ctypes.c_void_p(1 << 20)  # never dereferenced: the checks fail first
    a = dict(q=fake, k=fake, v=fake, dtype=1, B=1, Hq=32, Hkv=8, Lq=64, Lk=100, D=128, W=8)
    a.update(args)
    rc = lib.dropkv_scores(a["q"], 0, 0, 0, 1, a["k"], a["v"], a["dtype"], a["B"], a["Hq"], a["Hkv"], a["Lq"],
                           a["Lk"], a["D"], a["W"], 1e-6, 1, 0, 0, None, None, 0, None)
    assert rc == code
    assert msg in lib.dropkv_last_error().decode()


def test_select_argument_checks(lib):
    fake = ctypes.c_void_p(1 << 20)
    assert lib.dropkv_select(fake, 8, 100, 10, 8, 10, fake, None, fake, 1 << 20, None) == 1   # even kernel
    assert "odd" in lib.dropkv_last_error().decode()
    assert lib.dropkv_select(fake, 8, 100, 11, 8, 101, fake, None, fake, 1 << 20, None) == 1  # keep > Lk
    assert lib.dropkv_select(fake, 8, 100, 11, 8, 10, fake, None, fake, 16, None) == 3        # workspace
    assert "workspace too small" in lib.dropkv_last_error().decode()


def test_compact_argument_checks(lib):
    fake = ctypes.c_void_p(1 << 20)
    assert lib.dropkv_compact(fake, fake, 0, 0, 0, 3, 1, 1, 10, 8, fake, 4, fake, fake, None) == 1
    assert "elem_bytes" in lib.dropkv_last_error().decode()
    assert lib.dropkv_compact2(fake, fake, 0, 0, 0, -1, fake, fake, 0, 0, 0, 5, 2, 1, 1, 8, fake, 4, fake, fake,
                               None) == 1


def test_capacity_entry_argument_checks(lib):
    """dropkv_append / dropkv_evict_ld reject rows that do not fit the
    buffers before enqueuing anything."""
    fake = ctypes.c_void_p(1 << 20)
    # 10 rows at row 95 of a 100-row buffer
    assert lib.dropkv_append(fake, fake, 0, 0, 128, 2, 1, 8, 10, 128, fake, fake, 100, 95, None) == 1
    assert "do not fit" in lib.dropkv_last_error().decode()
    assert lib.dropkv_append(fake, fake, 0, 0, 128, 3, 1, 8, 10, 128, fake, fake, 100, 0, None) == 1
    assert "elem_bytes" in lib.dropkv_last_error().decode()
    # K/V row capacity (kv_ld = 50) below Lk = 100
    args = [fake, 0, 0, 0, 1, fake, fake, 50, 1, 1, 32, 8, 64, 100, 128, 8, 1e-6, 1, 0, 0, 11, 8, 10,
            None, fake, fake, fake, 10, fake, 1 << 30, None]
    assert lib.dropkv_evict_ld(*args) == 1
    assert "row capacity" in lib.dropkv_last_error().decode()
    args[7] = 100
    args[27] = 5  # output capacity below keep = 10
    assert lib.dropkv_evict_ld(*args) == 1
    assert "row capacity" in lib.dropkv_last_error().decode()


def test_noalloc_entry_refuses_shapes_beyond_its_scratch(lib):
    """dropkv_evict_noalloc checks its arguments and the scratch bound on the
    host, before it looks up the scratch or enqueues anything."""
    fake = ctypes.c_void_p(1 << 20)
    assert _lib.NOALLOC_SCRATCH_BYTES == 32 << 20
    # B4 Hq64 Hkv8 D128 Lk=131072 W32: 78 MiB of scratch
    need = lib.dropkv_evict_workspace_bytes(4, 64, 8, 131072, 128, 32, 0)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    args = [fake, 0, 0, 0, 1, fake, fake, 1, 4, 64, 8, 131072, 131072, 128, 32, 1e-6, 1, 0, 0, 11, 32, 6553,
            None, fake, fake, fake, None]
    assert lib.dropkv_evict_noalloc(*args) == 2
    msg = lib.dropkv_last_error().decode()
    assert "needs %d bytes of scratch" % need in msg and "dropkv_evict with a workspace" in msg
    args[14] = 0  # window 0: an argument error comes first
    assert lib.dropkv_evict_noalloc(*args) == 1
    assert "window must be positive" in lib.dropkv_last_error().decode()


def test_workspace_sizes_refuse_overflowing_shapes(lib):
    """Shapes whose window rows (B*Hq*W) or keys (B*Hkv*Lk) exceed 2^31-1
    get no workspace size (0) rather than a wrapped-around one."""
    assert lib.dropkv_scores_workspace_bytes(1 << 20, 32, 8, 32768, 128, 8, 0) == 0
    assert lib.dropkv_evict_workspace_bytes(1 << 20, 32, 8, 32768, 128, 8, 0) == 0
    assert lib.dropkv_scores_workspace_bytes(1, 1 << 22, 1 << 10, 4096, 128, 1 << 10, 0) == 0
    assert lib.dropkv_select_workspace_bytes(1 << 16, 1 << 16) == 0
    assert lib.dropkv_scores_workspace_bytes(1, 32, 8, 32768, 128, 8, 0) > 0


def _noalloc_max_keys(lib, B, Hq, Hkv, D, W):
    cap = _lib.NOALLOC_SCRATCH_BYTES
    lo, hi = 1, 1 << 26
    while lo < hi:
        m = (lo + hi + 1) // 2
        b = lib.dropkv_evict_workspace_bytes(B, Hq, Hkv, m, D, W, 0)
        lo, hi = (m, hi) if 0 < b <= cap else (lo, m - 1)
    return lo


def test_noalloc_limits_in_the_header_match_the_library(lib):
    """The key counts the header quotes for dropkv_evict_noalloc are the
    largest Lk whose dropkv_evict_workspace_bytes fits the static scratch,
    and the stress shape's figure is its workspace size."""
    import re
    text = open(HEADER).read()
    m = re.search(r"Llama-3\.1-8B layer \(B 1, Hq 32,\s*\*\s*Hkv 8, D 128, W 8\) up to (\d+) keys and a "
                  r"Qwen2-0\.5B layer \(B 1, Hq 14,\s*\*\s*Hkv 2, D 64, W 8\) up to (\d+) keys;.*?needs "
                  r"([0-9.]+) MiB", text, re.S)
    assert m, "no-alloc coverage sentence not found in the header"
    assert int(m.group(1)) == _noalloc_max_keys(lib, 1, 32, 8, 128, 8)
    assert int(m.group(2)) == _noalloc_max_keys(lib, 1, 14, 2, 64, 8)
    c5 = lib.dropkv_evict_workspace_bytes(4, 64, 8, 131072, 128, 32, 0) / 2 ** 20
    assert abs(float(m.group(3)) - c5) < 0.05
    assert c5 * 2 ** 20 > _lib.NOALLOC_SCRATCH_BYTES
