"""The C-ABI library loads without a GPU and exports every symbol of
include/yabt_hip.h; the ctypes table covers exactly those symbols; host-only
size queries answer without touching a device."""

import ctypes
import os
import re

from yabt_amd import _build, _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "yabt_hip.h")


def _declared():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(yabt_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built():
    assert os.path.exists(_build.LIB), "run __graft_entry__.build() first"


def test_exports_every_declared_symbol():
    lib = ctypes.CDLL(_build.LIB)
    names = _declared()
    assert len(names) >= 12
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_ctypes_table_matches_header():
    assert sorted(_lib.SIGNATURES) == _declared()


def test_host_size_queries():
    lib = _lib.load()
    a = lib.yabt_grow_workspace_bytes(10_000_000, 100, 255)
    # two u32 row lists + one int64 (3,F,256) slot per leaf dominate
    assert a >= 2 * 4 * 10_000_000 + 255 * 3 * 100 * 256 * 8
    assert a < 2 * (2 * 4 * 10_000_000 + 255 * 3 * 100 * 256 * 8)
    assert lib.yabt_grow_workspace_bytes(0, 0, 31) == 0
    assert lib.yabt_grow_workspace_bytes(100, 4, 0) == 0
    assert lib.yabt_hist_workspace_bytes() > 0
    assert lib.yabt_partition_workspace_bytes() > 0
    assert lib.yabt_best_split_workspace_bytes(100) >= 100 * 24


def _ref_hist_bytes(F, L):
    """fp32 (3, F, 256) histograms of the root and both children of every
    split the grower may compute: 3 L + 16 of them (16 per round)."""
    return (1 + 2 * (3 * L + 16)) * 3 * F * 256 * 4


def test_reference_grower_workspace_sizes():
    """The reference grower's bucket lists: 2 bytes per (row, feature), 4 with
    the sparse builder, all features at once up to 8 GiB, one feature at the
    minimum; plus the histogram slots and ~85 bytes per row: 16 row arrays of
    u32 ids (64), the partition's flag, ranks, p and q (13) and g, h (8)."""
    lib = _lib.load()
    n, F, L = 10_000_000, 100, 255
    hist = _ref_hist_bytes(F, L)
    full = lib.yabt_grow_ref_workspace_bytes(n, F, L, 0)
    assert 2 * n * F + hist + 85 * n < full < 2 * n * F + hist + 88 * n + (300 << 20)
    assert lib.yabt_grow_ref_workspace_bytes(n, F, L, 1) - full >= 2 * n * F
    low = lib.yabt_grow_ref_workspace_min_bytes(n, F, L, 0)
    assert full - low >= 2 * n * (F - 1)
    # 4M x 5000 would need 40 GB of lists: capped near 8 GiB
    nb, Fb, Lb = 4_000_000, 5000, 64
    hist = _ref_hist_bytes(Fb, Lb)
    big = lib.yabt_grow_ref_workspace_bytes(nb, Fb, Lb, 0)
    lists_of_one = 2 * (nb + 16 * 4096)
    assert (8 << 30) - lists_of_one + hist < big < (8 << 30) + hist + 88 * nb + (1 << 30)
    assert lib.yabt_grow_ref_workspace_bytes(100, 0, 31, 0) == 0
    assert lib.yabt_grow_ref_workspace_min_bytes(100, 4, 0, 0) == 0


def test_reference_root_order_sizes():
    """The per-fit root rank table: a uint16 rank per (feature, row) padded to
    whole 4096-row tiles, then 257 uint16 run starts, the uint16 longest run
    and the uint8 largest bin per (feature, tile)."""
    lib = _lib.load()
    def rounded(b):
        return (b + 255) // 256 * 256
    for n, F in [(10_000_000, 100), (4097, 3), (1, 1)]:
        tiles = -(-n // 4096)
        want = (rounded(2 * F * tiles * 4096) + rounded(2 * F * tiles * 257) + rounded(2 * F * tiles)
                + rounded(F * tiles))
        assert lib.yabt_ref_root_order_bytes(n, F) == want
    assert lib.yabt_ref_root_order_bytes(100, 0) == 0
    assert lib.yabt_ref_root_order_bytes(-1, 4) == 0
    rc = lib.yabt_ref_root_order(None, 0, 100, 4, None, 0, None)
    assert rc < 0 and "bad pointer" in _lib.last_error()


def test_argument_errors_are_reported_without_a_device():
    lib = _lib.load()
    rc = lib.yabt_grow(None, 0, None, 0, None, None, None, None, ctypes.c_float(0.5), 0, None, None, None, 10, 0,
                       ctypes.c_float(1), ctypes.c_float(0), ctypes.c_float(1e-3), 20,
                       ctypes.c_float(0.1), 31, 64, None, 0, None, None, None, None, None, None,
                       None, None)
    assert rc < 0
    assert "bad sizes" in _lib.last_error()
