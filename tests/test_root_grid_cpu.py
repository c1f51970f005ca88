"""The streaming root histogram's grid (csrc/hist.h: root_grid, root_block),
compiled for the CPU with g++: every (tile, row chunk) of the full tiles and
every tail block is dispatched exactly once, all tiles of a chunk land on
one die (block id % 8), no die takes more than its 32 one-block-per-CU
slots, and the chunks and tail spans cover the rows."""

import ctypes
import os
import re
import shutil
import subprocess

import numpy as np
import pytest

HIST_H = os.path.join(os.path.dirname(__file__), "..", "yabt_amd", "csrc", "hist.h")

PRELUDE = """#include <cstdint>
#include <algorithm>
#define __host__
#define __device__
#define __forceinline__ inline
using std::max;
using std::min;
"""

ENTRY = """
extern "C" int cpu_grid(int64_t n, int F, int aligned, int* g, int64_t* tail_rows, int* map, int map_cap) {
    const yabt::RootGrid r = yabt::root_grid(n, F, (const void*)(uintptr_t)(aligned ? 64 : 4),
                                             (const void*)(uintptr_t)64);
    g[0] = r.tiles; g[1] = r.chunks; g[2] = r.tail; g[3] = r.blocks; g[4] = r.xcd;
    *tail_rows = r.tail_rows;
    if (r.blocks > map_cap) return -1;
    for (int b = 0; b < r.blocks; ++b) {
        int tile, chunk, tb;
        const bool live = yabt::root_block(b, r.tiles, r.chunks, r.tail, r.xcd, tile, chunk, tb);
        map[4 * b] = live ? (tb >= 0 ? 2 : 1) : 0;
        map[4 * b + 1] = tile; map[4 * b + 2] = chunk; map[4 * b + 3] = tb;
    }
    return 0;
}
extern "C" int64_t cpu_chunk_rows(int64_t n, int chunks) { return yabt::root_chunk_rows(n, chunks); }
"""


@pytest.fixture(scope="module")
def grid(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    src = open(HIST_H).read()
    consts = [re.search(p, src).group(0) for p in (r"constexpr int HFL = \d+;", r"constexpr int RBLOCK = \d+;",
                                                   r"constexpr int RSTEP = RBLOCK;", r"constexpr int TAILF = \d+;",
                                                   r"constexpr int TSTEP = 2 \* RBLOCK;")]
    a = src.index("__host__ __device__ inline int64_t root_chunk_rows")
    b = src.index("\n}\n", a) + 3
    c = src.index("constexpr int RXCD = ")
    d = src.index("    return tb < tail;\n}\n", c) + len("    return tb < tail;\n}\n")
    body = "\n".join(consts) + "\n" + src[a:b] + "\n" + src[c:d]
    tmp = tmp_path_factory.mktemp("rgrid")
    cpp, so = tmp / "rgrid.cpp", tmp / "rgrid.so"
    cpp.write_text(PRELUDE + "namespace yabt {\n" + body + "\n}  // namespace yabt\n" + ENTRY)
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", str(cpp), "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.cpu_grid.argtypes = [ctypes.c_int64, ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                             ctypes.c_void_p, ctypes.c_int]
    lib.cpu_chunk_rows.restype = ctypes.c_int64
    lib.cpu_chunk_rows.argtypes = [ctypes.c_int64, ctypes.c_int]
    return lib


def _grid(lib, n, F, aligned=True):
    g = np.zeros(5, np.int32)
    tr = np.zeros(1, np.int64)
    m = np.zeros(4 * 4096, np.int32)
    assert lib.cpu_grid(n, F, int(aligned), g.ctypes.data, tr.ctypes.data, m.ctypes.data, 4096) == 0
    tiles, chunks, tail, blocks, xcd = (int(v) for v in g)
    return tiles, chunks, tail, blocks, xcd, int(tr[0]), m[: 4 * blocks].reshape(blocks, 4)


CASES = [(n, F) for n in (1, 2, 3, 1000, 4097, 65_536, 300_001, 1_000_000, 2_000_000, 4_000_000, 10_000_000)
         for F in (1, 3, 4, 5, 16, 17, 20, 28, 36, 50, 100, 112, 500, 513, 1000)]


@pytest.mark.parametrize("aligned", [True, False])
def test_root_grid_covers_each_piece_once(grid, aligned):
    for n, F in CASES:
        tiles, chunks, tail, blocks, xcd, tail_rows, m = _grid(grid, n, F, aligned)
        case = (n, F, aligned, tiles, chunks, tail)
        full = m[m[:, 0] == 1]
        tails = m[m[:, 0] == 2]
        pairs = {(int(t), int(c)) for _, t, c, _ in full}
        assert len(pairs) == len(full) == tiles * chunks, case
        assert pairs == {(t, c) for t in range(tiles) for c in range(chunks)}, case
        assert sorted(int(v) for v in tails[:, 3]) == list(range(tail)), case
        if tiles:
            per = grid.cpu_chunk_rows(n, chunks)
            assert per * chunks >= n and per % 1024 == 0, case
        if tail:
            assert tail_rows * tail >= n and tail_rows * (tail - 1) < n and tail_rows % 2048 == 0, case
        if xcd:
            assert blocks <= 256, case
            die = np.arange(blocks) % 8
            live = m[:, 0] > 0
            assert np.bincount(die[live], minlength=8).max() <= 32, case
            for c in range(chunks):   # every tile of a chunk on one die
                assert len({int(d) for d, row in zip(die, m) if row[0] == 1 and row[2] == c}) == 1, case


def test_root_grid_balances_the_tail_at_10m_x_100(grid):
    tiles, chunks, tail, blocks, xcd, tail_rows, _ = _grid(grid, 10_000_000, 100)
    assert (tiles, chunks, tail, blocks, xcd) == (6, 39, 22, 256, 1)
