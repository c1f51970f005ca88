"""The split-feature ranking's sort (csrc/leaf.hip, namespace rank), compiled
for the CPU with g++, against torch's CPU argsort (descending) of the counts
-- the ranking of the reference's _used_features (neural_leaves.py:27-31).
The first k positions must be identical, ties included, on random, sorted and
reverse-sorted count lists up to the device's 4096 features."""

import ctypes
import os
import shutil
import subprocess

import numpy as np
import pytest
import torch

LEAF_HIP = os.path.join(os.path.dirname(__file__), "..", "yabt_amd", "csrc", "leaf.hip")

PRELUDE = """#include <cstdint>
#include <cstdlib>
#define __device__
#define __forceinline__ inline
static inline int __clz(int x) { return __builtin_clz((unsigned)x); }
"""

ENTRY = """
extern "C" void cpu_rank(const int32_t* c, int m, int k, int32_t* out) {
    yabt::RankEl* v = (yabt::RankEl*)malloc(sizeof(yabt::RankEl) * (size_t)m);
    int stk[3 * 64];
    for (int i = 0; i < m; ++i) { v[i].c = c[i]; v[i].f = i; }
    yabt::rank::sort(v, m, k, stk);
    for (int i = 0; i < m; ++i) out[i] = v[i].f;
    free(v);
}
"""


@pytest.fixture(scope="module")
def cpu_rank(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    src = open(LEAF_HIP).read()
    a = src.index("struct RankEl {")
    b = src.index("}  // namespace rank") + len("}  // namespace rank")
    d = tmp_path_factory.mktemp("rank")
    cpp, so = d / "rank.cpp", d / "rank.so"
    cpp.write_text(PRELUDE + "namespace yabt {\n" + src[a:b] + "\n}  // namespace yabt\n" + ENTRY)
    subprocess.run(["g++", "-O2", "-shared", "-fPIC", str(cpp), "-o", str(so)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.cpu_rank.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]
    return lib


def test_rank_sort_equals_torch_cpu_argsort(cpu_rank):
    rng = np.random.default_rng(4)
    for trial in range(3000):
        m = int(rng.integers(1, 4097 if trial % 100 == 0 else 600))
        k = int(rng.integers(1, 9))
        hi = int(rng.choice([1, 2, 3, 5, 12, 40, 1000]))
        c = rng.integers(1, hi + 1, m).astype(np.int32)
        if trial % 3 == 0:
            c = np.sort(c)
        if trial % 3 == 1 and m > 3:
            c[: m // 2] = np.sort(c[: m // 2])[::-1]
        if trial % 7 == 0:
            c = np.ascontiguousarray(np.sort(c)[::-1])
        out = np.zeros(m, np.int32)
        cpu_rank.cpu_rank(c.ctypes.data, m, k, out.ctypes.data)
        want = torch.tensor(c.astype(np.int64)).argsort(descending=True).numpy()
        assert np.array_equal(out[:k], want[:k]), (trial, m, k)
