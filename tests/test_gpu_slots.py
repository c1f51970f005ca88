"""K-slot histogram (yabt_hist_slots) against the oracle, through the C ABI.

Bit-identical fp32 output to the oracle's exact fixed-point sums; within the
reference test's 1e-5 normwise tolerance of fp64 sums (test_cuda_hist.py:26-67);
rows outside [0, K) skipped; deterministic.
"""

import numpy as np
import pytest
import torch

from oracle import slots_oracle as SO
from tests.helpers import normwise_rel
from yabt_amd.hist_slots import build_hist

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda", 0) if torch.cuda.is_available() else None


def _case(seed, n, F, K, wkind, bad_slots=False):
    rng = np.random.default_rng(seed)
    binned = rng.integers(0, 256, size=(n, F), dtype=np.uint8)
    slot = np.zeros(n, np.int64) if K == 1 else rng.integers(0, K, size=n)
    if bad_slots:
        slot[rng.random(n) < 0.1] = -1
        slot[rng.random(n) < 0.05] = K
    g = rng.normal(size=n).astype(np.float32)
    h = (rng.random(n) + 0.1).astype(np.float32)
    w = {"ones": np.ones(n, np.float32), "mask": (rng.random(n) > 0.5).astype(np.float32),
         "random": rng.uniform(0, 3, size=n).astype(np.float32)}[wkind]
    if wkind == "mask":
        g, h = g * w, h * w          # the smaller-child form (test_cuda_hist.py:54-67)
    return binned, slot, g, h, w


def _run(binned, slot, g, h, w, K):
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(DEV)
    F = binned.shape[1]
    out = build_hist(t(binned), t(slot), t(g), t(h), t(w), K, F, 256)
    return out.cpu().numpy(), build_hist.last_shifts


@pytest.mark.parametrize("n,F,K,wkind,bad", [
    (20_000, 24, 1, "ones", False), (20_000, 24, 4, "ones", False), (20_000, 24, 31, "random", False),
    (8000, 16, 6, "mask", False), (50_000, 37, 300, "ones", True), (30_000, 5, 5000, "random", True),
    (7, 3, 2, "ones", False), (0, 4, 3, "ones", False),
])
def test_hist_slots_matches_oracle(n, F, K, wkind, bad):
    binned, slot, g, h, w = _case(n + K, n, F, K, wkind, bad)
    got, sh = _run(binned, slot, g, h, w, K)
    ref, rsh = SO.hist_slots_fixed(binned, slot, g, h, w, K)
    assert tuple(sh) == tuple(rsh)
    assert np.array_equal(got, ref)
    if n:
        f64 = SO.hist_slots_f64(binned, slot, g, h, w, K)
        for c in range(3):
            assert normwise_rel(got[c], f64[c]) < 1e-5
        a, _ = _run(binned, slot, g, h, w, K)
        assert np.array_equal(a, got)
