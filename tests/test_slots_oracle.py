"""The K-slot fixed-point oracle against fp64 brute force (CPU only)."""

import numpy as np

from oracle import slots_oracle as SO
from tests.helpers import normwise_rel


def test_fixed_point_slots_match_fp64():
    rng = np.random.default_rng(0)
    n, F, K = 3000, 5, 7
    binned = rng.integers(0, 256, size=(n, F), dtype=np.uint8)
    slot = rng.integers(-1, K + 1, size=n)          # some rows outside [0, K)
    g = rng.normal(size=n).astype(np.float32)
    h = rng.uniform(0.1, 1, size=n).astype(np.float32)
    w = (rng.random(n) < 0.5).astype(np.float32)
    got, _ = SO.hist_slots_fixed(binned, slot, g, h, w, K)
    ref = SO.hist_slots_f64(binned, slot, g, h, w, K)
    for c in range(3):
        assert normwise_rel(got[c], ref[c]) < 2e-7   # fp32 rounding of exact sums
    # unit weights: the third channel is the exact row count
    got1, _ = SO.hist_slots_fixed(binned, slot, g, h, np.ones(n, np.float32), K)
    ok = (slot >= 0) & (slot < K)
    cnt = np.zeros((K, F, 256))
    for f in range(F):
        np.add.at(cnt, (slot[ok], f, binned[ok, f]), 1.0)
    assert np.array_equal(got1[2], cnt.astype(np.float32))
