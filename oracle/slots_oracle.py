"""CPU oracle of the K-slot histogram (TEST INFRASTRUCTURE ONLY).

The reference op (yabt/_cuda/hist.cu:27-48 via yabt/cuda_hist.py:79-89) adds
(g, h, w) of row i into bin binned[i, f] of slot slot[i], for every feature,
in fp32.  The HIP op's contract is the exact fixed-point version of the same
sums: each channel quantised with the histograms' shift (oracle.quant_shift of
max|.| and n), summed in int64, rounded to fp32.  Only tests/ use this module.
Pinned by tests/test_slots_oracle.py against fp64 brute force.
"""

from __future__ import annotations

import numpy as np

from . import oracle as O


def shifts(g, h, w, n):
    return tuple(O.quant_shift(float(np.abs(v).max()) if v.size else 0.0, n) for v in (g, h, w))


def hist_slots_fixed(binned, slot, g, h, w, K):
    """(3, K, F, 256) fp32 and the shifts."""
    n, F = binned.shape
    ok = (slot >= 0) & (slot < K)
    sh = shifts(g[ok], h[ok], w[ok], n)
    q = np.zeros((3, K, F, 256), np.int64)
    rows = np.nonzero(ok)[0]
    for c, (v, s) in enumerate(zip((g, h, w), sh)):
        qv = np.rint(v[rows].astype(np.float64) * 2.0 ** s).astype(np.int64)
        for f in range(F):
            np.add.at(q[c], (slot[rows], f, binned[rows, f]), qv)
    out = np.stack([(q[c].astype(np.float64) * 2.0 ** -sh[c]).astype(np.float32) for c in range(3)])
    return out, sh


def hist_slots_f64(binned, slot, g, h, w, K):
    """fp64 brute force of the reference sums."""
    n, F = binned.shape
    ok = (slot >= 0) & (slot < K)
    out = np.zeros((3, K, F, 256))
    rows = np.nonzero(ok)[0]
    for c, v in enumerate((g, h, w)):
        for f in range(F):
            np.add.at(out[c], (slot[rows], f, binned[rows, f]), v[rows].astype(np.float64))
    return out
