"""ctypes front end of the CPU oracle (grow_oracle.c) and of the compiled
reference grow.c (oracle/_ref/libgrow_ref.so, when it has been built).

TEST INFRASTRUCTURE ONLY: used by tests/, ``__graft_entry__.smoke()`` and the
cpu_baseline leg of bench.py as the reference the HIP path is checked against
or timed beside.  Nothing in ``yabt_amd`` imports this module.

Argument marshalling follows ``grow_tree_c`` (yabt/grow_c.py:336-426): bins are
feature-major (F, n) uint8, grad/hess float32, lam/gamma/mcw/lr are rounded to
float32 (ctypes.c_float) exactly as the reference passes them.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_SO = os.path.join(HERE, "liboracle.so")
REF_SO = os.path.join(HERE, "_ref", "libgrow_ref.so")

MODE_FP32 = 0
MODE_FIXED = 1
B = 256

_LIB = None
_REF = None

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_flt = ctypes.c_float
_dbl = ctypes.c_double


def build() -> None:
    """Compile liboracle.so (and the reference, if its source is mounted)."""
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)
    if os.path.exists("/root/reference/yabt/_cgrow/grow.c"):
        subprocess.run(["make", "-s", "-C", HERE, "ref"], check=True)


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_vp)


def lib():
    global _LIB
    if _LIB is None:
        if not os.path.exists(ORACLE_SO):
            build()
        L = ctypes.CDLL(ORACLE_SO)
        L.or_quant_shift.restype = _int
        L.or_quant_shift.argtypes = [_flt, _i64]
        L.or_hist_shift.restype = _int
        L.or_hist_shift.argtypes = [_flt, _i64]
        L.or_quant_shifts.restype = _int
        L.or_quant_shifts.argtypes = [_vp, _vp, _i64, _vp, _vp]
        L.or_wide_shift.restype = _int
        L.or_wide_shift.argtypes = [_flt, _i64]
        L.or_hist_contract.restype = _int
        L.or_hist_contract.argtypes = [_vp, _vp, _i64, _vp, _vp]
        L.or_hist_f32.restype = None
        L.or_hist_f32.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp]
        L.or_hist_sparse_f32.restype = None
        L.or_hist_sparse_f32.argtypes = [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _int, _vp]
        L.or_hist_fixed.restype = None
        L.or_hist_fixed.argtypes = [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _int,
                                    _vp, _vp, _vp]
        L.or_best_split_f32.restype = _dbl
        L.or_best_split_f32.argtypes = [_vp, _vp, _dbl, _dbl, _dbl, _int, _vp, _vp, _int, _vp, _vp]
        L.or_best_split_fixed.restype = _dbl
        L.or_best_split_fixed.argtypes = [_vp, _vp, _vp, _int, _int, _vp, _dbl, _dbl, _dbl, _int,
                                          _vp, _vp, _int, _vp, _vp]
        L.or_compute_boost.restype = None
        L.or_compute_boost.argtypes = [_vp, _vp, _flt, _vp, _int]
        L.or_partition_twoptr.restype = _i64
        L.or_partition_twoptr.argtypes = [_vp, _vp, _i64, _i64, _int]
        L.or_partition_stable.restype = _i64
        L.or_partition_stable.argtypes = [_vp, _vp, _i64, _i64, _int, _vp]
        L.or_grow.restype = _int
        L.or_grow.argtypes = ([_int, _vp, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _vp, _vp,
                               _int, _vp, _i64, _int, _flt, _flt, _flt, _int, _flt, _int, _int,
                               _int] + [_vp] * 6 + [_vp] * 6)
        L.or_apply.restype = None
        L.or_apply.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _int, _int, _vp]
        _LIB = L
    return _LIB


def ref_available() -> bool:
    return os.path.exists(REF_SO)


def ref_lib():
    """The compiled reference grow.c (signature grow.c:243-250 / grow_c.py:168-200)."""
    global _REF
    if _REF is None:
        L = ctypes.CDLL(REF_SO)
        L.cgrow.restype = _int
        L.cgrow.argtypes = ([_vp, _vp, _vp, _vp, _vp, _flt, _int, _vp, _vp, _vp, _vp, _int, _vp,
                             _i64, _int, _int, _flt, _flt, _flt, _int, _flt, _int, _int, _int]
                            + [_vp] * 6)
        L.capply.restype = None
        L.capply.argtypes = [_vp, _vp, _vp, _vp, _vp, _i64, _int, _int, _vp]
        _REF = L
    return _REF


# --------------------------------------------------------------------------
# grower
# --------------------------------------------------------------------------

def _common_inputs(bins_fm, grad, hess, fmask, imat, sparse, nbins):
    bins_fm = np.ascontiguousarray(bins_fm, dtype=np.uint8)
    F, n = bins_fm.shape
    grad = np.ascontiguousarray(grad, dtype=np.float32)
    hess = np.ascontiguousarray(hess, dtype=np.float32)
    fm = (np.ones(F, np.uint8) if fmask is None
          else np.ascontiguousarray(np.asarray(fmask).astype(bool), dtype=np.uint8))
    use_imat = imat is not None
    im = (np.ascontiguousarray(imat, dtype=np.float32) if use_imat
          else np.zeros((1, 1), np.float32))
    if sparse is not None:
        sp = (np.ascontiguousarray(sparse[0], dtype=np.int64),
              np.ascontiguousarray(sparse[1], dtype=np.int32),
              np.ascontiguousarray(sparse[2], dtype=np.int32),
              np.ascontiguousarray(sparse[3], dtype=np.int32))
        use_sparse = 1
    else:
        sp = (np.zeros(1, np.int64), np.zeros(1, np.int32), np.zeros(1, np.int32),
              np.zeros(1, np.int32))
        use_sparse = 0
    nb = (np.full(F, B, np.int32) if nbins is None
          else np.ascontiguousarray(nbins, dtype=np.int32))
    return bins_fm, F, n, grad, hess, fm, use_imat, im, sp, use_sparse, nb


def grow(bins_fm, grad, hess, *, mode=MODE_FP32, fmask=None, imat=None, ib=0.5, sparse=None,
         nbins=None, lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=31,
         max_depth=64, n_threads=0, reference=False, keep_hist=False) -> dict:
    """Grow one tree.  ``reference=True`` runs the compiled reference cgrow
    (fp32 arithmetic only, no traces).  Returns the node arrays trimmed to
    n_nodes, plus rows/seg_lo/seg_hi/split_gain/quant traces for the oracle;
    ``keep_hist``: also "hist", every node's (3, F, 256) histogram as the
    grower scanned it (float32 in MODE_FP32, int64 fixed point in MODE_FIXED)."""
    bins_fm, F, n, grad, hess, fm, use_imat, im, sp, use_sparse, nb = _common_inputs(
        bins_fm, grad, hess, fmask, imat, sparse, nbins)
    nodes = 2 * int(max_leaves) + 1
    out = {k: np.empty(nodes, np.int64) for k in ("feature", "thr_bin", "left", "right", "depth")}
    out["value"] = np.empty(nodes, np.float32)
    scalars = [_flt(float(lam)), _flt(float(gamma)), _flt(float(mcw)), _int(int(msl)),
               _flt(float(lr)), _int(int(max_leaves)), _int(int(max_depth)), _int(int(n_threads))]
    outs = [_ptr(out[k]) for k in ("feature", "thr_bin", "left", "right", "value", "depth")]
    if reference:
        nn = ref_lib().cgrow(_ptr(bins_fm), _ptr(grad), _ptr(hess), _ptr(fm), _ptr(im),
                             _flt(float(ib)), _int(int(use_imat)), *[_ptr(a) for a in sp],
                             _int(use_sparse), _ptr(nb), _i64(n), _int(F), _int(B),
                             *scalars, *outs)
        res = {k: v[:nn] for k, v in out.items()}
        res["n_nodes"] = nn
        return res
    rows = np.empty(max(n, 1), np.int64)
    seg_lo = np.empty(nodes, np.int64)
    seg_hi = np.empty(nodes, np.int64)
    split_gain = np.empty(nodes, np.float64)
    quant = np.zeros(2, np.int32)
    hist = (np.empty((nodes, 3, F, B), np.float32 if mode == MODE_FP32 else np.int64) if keep_hist
            else None)
    nn = lib().or_grow(_int(mode), _ptr(bins_fm), _ptr(grad), _ptr(hess), _ptr(fm), _ptr(im),
                       _flt(float(ib)), _int(int(use_imat)), *[_ptr(a) for a in sp],
                       _int(use_sparse), _ptr(nb), _i64(n), _int(F), *scalars, *outs,
                       _ptr(rows), _ptr(seg_lo), _ptr(seg_hi), _ptr(split_gain), _ptr(quant),
                       _vp(0) if hist is None else _ptr(hist))
    if nn < 0:
        raise ValueError(f"oracle grow failed with status {nn}")
    res = {k: v[:nn] for k, v in out.items()}
    res.update(n_nodes=nn, rows=rows[:n], seg_lo=seg_lo[:nn], seg_hi=seg_hi[:nn],
               split_gain=split_gain[:nn], quant=(int(quant[0]), int(quant[1])))
    if hist is not None:
        res["hist"] = hist[:nn]
    return res


def leaf_of_rows(res: dict, n: int) -> np.ndarray:
    """Per-row leaf node id from an oracle trace (the partition membership)."""
    out = np.full(n, -1, np.int64)
    for nid in range(res["n_nodes"]):
        if res["feature"][nid] == -1:
            out[res["rows"][res["seg_lo"][nid]:res["seg_hi"][nid]]] = nid
    return out


# --------------------------------------------------------------------------
# pieces
# --------------------------------------------------------------------------

def quant_shift(maxabs: float, n: int) -> int:
    return int(lib().or_quant_shift(_flt(float(maxabs)), _i64(int(n))))


def hist_shift(maxabs: float, n: int) -> int:
    """The node histograms' shift (30 - min(k, 11) - e), or_hist_shift."""
    return int(lib().or_hist_shift(_flt(float(maxabs)), _i64(int(n))))


def wide_shift(maxabs: float, n: int) -> int:
    """The wide contract's shift (61 - max(k, 21) - e), or_wide_shift."""
    return int(lib().or_wide_shift(_flt(float(maxabs)), _i64(int(n))))


def hist_contract(grad, hess) -> tuple[int, int, int, tuple[int, int, int, int]]:
    """(sg, sh, wide, (R_g, R_h, M_g, M_h)) of or_hist_contract: the shifts the
    exact grower uses for this g/h, whether they are the wide contract's, and
    the narrow shifts' quantisation residuals and masses that decided it."""
    g = np.ascontiguousarray(grad, np.float32)
    h = np.ascontiguousarray(hess, np.float32)
    out = np.zeros(3, np.int32)
    sums = np.zeros(4, np.uint64)
    if lib().or_hist_contract(_ptr(g), _ptr(h), _i64(g.shape[0]), _ptr(out), _ptr(sums)):
        raise ValueError("non-finite gradient or hessian")
    return int(out[0]), int(out[1]), int(out[2]), tuple(int(v) for v in sums)


def quant_shifts(grad, hess) -> tuple[int, int]:
    g = np.ascontiguousarray(grad, np.float32)
    h = np.ascontiguousarray(hess, np.float32)
    sg = np.zeros(1, np.int32)
    sh = np.zeros(1, np.int32)
    if lib().or_quant_shifts(_ptr(g), _ptr(h), _i64(g.shape[0]), _ptr(sg), _ptr(sh)):
        raise ValueError("non-finite gradient or hessian")
    return int(sg[0]), int(sh[0])


def hist_f32(bins_fm, grad, hess, rows=None) -> np.ndarray:
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    rows = np.arange(n, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, np.int64)
    out = np.empty((3, F, B), np.float32)
    lib().or_hist_f32(_ptr(bins_fm), _ptr(np.ascontiguousarray(grad, np.float32)),
                      _ptr(np.ascontiguousarray(hess, np.float32)), _ptr(rows), _i64(0),
                      _i64(rows.shape[0]), _i64(n), _int(F), _ptr(out))
    return out


def hist_sparse_f32(sparse, grad, hess, F, rows=None) -> np.ndarray:
    indptr = np.ascontiguousarray(sparse[0], np.int64)
    n = indptr.shape[0] - 1
    rows = np.arange(n, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, np.int64)
    arrs = (indptr, np.ascontiguousarray(sparse[1], np.int32),
            np.ascontiguousarray(sparse[2], np.int32), np.ascontiguousarray(sparse[3], np.int32))
    out = np.empty((3, F, B), np.float32)
    lib().or_hist_sparse_f32(*[_ptr(a) for a in arrs],
                             _ptr(np.ascontiguousarray(grad, np.float32)),
                             _ptr(np.ascontiguousarray(hess, np.float32)), _ptr(rows), _i64(0),
                             _i64(rows.shape[0]), _int(F), _ptr(out))
    return out


def hist_fixed(bins_fm, grad, hess, sg, sh, rows=None) -> np.ndarray:
    """Exact int64 histogram, shape (3, F, 256): [sum q(g), sum q(h), count]."""
    bins_fm = np.ascontiguousarray(bins_fm, np.uint8)
    F, n = bins_fm.shape
    rows = np.arange(n, dtype=np.int64) if rows is None else np.ascontiguousarray(rows, np.int64)
    out = np.empty((3, F, B), np.int64)
    lib().or_hist_fixed(_ptr(bins_fm), _ptr(np.ascontiguousarray(grad, np.float32)),
                        _ptr(np.ascontiguousarray(hess, np.float32)), _ptr(rows), _i64(0),
                        _i64(rows.shape[0]), _i64(n), _int(F), _int(sg), _int(sh),
                        _ptr(out[0]), _ptr(out[1]), _ptr(out[2]))
    return out


def best_split_f32(hist, nbins=None, lam=1.0, gamma=0.0, mcw=1e-3, msl=20, fmask=None,
                   boost=None) -> tuple[float, int, int]:
    hist = np.ascontiguousarray(hist, np.float32)
    F = hist.shape[1]
    nb = np.full(F, B, np.int32) if nbins is None else np.ascontiguousarray(nbins, np.int32)
    fm = np.ones(F, np.uint8) if fmask is None else np.ascontiguousarray(fmask, np.uint8)
    bo = np.ones(F, np.float32) if boost is None else np.ascontiguousarray(boost, np.float32)
    f = np.zeros(1, np.int32)
    b = np.zeros(1, np.int32)
    g = lib().or_best_split_f32(_ptr(hist), _ptr(nb), float(np.float32(lam)),
                                float(np.float32(gamma)), float(np.float32(mcw)), int(msl),
                                _ptr(fm), _ptr(bo), _int(F), _ptr(f), _ptr(b))
    return float(g), int(f[0]), int(b[0])


def best_split_fixed(qhist, sg, sh, nbins=None, lam=1.0, gamma=0.0, mcw=1e-3, msl=20,
                     fmask=None, boost=None) -> tuple[float, int, int]:
    qhist = np.ascontiguousarray(qhist, np.int64)
    F = qhist.shape[1]
    nb = np.full(F, B, np.int32) if nbins is None else np.ascontiguousarray(nbins, np.int32)
    fm = np.ones(F, np.uint8) if fmask is None else np.ascontiguousarray(fmask, np.uint8)
    bo = np.ones(F, np.float32) if boost is None else np.ascontiguousarray(boost, np.float32)
    f = np.zeros(1, np.int32)
    b = np.zeros(1, np.int32)
    g = lib().or_best_split_fixed(_ptr(qhist[0]), _ptr(qhist[1]), _ptr(qhist[2]), _int(sg),
                                  _int(sh), _ptr(nb), float(np.float32(lam)),
                                  float(np.float32(gamma)), float(np.float32(mcw)), int(msl),
                                  _ptr(fm), _ptr(bo), _int(F), _ptr(f), _ptr(b))
    return float(g), int(f[0]), int(b[0])


def compute_boost(path, imat, ib) -> np.ndarray:
    path = np.ascontiguousarray(path, np.uint8)
    imat = np.ascontiguousarray(imat, np.float32)
    F = path.shape[0]
    out = np.empty(F, np.float32)
    lib().or_compute_boost(_ptr(path), _ptr(imat), _flt(float(ib)), _ptr(out), _int(F))
    return out


def partition(col, rows, b, stable=False) -> tuple[np.ndarray, int]:
    col = np.ascontiguousarray(col, np.uint8)
    rows = np.array(rows, dtype=np.int64, copy=True)
    m = rows.shape[0]
    if stable:
        tmp = np.empty(max(m, 1), np.int64)
        mid = lib().or_partition_stable(_ptr(col), _ptr(rows), _i64(0), _i64(m), _int(b), _ptr(tmp))
    else:
        mid = lib().or_partition_twoptr(_ptr(col), _ptr(rows), _i64(0), _i64(m), _int(b))
    return rows, int(mid)


def apply(X, feature, threshold, left, right, n_threads=0, reference=False) -> np.ndarray:
    X = np.ascontiguousarray(X, np.float32)
    n, F = X.shape
    arrs = (np.ascontiguousarray(feature, np.int64), np.ascontiguousarray(threshold, np.float32),
            np.ascontiguousarray(left, np.int64), np.ascontiguousarray(right, np.int64))
    out = np.empty(n, np.int64)
    fn = ref_lib().capply if reference else lib().or_apply
    fn(_ptr(X), *[_ptr(a) for a in arrs], _i64(n), _int(F), _int(int(n_threads)), _ptr(out))
    return out
