"""HIP grower: a drop-in for ``grow_tree_c`` (yabt/grow_c.py:336-452).

``grow_tree_hip`` takes exactly ``grow_tree_c``'s arguments and returns the
same ``Tree``; it grows the tree on the GPU through ``yabt_grow``
(include/yabt_hip.h).  Differences from the reference, all deliberate:

* arithmetic: histograms are exact int64 fixed point (see include/yabt_hip.h),
  so results are deterministic and sibling subtraction is exact; the split
  (feature, bin) sequence and leaf membership match the reference grower
  except where the reference's fp32 rounding decides a tie;
* ``sparse_layout``: with exact sums the sparse builder (grow.c:68-107) and
  the dense one give identical histograms, so "exact" ignores it;
  "reference" follows it (cgrow's sparse arithmetic on the layout's default
  bins, which must describe ``binned`` as ``build_sparse_layout`` makes it);
* ``n_threads`` is accepted and ignored (no host threads);
* inputs on the CPU are copied to the current HIP device once per binned
  matrix (cached); the returned Tree lives on ``binned.device`` as in the
  reference.

The module never falls back to a CPU path: if the library or a HIP device is
missing, ``grow_tree_hip`` raises.
"""

from __future__ import annotations

import collections
import ctypes
import threading
import weakref

import numpy as np
import torch

from . import _lib
from .tree import LEAF, Tree, TreeParams

MAX_BINS = 256

_CACHE_LOCK = threading.Lock()
# id(binned) -> (state, layouts); an entry is dropped when its tensor dies (a
# WeakKeyDictionary would compare tensor keys with ==, which is elementwise)
_LAYOUTS: dict[int, tuple] = {}


def _round16(x: int) -> int:
    return (x + 15) // 16 * 16


def _ptr(t: torch.Tensor | None):
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


# Read-only device tensors every call would otherwise rebuild (the all-ones
# feature mask, the unused interaction matrix, an nbins table): made once per
# device and value, complete before first use (the making stream is waited
# for), never written (the C ABI takes them as const).  Shared by every host
# thread under a lock; at most _DEV_CONST_MAX entries, least recently used
# first out.  Each use records the caller's stream on the tensor, so when an
# evicted entry's memory returns to torch's caching allocator it is not
# reused before the kernels already enqueued on those streams have run.
_DEV_CONST: collections.OrderedDict = collections.OrderedDict()
_DEV_CONST_LOCK = threading.Lock()
_DEV_CONST_MAX = 256


def _dev_const(key, make) -> torch.Tensor:
    with _DEV_CONST_LOCK:
        t = _DEV_CONST.get(key)
        if t is None:
            t = make()
            torch.cuda.current_stream(t.device).synchronize()
            _DEV_CONST[key] = t
            if len(_DEV_CONST) > _DEV_CONST_MAX:
                _DEV_CONST.popitem(last=False)
        else:
            _DEV_CONST.move_to_end(key)
        t.record_stream(torch.cuda.current_stream(t.device))
        return t


def _dev_f32(t: torch.Tensor, dev: torch.device) -> torch.Tensor:
    """Contiguous float32 copy on ``dev`` whose data is 16-byte aligned (the
    kernels use 16-byte vector loads)."""
    t = t.detach().to(dev, torch.float32).contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("yabt_amd: no HIP device available")
    return torch.device("cuda", torch.cuda.current_device())


class BinLayouts:
    """Both device layouts of one binned matrix: feature-major (F, ld_fm) for
    streaming and partitions, row-major (n, ld_rm) for gathered child nodes."""

    def __init__(self, fm: torch.Tensor, rm: torch.Tensor, n: int, F: int):
        self.fm, self.rm, self.n, self.F = fm, rm, n, F
        self.ld_fm = fm.shape[1]
        self.ld_rm = rm.shape[1]
        self._default = None
        self._counts = None
        self._root_order = None
        # The lazily made tables below are shared by every host thread that
        # grows on this layout, each on its own stream: one thread makes a
        # table under the lock, waits for its stream, and only then publishes
        # it, so a kernel on another stream never reads it half written.
        self._lock = threading.Lock()

    def _publish(self, t: torch.Tensor) -> torch.Tensor:
        torch.cuda.current_stream(self.fm.device).synchronize()
        return t

    def counts(self) -> torch.Tensor:
        """The per-fit count table of the bins (yabt_bin_counts), made once
        per layout: the per-(feature, bin) row counts (F, 256) uint32, the
        count plane of every root histogram over these bins, which the
        growers take instead of recounting the rows each tree, then each
        feature's largest bin count per 65536-row segment, which tells the
        root which row chunks need no epochs."""
        if self._counts is None:
            with self._lock:
                if self._counts is None:
                    lib = _lib.load()
                    dev = self.fm.device
                    words = int(lib.yabt_bin_counts_words(self.n, self.F))
                    c = torch.empty(words, dtype=torch.int32, device=dev)
                    _lib.check(lib.yabt_bin_counts(_ptr(self.fm), self.ld_fm, self.n, self.F, _ptr(c),
                                                   _stream(dev)), "yabt_bin_counts")
                    self._counts = self._publish(c)
        return self._counts

    def ref_root_order(self) -> torch.Tensor:
        """The root rank table of the reference-arithmetic grower's dense
        builder (yabt_ref_root_order), built once per layout: each row's rank
        in its bin inside its 4096-row tile, per feature, which every tree's
        root histogram on these bins reuses.  F * ceil(n / 4096) * 4096
        uint16 ranks plus the tiles' bin starts (yabt_ref_root_order_bytes):
        2.0 GB at 10M rows x 100 features, kept until the layout dies or
        release_ref_root_order() drops it."""
        if self._root_order is None:
            with self._lock:
                if self._root_order is None:
                    lib = _lib.load()
                    dev = self.fm.device
                    nbytes = int(lib.yabt_ref_root_order_bytes(self.n, self.F))
                    if nbytes == 0:
                        raise ValueError("yabt_ref_root_order: invalid sizes")
                    buf = torch.empty(nbytes, dtype=torch.uint8, device=dev)
                    _lib.check(lib.yabt_ref_root_order(_ptr(self.fm), self.ld_fm, self.n, self.F, _ptr(buf),
                                                       nbytes, _stream(dev)), "yabt_ref_root_order")
                    self._root_order = self._publish(buf)
        return self._root_order

    def release_ref_root_order(self) -> None:
        """Drop the reference-arithmetic root rank table (the largest per-fit
        table, see ref_root_order); the next reference-arithmetic tree on this
        layout rebuilds it.  Call it when no grower on this layout is running:
        the memory goes back to torch's caching allocator (the device is
        waited for first, so no enqueued kernel can still read it)."""
        with self._lock:
            if self._root_order is not None:
                torch.cuda.synchronize(self.fm.device)
                self._root_order = None

    # a default bin is skipped only where it holds at least this share of the
    # sampled rows; below it the per-update test costs more than it saves
    SKIP_MIN_SHARE = 0.125

    def default_bin(self, sample: int = 65536) -> torch.Tensor | None:
        """Most frequent bin per feature over an evenly spaced row sample (the
        sparse layout's default bin, grow_numba.py:341-367, estimated), -1 for
        features whose modal bin holds under SKIP_MIN_SHARE of the sample, or
        None when no feature qualifies.  Any choice gives identical
        histograms; this one skips the most rows where skipping pays."""
        if self._default is None:
            with self._lock:
                if self._default is None:
                    self._default = self._make_default_bin(sample)
        return self._default if self._default is not False else None

    def _make_default_bin(self, sample: int):
        F, n = self.F, self.n
        if n == 0:
            return False
        idx = torch.linspace(0, n - 1, min(n, sample), device=self.fm.device).long()
        cols = self.fm[:, idx].long()                       # (F, s)
        counts = torch.zeros((F, MAX_BINS), dtype=torch.int64, device=self.fm.device)
        counts.scatter_add_(1, cols, torch.ones_like(cols))
        top, arg = counts.max(dim=1)
        frequent = top.double() >= self.SKIP_MIN_SHARE * idx.numel()
        if not bool(frequent.any()):   # waits for the stream
            return False
        return self._publish(torch.where(frequent, arg, torch.full_like(arg, -1)).to(torch.int32).contiguous())


def make_layouts(binned: torch.Tensor, dev: torch.device,
                 binned_fmajor: np.ndarray | None = None) -> BinLayouts:
    """Device copies of binned (n, F) uint8 in both padded layouts."""
    n, F = binned.shape
    ld_fm, ld_rm = max(16, _round16(n)), _lib.row_stride(F)
    fm = torch.zeros((F, ld_fm), dtype=torch.uint8, device=dev)
    if binned_fmajor is not None:
        fm[:, :n].copy_(torch.from_numpy(np.ascontiguousarray(binned_fmajor, dtype=np.uint8)))
    else:
        fm[:, :n].copy_(binned.to(dev, torch.uint8).t())
    rm = torch.zeros((max(n, 1), ld_rm), dtype=torch.uint8, device=dev)
    lib = _lib.load()
    _lib.check(lib.yabt_transpose_bins(_ptr(fm), ld_fm, n, F, _ptr(rm), ld_rm, _stream(dev)),
               "yabt_transpose_bins")
    # the copies and the transpose ran on this thread's stream; the layouts
    # may be used from other streams next (layouts_for shares them)
    torch.cuda.current_stream(dev).synchronize()
    return BinLayouts(fm, rm, n, F)


def layouts_for(binned: torch.Tensor, dev: torch.device,
                binned_fmajor: np.ndarray | None = None) -> BinLayouts:
    """Cached per binned tensor (keyed by object, checked against its version),
    mirroring the reference's cached feature-major copy (boosting.py:454-459)."""
    key_state = (binned._version, binned.data_ptr(), tuple(binned.shape), dev)
    key = id(binned)
    with _CACHE_LOCK:
        hit = _LAYOUTS.get(key)
        if hit is not None and hit[0] == key_state:
            return hit[1]
    lay = make_layouts(binned, dev, binned_fmajor)
    with _CACHE_LOCK:
        if key not in _LAYOUTS:
            # runs when binned dies, before its id can be reused
            weakref.finalize(binned, _LAYOUTS.pop, key, None)
        _LAYOUTS[key] = (key_state, lay)
    return lay


def _workspace(dev: torch.device, nbytes: int) -> torch.Tensor:
    """Device workspace of one grow call, from torch's caching allocator on
    the current stream (reused across calls without new allocations; each
    call, and each host thread on its own stream, gets its own, as cgrow
    takes its scratch per call, grow.c:271-287)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev)


def nbins_of(binner, F: int) -> np.ndarray:
    """Used bins per feature, min(len(edges)+1, 256) (grow_c.py:395-401)."""
    nb = getattr(binner, "_c_nbins", None)
    if nb is None or nb.shape[0] != F:
        nb = np.fromiter((min(len(e) + 1, MAX_BINS) for e in binner.edges_), dtype=np.int32, count=F)
        binner._c_nbins = nb
    return nb


class GrowResult:
    """Device outputs of one yabt_grow call (node arrays trimmed to n_nodes)."""

    def __init__(self, feature, thr_bin, left, right, value, depth, n_nodes, workspace, status):
        self.feature, self.thr_bin, self.left, self.right = feature, thr_bin, left, right
        self.value, self.depth, self.n_nodes = value, depth, n_nodes
        self._ws, self._status = workspace, status


ARITHMETICS = ("exact", "reference")
GROWTHS = ("auto", "sequential", "levelwise", "rounds")
ROUNDS_MAX_LEAVES = 1024


def grow_device(lay: BinLayouts, grad: torch.Tensor, hess: torch.Tensor, nbins: np.ndarray, *,
                fmask=None, imat=None, ib: float = 0.5, lam=1.0, gamma=0.0, mcw=1e-3, msl=20,
                lr=0.1, max_leaves=31, max_depth=64, default_bin="auto",
                sync: bool = True, arithmetic: str = "exact", batched: bool | None = None,
                growth: str = "auto") -> GrowResult:
    """One grow call on device-resident layouts.  grad/hess must be on the
    layouts' device; parameters are rounded to float32 as ctypes.c_float
    rounds them in the reference (grow_c.py:418-421).

    ``arithmetic``: "exact" (yabt_grow: exact fixed-point sums, the whole
    tree on the device) or "reference" (yabt_grow_ref: cgrow's own fp32
    arithmetic and row order, the same trees as the reference bit for bit,
    one host round trip per round of up to 16 splits).

    ``growth`` ("exact" only; every choice gives the same tree bit for bit):
    "sequential" (yabt_grow, one split per launch triple, all on the
    device), "levelwise" (yabt_grow_levelwise: depth by depth, needs
    max_leaves >= 2^max_depth so that the leaf budget cannot bind), "rounds"
    (yabt_grow_batched: up to 16 splits per round, max_leaves <= 1024), or
    "auto": levelwise where the budget cannot bind, else rounds, else
    sequential.  ``batched`` True / False is the older spelling of
    "levelwise" / "sequential".

    ``default_bin``: with "exact" (not levelwise) a shortcut that leaves the
    sums unchanged -- "auto" uses the layouts' most frequent bin per feature,
    None disables the skip, or an (F,) int array.  With "reference" it picks
    cgrow's histogram builder: an (F,) array of default bins in [0, 255] is
    the sparse builder (grow.c:68-107) over those bins; "auto" or None is the
    dense builder."""
    if arithmetic not in ARITHMETICS:
        raise ValueError(f"arithmetic must be one of {ARITHMETICS}")
    if arithmetic == "reference":
        db = None if default_bin is None or isinstance(default_bin, str) else default_bin
        return _grow_device_ref(lay, grad, hess, nbins, fmask=fmask, imat=imat, ib=ib, lam=lam, gamma=gamma,
                                mcw=mcw, msl=msl, lr=lr, max_leaves=max_leaves, max_depth=max_depth,
                                default_bin=db)
    can_batch = 0 <= int(max_depth) <= 16 and int(max_leaves) >= (1 << int(max_depth)) and int(max_leaves) <= 65535
    if batched is not None:
        growth = "levelwise" if batched else "sequential"
    if growth not in GROWTHS:
        raise ValueError(f"growth must be one of {GROWTHS}")
    if growth == "auto":
        if can_batch and lay.n < 2 ** 31:
            growth = "levelwise"
        elif int(max_leaves) <= ROUNDS_MAX_LEAVES and lay.n <= 0xFFFFFFFF:
            growth = "rounds"
        else:
            growth = "sequential"
    if growth == "levelwise":
        if not can_batch:
            raise ValueError("batched growth needs max_leaves >= 2^max_depth and max_depth <= 16")
        return _grow_device_level(lay, grad, hess, nbins, fmask=fmask, imat=imat, ib=ib, lam=lam, gamma=gamma,
                                  mcw=mcw, msl=msl, lr=lr, max_leaves=max_leaves, max_depth=max_depth)
    rounds = growth == "rounds"
    if rounds and int(max_leaves) > ROUNDS_MAX_LEAVES:
        raise ValueError(f"growth in rounds needs max_leaves <= {ROUNDS_MAX_LEAVES}")
    lib = _lib.load()
    dev = lay.fm.device
    n, F = lay.n, lay.F
    g = _dev_f32(grad, dev)
    h = _dev_f32(hess, dev)
    if g.shape[0] != n or h.shape[0] != n:
        raise ValueError("grad/hess length must equal the number of rows")
    fm = (_dev_const((dev, "ones_u8", F), lambda: torch.ones(F, dtype=torch.uint8, device=dev)) if fmask is None
          else torch.as_tensor(fmask).to(dev).bool().to(torch.uint8).contiguous())
    use_imat = imat is not None
    im = (torch.as_tensor(imat).to(dev, torch.float32).contiguous() if use_imat
          else _dev_const((dev, "zero_f32"), lambda: torch.zeros(1, dtype=torch.float32, device=dev)))
    if use_imat and tuple(im.shape) != (F, F):
        raise ValueError("interaction_matrix must be (F, F)")
    nbc = np.ascontiguousarray(nbins, dtype=np.int32)
    nb = _dev_const((dev, "nbins", nbc.tobytes()), lambda: torch.from_numpy(nbc.copy()).to(dev))
    if isinstance(default_bin, str):
        db = lay.default_bin()
    elif default_bin is None:
        db = None
    else:
        db = torch.as_tensor(np.asarray(default_bin, np.int32)).to(dev)
    L = int(max_leaves)
    N = 2 * L + 1
    if rounds:
        return _grow_device_rounds(lib, lay, g, h, fm, im, use_imat, nb, db, ib=ib, lam=lam, gamma=gamma,
                                   mcw=mcw, msl=msl, lr=lr, max_leaves=L, max_depth=max_depth)
    nbytes = int(lib.yabt_grow_workspace_bytes(n, F, L))
    if nbytes == 0:
        raise ValueError("yabt_grow: invalid sizes")
    ws = _workspace(dev, nbytes)
    out_i = torch.empty((5, N), dtype=torch.int64, device=dev)
    value = torch.empty(N, dtype=torch.float32, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = lib.yabt_grow(
        _ptr(lay.fm), lay.ld_fm, _ptr(lay.rm), lay.ld_rm, _ptr(g), _ptr(h), _ptr(fm), _ptr(im),
        ctypes.c_float(float(ib)), int(use_imat), _ptr(nb), _ptr(db), _ptr(lay.counts()), n, F,
        ctypes.c_float(float(lam)), ctypes.c_float(float(gamma)), ctypes.c_float(float(mcw)),
        int(msl), ctypes.c_float(float(lr)), L, int(max_depth), _ptr(ws), ws.numel(),
        _ptr(out_i[0]), _ptr(out_i[1]), _ptr(out_i[2]), _ptr(out_i[3]), _ptr(value),
        _ptr(out_i[4]), _ptr(status), _stream(dev))
    _lib.check(rc, "yabt_grow")
    # per-row leaf ids now, while the workspace still holds this tree's rows
    leaf = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    if n > 0:
        _lib.check(lib.yabt_grow_leaf_ids(_ptr(ws), n, F, L, _ptr(out_i[0]), _ptr(out_i[4]), _ptr(status),
                                          _ptr(leaf), _stream(dev)), "yabt_grow_leaf_ids")
    res = GrowResult(out_i[0], out_i[1], out_i[2], out_i[3], value, out_i[4], None, None, status)
    res.leaf_of_row = leaf[:n]
    res._keep = (g, h, fm, im, nb, db, ws)   # alive until sync=False callers are done with the stream
    if sync:
        nn = int(status.item())
        if nn < 0:
            raise ValueError("yabt_grow: gradients or hessians contain non-finite values")
        res.n_nodes = nn
        for k in ("feature", "thr_bin", "left", "right", "value", "depth"):
            setattr(res, k, getattr(res, k)[:nn])
    return res


def _grow_device_rounds(lib, lay: BinLayouts, g, h, fm, im, use_imat, nb, db, *, ib, lam, gamma, mcw, msl, lr,
                        max_leaves, max_depth) -> GrowResult:
    """yabt_grow_batched: yabt_grow's tree with up to 16 splits per round
    (synchronous); per-row leaf ids come with it."""
    dev = lay.fm.device
    n, F = lay.n, lay.F
    L = int(max_leaves)
    N = 2 * L + 1
    nbytes = int(lib.yabt_grow_batched_workspace_bytes(n, F, L))
    if nbytes == 0:
        raise ValueError("yabt_grow_batched: invalid sizes")
    ws = _workspace(dev, nbytes)
    out_i = torch.empty((5, N), dtype=torch.int64, device=dev)
    value = torch.empty(N, dtype=torch.float32, device=dev)
    leaf = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    status = torch.empty(3, dtype=torch.int32, device=dev)   # cleared by the grower's set-up launch
    rc = lib.yabt_grow_batched(
        _ptr(lay.fm), lay.ld_fm, _ptr(lay.rm), lay.ld_rm, _ptr(g), _ptr(h), _ptr(fm), _ptr(im),
        ctypes.c_float(float(ib)), int(use_imat), _ptr(nb), _ptr(db), _ptr(lay.counts()), n, F,
        ctypes.c_float(float(lam)), ctypes.c_float(float(gamma)), ctypes.c_float(float(mcw)),
        int(msl), ctypes.c_float(float(lr)), L, int(max_depth), _ptr(ws), ws.numel(),
        _ptr(out_i[0]), _ptr(out_i[1]), _ptr(out_i[2]), _ptr(out_i[3]), _ptr(value), _ptr(out_i[4]),
        _ptr(leaf), _ptr(status), _stream(dev))
    _lib.check(rc, "yabt_grow_batched")
    k, rounds, computed = (int(v) for v in status.cpu())
    if k == -1:
        raise ValueError("yabt_grow: gradients or hessians contain non-finite values")
    if k < 0:
        raise RuntimeError(f"yabt_grow_batched failed ({k})")
    res = GrowResult(out_i[0][:k], out_i[1][:k], out_i[2][:k], out_i[3][:k], value[:k], out_i[4][:k], k, ws,
                     status)
    res.leaf_of_row = leaf[:n]
    res.rounds, res.splits_computed = rounds, computed
    return res


def _grow_device_level(lay: BinLayouts, grad, hess, nbins, *, fmask, imat, ib, lam, gamma, mcw, msl, lr,
                       max_leaves, max_depth) -> GrowResult:
    """yabt_grow_levelwise: depth-batched growth, yabt_grow's tree (synchronous)."""
    lib = _lib.load()
    dev = lay.fm.device
    n, F = lay.n, lay.F
    g = _dev_f32(grad, dev)
    h = _dev_f32(hess, dev)
    if g.shape[0] != n or h.shape[0] != n:
        raise ValueError("grad/hess length must equal the number of rows")
    fm = (_dev_const((dev, "ones_u8", F), lambda: torch.ones(F, dtype=torch.uint8, device=dev)) if fmask is None
          else torch.as_tensor(fmask).to(dev).bool().to(torch.uint8).contiguous())
    use_imat = imat is not None
    im = (torch.as_tensor(imat).to(dev, torch.float32).contiguous() if use_imat
          else _dev_const((dev, "zero_f32"), lambda: torch.zeros(1, dtype=torch.float32, device=dev)))
    if use_imat and tuple(im.shape) != (F, F):
        raise ValueError("interaction_matrix must be (F, F)")
    nbc = np.ascontiguousarray(nbins, dtype=np.int32)
    nb = _dev_const((dev, "nbins", nbc.tobytes()), lambda: torch.from_numpy(nbc.copy()).to(dev))
    L = int(max_leaves)
    N = 2 * L + 1
    nbytes = int(lib.yabt_grow_levelwise_workspace_bytes(n, F, L, int(max_depth)))
    if nbytes == 0:
        raise ValueError("yabt_grow_levelwise: invalid sizes")
    ws = _workspace(dev, nbytes)
    out_i = torch.empty((5, N), dtype=torch.int64, device=dev)
    value = torch.empty(N, dtype=torch.float32, device=dev)
    leaf = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    status = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = lib.yabt_grow_levelwise(
        _ptr(lay.fm), lay.ld_fm, _ptr(lay.rm), lay.ld_rm, _ptr(g), _ptr(h), _ptr(fm), _ptr(im),
        ctypes.c_float(float(ib)), int(use_imat), _ptr(nb), _ptr(lay.counts()), n, F,
        ctypes.c_float(float(lam)), ctypes.c_float(float(gamma)), ctypes.c_float(float(mcw)),
        int(msl), ctypes.c_float(float(lr)), L, int(max_depth), _ptr(ws), ws.numel(),
        _ptr(out_i[0]), _ptr(out_i[1]), _ptr(out_i[2]), _ptr(out_i[3]), _ptr(value), _ptr(out_i[4]),
        _ptr(leaf), _ptr(status), _stream(dev))
    _lib.check(rc, "yabt_grow_levelwise")
    k = int(status.item())
    if k < 0:
        raise ValueError("yabt_grow: gradients or hessians contain non-finite values")
    res = GrowResult(out_i[0][:k], out_i[1][:k], out_i[2][:k], out_i[3][:k], value[:k], out_i[4][:k], k, ws,
                     status)
    res.leaf_of_row = leaf[:n]
    return res


def _grow_device_ref(lay: BinLayouts, grad, hess, nbins, *, fmask, imat, ib, lam, gamma, mcw, msl, lr,
                     max_leaves, max_depth, default_bin=None, workspace_bytes=None,
                     root_order: bool = True) -> GrowResult:
    """yabt_grow_ref: cgrow's arithmetic on the device (synchronous);
    default_bin selects cgrow's sparse builder.  workspace_bytes (None: the
    library's recommended size) may be anything from
    yabt_grow_ref_workspace_min_bytes up: features are bucketed in groups
    that fit.  root_order: the dense builder's root reads the layout's cached
    rank table (BinLayouts.ref_root_order) instead of bucketing every tree."""
    lib = _lib.load()
    dev = lay.fm.device
    n, F = lay.n, lay.F
    g = _dev_f32(grad, dev)
    h = _dev_f32(hess, dev)
    if g.shape[0] != n or h.shape[0] != n:
        raise ValueError("grad/hess length must equal the number of rows")
    fm = (_dev_const((dev, "ones_u8", F), lambda: torch.ones(F, dtype=torch.uint8, device=dev)) if fmask is None
          else torch.as_tensor(fmask).to(dev).bool().to(torch.uint8).contiguous())
    use_imat = imat is not None
    im = (torch.as_tensor(imat).to(dev, torch.float32).contiguous() if use_imat
          else _dev_const((dev, "zero_f32"), lambda: torch.zeros(1, dtype=torch.float32, device=dev)))
    if use_imat and tuple(im.shape) != (F, F):
        raise ValueError("interaction_matrix must be (F, F)")
    nbc = np.ascontiguousarray(nbins, dtype=np.int32)
    nb = _dev_const((dev, "nbins", nbc.tobytes()), lambda: torch.from_numpy(nbc.copy()).to(dev))
    db = None
    if default_bin is not None:
        db = torch.as_tensor(default_bin).to(dev, torch.int32).contiguous()
        if tuple(db.shape) != (F,):
            raise ValueError("default_bin must have one entry per feature")
    L = int(max_leaves)
    N = 2 * L + 1
    nbytes = int(lib.yabt_grow_ref_workspace_bytes(n, F, L, int(db is not None)))
    if nbytes == 0:
        raise ValueError("yabt_grow_ref: invalid sizes")
    if workspace_bytes is not None:
        nbytes = int(workspace_bytes)
    ws = _workspace(dev, nbytes)
    ro = lay.ref_root_order() if (root_order and db is None and n > 0) else None
    out_i = torch.empty((5, N), dtype=torch.int64, device=dev)
    value = torch.empty(N, dtype=torch.float32, device=dev)
    leaf = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    rows = torch.empty(max(n, 1), dtype=torch.int64, device=dev)
    nn = torch.zeros(1, dtype=torch.int32, device=dev)
    rc = lib.yabt_grow_ref(
        _ptr(lay.fm), lay.ld_fm, _ptr(lay.rm), lay.ld_rm, _ptr(g), _ptr(h), _ptr(fm), _ptr(im),
        ctypes.c_float(float(ib)), int(use_imat), _ptr(nb), _ptr(db), n, F,
        ctypes.c_float(float(lam)), ctypes.c_float(float(gamma)), ctypes.c_float(float(mcw)),
        int(msl), ctypes.c_float(float(lr)), L, int(max_depth), _ptr(ws), nbytes, _ptr(ro),
        _ptr(out_i[0]), _ptr(out_i[1]), _ptr(out_i[2]), _ptr(out_i[3]), _ptr(value), _ptr(out_i[4]),
        _ptr(leaf), _ptr(rows), _ptr(nn), _stream(dev))
    _lib.check(rc, "yabt_grow_ref")
    k = int(nn.item())
    res = GrowResult(out_i[0][:k], out_i[1][:k], out_i[2][:k], out_i[3][:k], value[:k], out_i[4][:k], k, ws, nn)
    res.leaf_of_row = leaf[:n]
    res.rows = rows[:n]
    return res


def leaf_ids(res: GrowResult, n: int, F: int, max_leaves: int) -> torch.Tensor:
    """Per-row leaf node ids of a grown tree, from its final partition (every
    grower fills them when it returns, so a later grow cannot change them)."""
    del F, max_leaves
    out = res.leaf_of_row
    if out.shape[0] != n:
        raise ValueError(f"leaf_ids: the tree was grown on {out.shape[0]} rows, not {n}")
    return out


def _edge_table(binner, F: int, dev: torch.device):
    """(F, 256) float32 table with edge_value(f, b) = edges_f[min(b, len-1)]
    (binning.py:126-129), cached on the binner per device."""
    cache = getattr(binner, "_hip_edge_table", None)
    if cache is not None and cache[0] == dev and cache[1].shape[0] == F:
        return cache[1], cache[2]
    tab = np.zeros((F, MAX_BINS), dtype=np.float32)
    for f, e in enumerate(binner.edges_):
        e = np.asarray(e.cpu() if isinstance(e, torch.Tensor) else e, dtype=np.float32)
        if e.size == 0:
            continue  # no edges: no split on f can be chosen (nbins == 1)
        idx = np.minimum(np.arange(MAX_BINS), e.size - 1)
        tab[f] = e[idx]
    scales = torch.as_tensor(binner.scales_, dtype=torch.float32).clamp_min(1e-12)
    out = (torch.from_numpy(tab).to(dev), scales.to(dev))
    binner._hip_edge_table = (dev, out[0], out[1])
    return out


def grow_tree_hip(
    binned: torch.Tensor,
    grad: torch.Tensor,
    hess: torch.Tensor,
    binner,
    params: TreeParams,
    feature_mask: torch.Tensor | None = None,
    interaction_matrix: torch.Tensor | None = None,
    interaction_boost: float = 0.5,
    sparse_layout=None,
    n_threads: int = 0,
    binned_fmajor: np.ndarray | None = None,
    arithmetic: str = "exact",
) -> Tree:
    """Drop-in for ``grow_tree_c`` (yabt/grow_c.py:336-452) on a HIP device;
    ``arithmetic`` as in ``grow_device`` ("reference": cgrow's trees bit for
    bit, with cgrow's sparse builder when ``sparse_layout`` is given,
    grow_c.py:382-393)."""
    del n_threads  # see module docstring
    out_dev = binned.device
    dev = binned.device if binned.device.type == "cuda" else _device()
    n, F = binned.shape
    lay = layouts_for(binned, dev, binned_fmajor)
    db = "auto"
    if sparse_layout is not None and arithmetic == "reference":
        db = np.ascontiguousarray(sparse_layout[3], dtype=np.int64)
        if db.shape != (F,) or db.min(initial=0) < 0 or db.max(initial=0) >= MAX_BINS:
            raise ValueError("sparse_layout's default bins must be (F,) in [0, 255]")
    res = grow_device(lay, grad, hess, nbins_of(binner, F), fmask=feature_mask,
                      imat=interaction_matrix, ib=interaction_boost, lam=params.reg_lambda,
                      gamma=params.gamma, mcw=params.min_child_weight,
                      msl=params.min_samples_leaf, lr=params.learning_rate,
                      max_leaves=params.max_leaves, max_depth=params.max_depth, default_bin=db,
                      arithmetic=arithmetic)
    return tree_from_result(res, binner, F, out_dev)


def tree_from_result(res: GrowResult, binner, F: int, out_dev: torch.device) -> Tree:
    """Thresholds and gate scales from the binner (grow_c.py:435-452)."""
    dev = res.feature.device
    tab, scales = _edge_table(binner, F, dev)
    feat = res.feature
    internal = feat != LEAF
    fc = feat.clamp(min=0)
    threshold = torch.where(internal, tab[fc, res.thr_bin.clamp(0, MAX_BINS - 1)],
                            torch.zeros((), device=dev))
    gate = torch.where(internal, scales[fc], torch.ones((), device=dev))
    depth = int(res.depth.max()) + 1
    return Tree(feature=feat.to(out_dev), threshold=threshold.to(out_dev), left=res.left.to(out_dev),
                right=res.right.to(out_dev), value=res.value.to(out_dev), depth=depth,
                gate_scale=gate.to(out_dev))


def apply_hip(X: torch.Tensor, feature: torch.Tensor, threshold: torch.Tensor,
              left: torch.Tensor, right: torch.Tensor) -> torch.Tensor:
    """Leaf index per row of raw X on the GPU; drop-in for ``apply_c``
    (yabt/grow_c.py:305-333)."""
    lib = _lib.load()
    dev = X.device if X.device.type == "cuda" else _device()
    Xd = X.detach().to(dev, torch.float32).contiguous()
    n, F = Xd.shape
    fe = feature.to(dev, torch.int64).contiguous()
    th = threshold.to(dev, torch.float32).contiguous()
    le = left.to(dev, torch.int64).contiguous()
    ri = right.to(dev, torch.int64).contiguous()
    out = torch.empty(n, dtype=torch.int64, device=dev)
    if n > 0:
        _lib.check(lib.yabt_apply(_ptr(Xd), F, n, F, _ptr(fe), _ptr(th), _ptr(le), _ptr(ri),
                                  int(fe.shape[0]), _ptr(out), _stream(dev)), "yabt_apply")
    return out.to(X.device)


def is_available() -> bool:
    return _lib.is_available()


# ---------------------------------------------------------------------------
# per-stage entry points (exposed for tests and benchmarks)
# ---------------------------------------------------------------------------

def hist(lay: BinLayouts, grad: torch.Tensor, hess: torch.Tensor,
         rows: torch.Tensor | None = None) -> tuple[torch.Tensor, tuple[int, int, int]]:
    """Exact (3, F, 256) int64 histogram over ``rows`` (uint32/int) or all rows,
    with the shifts and the contract (sg, sh, wide) chosen from grad/hess."""
    lib = _lib.load()
    dev = lay.fm.device
    g = _dev_f32(grad, dev)
    h = _dev_f32(hess, dev)
    r = None if rows is None else rows.to(dev, torch.int32).contiguous()
    m = 0 if r is None else r.shape[0]
    if r is not None and m == 0:
        r = torch.zeros(1, dtype=torch.int32, device=dev)  # non-NULL: "no rows", not "all rows"
    out = torch.empty((3, lay.F, MAX_BINS), dtype=torch.int64, device=dev)
    shifts = torch.zeros(3, dtype=torch.int32, device=dev)
    ws = torch.empty(int(lib.yabt_hist_workspace_bytes()), dtype=torch.uint8, device=dev)
    _lib.check(lib.yabt_hist(_ptr(lay.fm), lay.ld_fm, _ptr(lay.rm), lay.ld_rm, _ptr(g), _ptr(h),
                             lay.n, lay.F, _ptr(r), m, _ptr(ws), _ptr(out), _ptr(shifts),
                             _stream(dev)), "yabt_hist")
    s = shifts.cpu().tolist()
    return out, (int(s[0]), int(s[1]), int(s[2]))


def ref_root_hist(lay: BinLayouts, grad: torch.Tensor, hess: torch.Tensor) -> torch.Tensor:
    """The root's (3, F, 256) float32 histogram in the reference arithmetic
    (cgrow's row-order fp32 sums, grow.c:37-62), from the layout's cached
    root rank table."""
    lib = _lib.load()
    dev = lay.fm.device
    g = _dev_f32(grad, dev)
    h = _dev_f32(hess, dev)
    ro = lay.ref_root_order()
    out = torch.empty((3, lay.F, MAX_BINS), dtype=torch.float32, device=dev)
    _lib.check(lib.yabt_ref_root_hist(_ptr(lay.fm), lay.ld_fm, _ptr(g), _ptr(h), lay.n, lay.F, _ptr(ro),
                                      ro.numel(), _ptr(out), _stream(dev)), "yabt_ref_root_hist")
    return out


def best_split(qhist: torch.Tensor, sg: int, sh: int, nbins=None, lam=1.0, gamma=0.0, mcw=1e-3,
               msl=20, fmask=None, boost=None) -> tuple[float, int, int]:
    lib = _lib.load()
    dev = qhist.device
    F = qhist.shape[1]
    nb = (torch.full((F,), MAX_BINS, dtype=torch.int32, device=dev) if nbins is None
          else torch.as_tensor(np.asarray(nbins, np.int32)).to(dev))
    fm = (torch.ones(F, dtype=torch.uint8, device=dev) if fmask is None
          else torch.as_tensor(np.asarray(fmask).astype(np.uint8)).to(dev))
    bo = None if boost is None else torch.as_tensor(np.asarray(boost, np.float32)).to(dev)
    ws = torch.empty(int(lib.yabt_best_split_workspace_bytes(F)), dtype=torch.uint8, device=dev)
    og = torch.empty(1, dtype=torch.float64, device=dev)
    ofb = torch.empty(2, dtype=torch.int32, device=dev)
    q = qhist.contiguous()
    _lib.check(lib.yabt_best_split(_ptr(q), F, _ptr(nb), _ptr(fm), _ptr(bo), int(sg), int(sh),
                                   float(np.float32(lam)), float(np.float32(gamma)),
                                   float(np.float32(mcw)), int(msl), _ptr(ws), _ptr(og), _ptr(ofb),
                                   _stream(dev)), "yabt_best_split")
    fb = ofb.cpu().tolist()
    return float(og.item()), int(fb[0]), int(fb[1])


def partition(lay: BinLayouts, f: int, b: int,
              rows: torch.Tensor | None = None, m: int | None = None) -> tuple[torch.Tensor, int]:
    lib = _lib.load()
    dev = lay.fm.device
    r = None if rows is None else rows.to(dev, torch.int32).contiguous()
    mm = (lay.n if m is None else int(m)) if r is None else r.shape[0]
    if r is not None and mm == 0:
        r = torch.zeros(1, dtype=torch.int32, device=dev)  # non-NULL: "no rows", not "positions"
    out = torch.empty(max(mm, 1), dtype=torch.int32, device=dev)
    ws = torch.empty(int(lib.yabt_partition_workspace_bytes()), dtype=torch.uint8, device=dev)
    mid = torch.zeros(1, dtype=torch.int64, device=dev)
    _lib.check(lib.yabt_partition(_ptr(lay.fm), lay.ld_fm, lay.n, int(f), int(b), _ptr(r), mm,
                                  _ptr(out), _ptr(ws), _ptr(mid), _stream(dev)), "yabt_partition")
    return out[:mm], int(mid.item())
