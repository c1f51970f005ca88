"""Benchmark of the HIP tree-growing path on one MI355X.

Workload: one best-first tree over a dense binned matrix of 10 000 000 rows x
100 features of uint8 bins uniform on 0..255, gradients N(0,1), hessians
U(0.1,1) (fp32), 255 leaves, min_samples_leaf 20, min_child_weight 1e-3,
lambda 1, gamma 0, lr 0.1, identity binner (nbins 256).  Inputs are generated
on the device and resident in HBM before timing.

A step is one full tree: root histogram, 254 splits (partition + smaller
child histogram + sibling subtraction + split scans; grown in rounds of up
to 16 computed splits, committed in best-first order), then the linear leaf
models (K = 8 most used split features, raw input x = float(bin), g and h at
margin + value[leaf] for a quadratic objective: g + h * value[leaf], h;
min 50 rows, l2 1).  ``value`` is the tree's histogram work, sum over built
nodes of rows x features (row.feature updates), divided by the measured time
per step, in G updates/s; ``ms_grow`` is the same loop without the leaf
models.

Also reported:
  * root_hist: the streaming root-histogram kernel timed alone with HIP events
    (10M x 100 = 1.0e9 updates per launch); ``roofline`` is computed from it:
    algorithmic bytes per launch = n*F (bins) + 8n (fp32 g, h) = 1.08 GB;
  * cpu_baseline: the reference grow.c (compiled from the reference sources
    into oracle/_ref/, kind "reference") or, if that library is absent, the
    oracle's restatement of it (kind "port"), on one tree of the full
    10M x 100 workload (host RNG inputs of the same distribution), timed on
    this host's cores with the host's CPU model and core count.

``roofline.traffic`` (HBM bytes per root-histogram launch) is read from the
committed counter summary profiles/k_hist_root_10Mx100_traffic.md, made by two
rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE) over ``bench.py --counters``,
which launches a plain copy kernel of known size (for the counter scale) and
the root-histogram kernel, three times each.

Also reported, outside the timed region: ``reference_arithmetic`` (the same
tree grown with the reference's own fp32 arithmetic, yabt_grow_ref, whose
trees equal grow.c's: ms per tree with and without the leaf models, its root
histogram's time and share of HBM peak, and its split differences from the
exact tree, see reference_arithmetic), ``leaf_gram`` (the linear-leaf step
with the Gram sums on the VALU in exact fixed point and in fp64 on the matrix
cores, see leaf_gram_compare) and ``boosting`` (whole estimator fits, see
boosting_fits).

Usage: python bench.py [--gpus 1] [--steps 5] [--warmup 1] [--no-cpu]
                       [--ref-steps 1] [--no-boosting]
       python bench.py --counters
       python bench.py --leaf-compare
       python bench.py --boosting-only
"""

from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "histogram G row·feature updates/s + ms/tree at 10M×100, % of HBM peak"
HBM_PEAK_GBS = 8000.0
N_ROWS, N_FEAT, MAX_LEAVES = 10_000_000, 100, 255
PARAMS = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=MAX_LEAVES, max_depth=64)


class LeafNetParams:
    learning_rate = 0.1
    leaf_net_features = 8
    leaf_net_min_samples = 50
    leaf_net_l2 = 1.0
    leaf_net_hidden = 0


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def growth_of(res) -> str:
    """Which grower produced ``res``: best-first split by split, or in rounds
    of several computed splits (with the round count)."""
    rounds = getattr(res, "rounds", None)
    if rounds is None:
        return "sequential"
    return f"rounds ({rounds} rounds, {res.splits_computed} splits computed)"


def node_sizes(feature, left, right, leaf_of_row) -> np.ndarray:
    """Rows per node from per-row leaf ids (children have larger ids)."""
    size = np.bincount(leaf_of_row, minlength=len(feature)).astype(np.int64)
    for nid in range(len(feature) - 1, -1, -1):
        if feature[nid] >= 0:
            size[nid] = size[left[nid]] + size[right[nid]]
    return size


def tree_updates(feature, left, right, sizes, F) -> int:
    """Histogram work of one tree: the root plus the smaller child of every
    split (ties to the left, grow.c:355), times F."""
    rows = int(sizes[0])
    for nid in np.nonzero(feature >= 0)[0]:
        rows += int(min(sizes[left[nid]], sizes[right[nid]]))
    return rows * F


def gpu_inputs(torch, n, F, seed=0):
    from yabt_amd import grow_hip as G
    dev = torch.device("cuda", 0)
    gen = torch.Generator(device=dev)
    gen.manual_seed(seed)
    ld_fm = (n + 15) // 16 * 16
    fm = torch.randint(0, 256, (F, ld_fm), generator=gen, dtype=torch.uint8, device=dev)
    ld_rm = G._lib.row_stride(F)
    rm = torch.zeros((n, ld_rm), dtype=torch.uint8, device=dev)
    lib = G._lib.load()
    G._lib.check(lib.yabt_transpose_bins(G._ptr(fm), ld_fm, n, F, G._ptr(rm), ld_rm, G._stream(dev)),
                 "yabt_transpose_bins")
    g = torch.randn(n, generator=gen, device=dev, dtype=torch.float32)
    h = torch.rand(n, generator=gen, device=dev, dtype=torch.float32) * 0.9 + 0.1
    torch.cuda.synchronize()
    return G.BinLayouts(fm, rm, n, F), g, h


def time_root_hist(torch, lay, g, h, reps=50, warm=50):
    """Average duration of the streaming root-histogram kernel (one launch per
    call of yabt_hist_root, the per-fit bin counts given), HIP events on the
    launch stream, after ``warm`` untimed launches (the first few dozen run
    slower while the device clocks up)."""
    from yabt_amd import grow_hip as G
    from yabt_amd import _lib
    dev = lay.fm.device
    lib = _lib.load()
    out = torch.zeros((3, lay.F, 256), dtype=torch.int64, device=dev)
    _, (sg, sh, wide) = G.hist(lay, g, h)
    counts = lay.counts()
    stream = torch.cuda.current_stream(dev)

    def launch():
        _lib.check(lib.yabt_hist_root(G._ptr(lay.fm), lay.ld_fm, G._ptr(g), G._ptr(h), lay.n, lay.F,
                                      G._ptr(counts), sg, sh, wide, G._ptr(out), G._stream(dev)),
                   "yabt_hist_root")

    for _ in range(warm):
        launch()
    torch.cuda.synchronize()
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(reps)]
    for i in range(reps):
        starts[i].record(stream)
        launch()
        ends[i].record(stream)
    torch.cuda.synchronize()
    ms = [s.elapsed_time(e) for s, e in zip(starts, ends)]
    return float(np.mean(ms)), float(np.median(ms))


def time_bin_counts(torch, lay, reps=5):
    """Per-fit setup of the root histogram: yabt_bin_counts over the bins
    (mean of ``reps`` calls, HIP events)."""
    from yabt_amd import grow_hip as G
    from yabt_amd import _lib
    dev = lay.fm.device
    lib = _lib.load()
    c = torch.empty(int(lib.yabt_bin_counts_words(lay.n, lay.F)), dtype=torch.int32, device=dev)
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    _lib.check(lib.yabt_bin_counts(G._ptr(lay.fm), lay.ld_fm, lay.n, lay.F, G._ptr(c), G._stream(dev)),
               "yabt_bin_counts")
    torch.cuda.synchronize()
    e0.record(stream)
    for _ in range(reps):
        lib.yabt_bin_counts(G._ptr(lay.fm), lay.ld_fm, lay.n, lay.F, G._ptr(c), G._stream(dev))
    e1.record(stream)
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / reps


TRAFFIC_FILE = os.path.join(ROOT, "profiles", "k_hist_root_10Mx100_traffic.md")
COPY_ELEMS = 1 << 28          # fp32 elements of the copy kernel: 1 GiB read + 1 GiB written


def counter_launches(torch, lay, g, h) -> None:
    """Kernels for the rocprofv3 --pmc passes: a plain elementwise copy of
    known size (torch.neg over 2^28 fp32: 1 GiB read, 1 GiB written) and the
    root-histogram kernel, three launches each."""
    from yabt_amd import grow_hip as G
    from yabt_amd import _lib
    dev = lay.fm.device
    x = torch.ones(COPY_ELEMS, dtype=torch.float32, device=dev)
    y = torch.empty_like(x)
    for _ in range(3):
        torch.neg(x, out=y)
    torch.cuda.synchronize()
    del x, y
    lib = _lib.load()
    out = torch.zeros((3, lay.F, 256), dtype=torch.int64, device=dev)
    _, (sg, sh, wide) = G.hist(lay, g, h)
    counts = lay.counts()
    for _ in range(3):
        _lib.check(lib.yabt_hist_root(G._ptr(lay.fm), lay.ld_fm, G._ptr(g), G._ptr(h), lay.n, lay.F,
                                      G._ptr(counts), sg, sh, wide, G._ptr(out), G._stream(dev)),
                   "yabt_hist_root")
    torch.cuda.synchronize()


def committed_traffic():
    """HBM bytes per root-histogram launch from the committed counter summary
    (a line `traffic_bytes_per_launch: N`), or None."""
    try:
        with open(TRAFFIC_FILE) as fh:
            m = re.search(r"traffic_bytes_per_launch:\s*([0-9]+)", fh.read())
        return int(m.group(1)) if m else None
    except OSError:
        return None


def host_cpu() -> dict:
    """The host's CPU model, physical cores and the logical CPUs this process
    may use (from /proc/cpuinfo and the affinity mask)."""
    model, cores = None, set()
    phys = core = None
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                k, _, v = line.partition(":")
                k, v = k.strip(), v.strip()
                if k == "model name" and model is None:
                    model = v
                elif k == "physical id":
                    phys = v
                elif k == "core id":
                    core = v
                elif not k and phys is not None and core is not None:
                    cores.add((phys, core))
                    phys = core = None
        if phys is not None and core is not None:
            cores.add((phys, core))
    except OSError:
        pass
    logical = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"model": model, "physical_cores": len(cores) or None, "logical_cpus": logical}


def tree_updates_cpu(O, reference, bins_fm, res, threads, chunk=1_000_000) -> int:
    """Histogram work of a CPU-grown tree (as tree_updates), its per-row leaf
    ids routed in row chunks (fp32 copies of the bins, one chunk at a time)."""
    F, n = bins_fm.shape
    thr = np.where(res["feature"] >= 0, res["thr_bin"], 0).astype(np.float32)
    leaf = np.empty(n, np.int64)
    for r0 in range(0, n, chunk):
        X = np.ascontiguousarray(bins_fm[:, r0:r0 + chunk].T, dtype=np.float32)
        leaf[r0:r0 + chunk] = O.apply(X, res["feature"], thr, res["left"], res["right"], n_threads=threads,
                                      reference=reference)
    sizes = node_sizes(res["feature"], res["left"], res["right"], leaf)
    return tree_updates(res["feature"], res["left"], res["right"], sizes, F)


def cpu_baseline(inputs=None, gpu_ref_tree=None, budget_s: float = 20.0) -> dict:
    """Reference grow.c (or its restatement) on the full workload: one
    255-leaf tree over the same 10M x 100 inputs the GPU lines used (copied
    to the host: feature-major bins, g, h), or host RNG inputs of the same
    distribution when none are given.  With the GPU's reference-arithmetic
    tree of the same inputs (node arrays), whether the two trees are equal
    node for node (features, thresholds, children, value bits)."""
    from oracle import oracle as O
    reference = O.ref_available()
    cpu = host_cpu()
    threads = min(cpu["logical_cpus"], 8)   # the reference default (grow_c.py:283-302)
    F, n = N_FEAT, N_ROWS
    if inputs is not None:
        bins_fm, g, h = inputs
        source = "the GPU lines' own inputs (device RNG, seed 0), copied to the host"
    else:
        rng = np.random.default_rng(0)
        bins_fm = rng.integers(0, 256, size=(F, n), dtype=np.uint8)
        g = rng.normal(size=n).astype(np.float32)
        h = rng.uniform(0.1, 1.0, size=n).astype(np.float32)
        source = "host RNG inputs of the same distribution"
    kw = dict(PARAMS, nbins=np.full(F, 256, np.int32), n_threads=threads)
    times = []
    res = None
    t_start = time.perf_counter()
    for _ in range(4):  # warm-up + up to 3 timed runs within the budget
        t0 = time.perf_counter()
        res = O.grow(bins_fm, g, h, reference=reference, **kw)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > budget_s:
            break
    timed = times[1:] if len(times) > 1 else times
    sec = float(np.median(timed))
    upd = tree_updates_cpu(O, reference, bins_fm, res, threads)
    out = {"value": round(upd / sec / 1e9, 4), "unit": "G row·feature updates/s",
           "cores": threads, "kind": "reference" if reference else "port",
           "ms_per_tree": round(sec * 1e3, 1),
           "sample": f"one 255-leaf tree on 10,000,000 x 100 uniform u8 bins (the full workload), "
                     f"{source}, {len(timed)} timed run(s) after 1 warm-up, median; {threads} OpenMP threads",
           "host_cpu": cpu}
    if gpu_ref_tree is not None and reference:
        same = all(np.array_equal(np.asarray(res[k]), gpu_ref_tree[k]) for k in ("feature", "thr_bin", "left", "right"))
        same = same and np.array_equal(np.asarray(res["value"], np.float32).view(np.uint32),
                                       gpu_ref_tree["value"].view(np.uint32))
        out["same_tree_as_gpu_reference_arithmetic"] = bool(same)
    # the same tree on every logical CPU the process may use
    all_threads = cpu["logical_cpus"]
    t0 = time.perf_counter()
    O.grow(bins_fm, g, h, reference=reference, **dict(kw, n_threads=all_threads))
    sec_all = time.perf_counter() - t0
    out["all_cores"] = {"threads": all_threads, "ms_per_tree": round(sec_all * 1e3, 1),
                        "value": round(upd / sec_all / 1e9, 4)}
    del bins_fm, g, h
    out["other_workloads"] = cpu_other_workloads(O, reference, threads)
    return out


def reference_arithmetic(torch, lay, g, h, nbins, steps: int, exact_res, neural: bool) -> dict:
    """The same tree grown with the reference's own fp32 arithmetic
    (yabt_grow_ref, whose trees equal grow.c's node for node): ms per tree for
    the grower alone and with the leaf models, its root histogram (cgrow's
    row-order fp32 chains from the per-fit rank table) with its share of HBM
    peak, the per-fit rank table's cost, and the internal nodes whose
    (feature, bin) differ from the exact tree's."""
    from yabt_amd import grow_hip as G
    from yabt_amd.neural_leaves import fit_leaf_networks_binned
    from yabt_amd.tree import Tree
    n, F = lay.n, lay.F
    log(f"[bench] reference-arithmetic trees: {steps}")
    t0 = time.perf_counter()
    lay.ref_root_order()
    torch.cuda.synchronize()
    order_ms = (time.perf_counter() - t0) * 1e3

    def grow():
        return G.grow_device(lay, g, h, nbins, arithmetic="reference", **PARAMS)

    def with_leaves():
        res = grow()
        leaf = G.leaf_ids(res, n, F, MAX_LEAVES)
        tree = Tree(res.feature, res.thr_bin.float(), res.left, res.right, res.value, 0)
        return res, fit_leaf_networks_binned(tree, lay.fm, g + h * res.value[leaf], h, leaf, LeafNetParams, n=n)

    res = grow()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        res = grow()
    torch.cuda.synchronize()
    ms_grow = (time.perf_counter() - t0) * 1e3 / steps
    out = {"ms_grow": round(ms_grow, 2)}
    if neural:
        with_leaves()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            with_leaves()
        torch.cuda.synchronize()
        out["ms_per_tree"] = round((time.perf_counter() - t0) * 1e3 / steps, 2)
    # the root histogram alone, HIP events on the launch stream
    for _ in range(5):
        G.ref_root_hist(lay, g, h)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 10
    e0.record(stream)
    for _ in range(reps):
        G.ref_root_hist(lay, g, h)
    e1.record(stream)
    torch.cuda.synchronize()
    root_ms = e0.elapsed_time(e1) / reps
    root_bytes = n * F + 8 * n
    out["root_hist"] = {"ms": round(root_ms, 3), "GBps": round(root_bytes / (root_ms * 1e-3) / 1e9, 1),
                        "frac_hbm": round(root_bytes / (root_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                        "kernel": "k_rank_chain (row-order fp32 chains, one block per feature)"}
    out["fit_setup"] = {"root_order_ms": round(order_ms, 2),
                        "note": "per-fit root rank table (yabt_ref_root_order), outside the step"}
    # split sequence against the exact tree's
    a = {k: getattr(exact_res, k)[:exact_res.n_nodes].cpu().numpy() for k in ("feature", "thr_bin", "left")}
    b = {k: getattr(res, k)[:res.n_nodes].cpu().numpy() for k in ("feature", "thr_bin", "left")}
    same_shape = a["feature"].shape == b["feature"].shape and np.array_equal(a["left"], b["left"])
    m = min(a["feature"].size, b["feature"].size)
    internal = (a["feature"][:m] >= 0) | (b["feature"][:m] >= 0)
    differ = internal & ((a["feature"][:m] != b["feature"][:m]) | (a["thr_bin"][:m] != b["thr_bin"][:m]))
    out["vs_exact"] = {"internal_nodes": int(internal.sum()), "split_differences": int(differ.sum()),
                       "same_node_layout": bool(same_shape)}
    tree = {k: getattr(res, k)[:res.n_nodes].cpu().numpy() for k in ("feature", "thr_bin", "left", "right",
                                                                      "value")}
    return out, tree


def leaf_gram_compare(torch, lay, g, h, nbins, reps: int = 10) -> dict:
    """The linear-leaf step of one 255-leaf tree (moments, fit, fold; g, h at
    margin + value[leaf] of a quadratic objective) with the Gram sums on the
    VALU in exact int64 fixed point ("exact", the default) and in fp64 on the
    matrix cores ("mfma": v_mfma_f64_16x16x4_f64): ms per step, mean of
    ``reps`` after two warm-ups each, wall clock around device syncs."""
    from yabt_amd import grow_hip as G
    from yabt_amd import neural_leaves as NL
    from yabt_amd.neural_leaves import fit_leaf_networks_binned
    from yabt_amd.tree import Tree
    n = lay.n
    res = G.grow_device(lay, g, h, nbins, **PARAMS)
    leaf = G.leaf_ids(res, n, lay.F, MAX_LEAVES)
    tree = Tree(res.feature, res.thr_bin.float(), res.left, res.right, res.value, 0)
    g2 = g + h * res.value[leaf]
    out = {}
    keep = NL.GRAM
    try:
        for mode in ("exact", "mfma"):
            NL.GRAM = mode
            for _ in range(2):
                fit_leaf_networks_binned(tree, lay.fm, g2, h, leaf, LeafNetParams, n=n)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(reps):
                fit_leaf_networks_binned(tree, lay.fm, g2, h, leaf, LeafNetParams, n=n)
            torch.cuda.synchronize()
            out[f"ms_leaf_step_{mode}"] = round((time.perf_counter() - t0) * 1e3 / reps, 3)
    finally:
        NL.GRAM = keep
    out["default"] = keep
    return out


def cpu_other_workloads(O, reference: bool, threads: int) -> dict:
    """The same C grower, one tree each, on the other tree workloads (context
    for the estimator timings): the binary 1M x 28 workload (28 bins, depth 8,
    g = 0.5 - y, h = 0.25 from p = 0.5), and a 400 000-row sample (1/10) of the
    4M x 500 depth-6 mostly-zero workload through the sparse builder the
    reference picks for it (grow.c:68-107, which is serial)."""
    out = {}
    rng = np.random.default_rng(1)
    n, F = 1_000_000, 28
    bins = rng.integers(0, 28, size=(F, n), dtype=np.uint8)
    y = (rng.random(n) < 0.5).astype(np.float32)
    g = (np.float32(0.5) - y).astype(np.float32)
    h = np.full(n, 0.25, np.float32)
    kw = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=256, max_depth=8,
              nbins=np.full(F, 28, np.int32), n_threads=threads)
    O.grow(bins, g, h, reference=reference, **kw)
    t0 = time.perf_counter()
    O.grow(bins, g, h, reference=reference, **kw)
    out["binary_1Mx28_depth8_ms_per_tree"] = round((time.perf_counter() - t0) * 1e3, 1)
    n, F = 400_000, 500
    bins = rng.integers(1, 256, size=(n, F), dtype=np.uint8)
    bins[rng.random((n, F), dtype=np.float32) < 0.9] = 0
    g = rng.laplace(size=n).astype(np.float32)
    h = np.ones(n, np.float32)
    nondef = bins != 0
    indptr = np.concatenate([[0], np.cumsum(nondef.sum(axis=1))]).astype(np.int64)
    r, c = np.nonzero(nondef)
    layout = (indptr, c.astype(np.int32), bins[r, c].astype(np.int32), np.zeros(F, np.int32))
    bins_fm = np.ascontiguousarray(bins.T)
    del bins, nondef, r, c
    kw = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=64, max_depth=6,
              nbins=np.full(F, 256, np.int32), n_threads=threads)
    t0 = time.perf_counter()
    O.grow(bins_fm, g, h, reference=reference, sparse=layout, **kw)
    out["depth6_400kx500_sparse_ms_per_tree"] = round((time.perf_counter() - t0) * 1e3, 1)
    return out


def depthwise_trees(torch, trees: int = 10) -> dict:
    """ms per tree of the 4 000 000 x 500 skewed workload: each column bin 0
    with probability 0.9 else uniform on 1..255, g ~ Laplace(0, 1), h = 1,
    max_depth 6, 64 leaves, min_samples_leaf 20, with the margin update of a
    squared loss (y = -g0, margin0 = 0) between trees; grown depth by depth
    (the leaf budget cannot bind) and, for comparison, split by split; and
    in the reference arithmetic with cgrow's sparse builder (default bin 0),
    the builder the reference picks for data this sparse."""
    from yabt_amd import grow_hip as G
    from yabt_amd import boost_ops
    from yabt_amd.losses import MSELoss
    from yabt_amd.tree import Tree
    dev = torch.device("cuda", 0)
    n, F = 4_000_000, 500
    gen = torch.Generator(device=dev).manual_seed(0)
    b = torch.randint(1, 256, (n, F), dtype=torch.uint8, device=dev, generator=gen)
    b[torch.rand((n, F), device=dev, generator=gen) < 0.9] = 0
    lay = G.make_layouts(b, dev)
    del b
    u = torch.rand(n, device=dev, generator=gen) - 0.5
    g0 = -torch.sign(u) * torch.log1p(-2 * u.abs())            # Laplace(0, 1)
    y = -g0
    nbins = np.full(F, 256, np.int32)
    P = dict(lam=1.0, gamma=0.0, mcw=1e-3, msl=20, lr=0.1, max_leaves=64, max_depth=6)
    out = {}
    modes = [("batched", dict(batched=True), trees), ("sequential", dict(batched=False), trees),
             ("reference_sparse", dict(arithmetic="reference", default_bin=np.zeros(F, np.int32)), min(trees, 3))]
    for name, kw, k_trees in modes:
        margin = torch.zeros(n, device=dev)
        def tree_step():
            g, h = boost_ops.grad_hess(MSELoss(), margin, y)
            res = G.grow_device(lay, g, h, nbins, **kw, **P)
            leaf = G.leaf_ids(res, n, F, P["max_leaves"])
            boost_ops.margin_update(margin, leaf, Tree(res.feature, res.thr_bin.float(), res.left, res.right,
                                                       res.value, 0), None)
        tree_step()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(k_trees):
            tree_step()
        torch.cuda.synchronize()
        out["depth6_4Mx500_skewed_ms_per_tree_" + name] = round((time.perf_counter() - t0) * 1e3 / k_trees, 2)
    del lay
    torch.cuda.empty_cache()
    return out


def multiclass_fit(torch) -> dict:
    """Wall time of the 10-class estimator on X ~ N(0,1) 2 000 000 x 50 fp32,
    y = argmax(X W + Gumbel noise), W ~ N(0,1) (50, 10): one-vs-rest boosters
    of 20 trees each, 63 leaves, linear leaf models over 8 inputs with
    leaf_net_l2 1e-3, 256 bins (binning of every class's booster included),
    after one warm-up fit on 50 000 rows."""
    from yabt_amd import YABTClassifier
    rng = np.random.default_rng(0)
    n, F, C = 2_000_000, 50, 10
    X = rng.normal(size=(n, F)).astype(np.float32)
    W = rng.normal(size=(F, C)).astype(np.float32)
    y = np.argmax(X @ W + rng.gumbel(size=(n, C)).astype(np.float32), axis=1).astype(np.float32)
    mk = lambda t: YABTClassifier(n_estimators=t, max_leaves=63, leaf_net_l2=1e-3, max_bins=256)
    mk(2).fit(X[:50_000], y[:50_000])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    mk(20).fit(X, y)
    torch.cuda.synchronize()
    sec = time.perf_counter() - t0
    return {"multiclass_2Mx50_10cls_20trees_s": round(sec, 2),
            "multiclass_2Mx50_ms_per_tree": round(sec * 1e3 / (20 * C), 2)}


def exact_departures(torch, X, y, n_trees=100) -> dict:
    """Untimed: the binary fit in the reference arithmetic (cgrow's trees),
    and at each of its trees the same grower inputs (g, h, interaction
    matrix, parameters) grown again in the exact arithmetic.  The two trees
    are compared as split sets, node by node along paths from the root
    (yabt_amd.divergence: with 256 leaves at depth 8 the order of splits
    cannot change the set); for each tree that differs, the first differing
    node's rows give the float64 gains of the two arithmetics' choices and
    the bound on how far either arithmetic's gains can be from them."""
    from yabt_amd import Booster, LogLoss, YABTClassifier
    from yabt_amd import divergence as D
    from yabt_amd import grow_hip as G
    keys = ("feature", "thr_bin", "left", "right", "value")
    diffs = []

    def on_tree(t, inp, res):
        lay, g, h, nb = inp["layouts"], inp["grad"], inp["hess"], inp["nbins"]
        kw = {k: inp[k] for k in ("fmask", "imat", "ib", "lam", "gamma", "mcw", "msl", "lr", "max_leaves",
                                  "max_depth")}
        ex = G.grow_device(lay, g, h, nb, arithmetic="exact", **kw)
        a = {k: getattr(ex, k).cpu().numpy() for k in keys}
        b = {k: getattr(res, k).cpu().numpy() for k in keys}
        cd = D.canonical_first_difference(a, b)
        if cd is None:
            return
        rec = {"tree": t, "exact_split": cd["a"], "reference_split": cd["b"]}
        if cd["a"] is not None and cd["b"] is not None:
            _, (sg, sh, _) = G.hist(lay, g, h)
            imat = None if inp["imat"] is None else inp["imat"].cpu().numpy()
            node = cd["node_b"]
            gap = D.decision_gap(b, {"a": (node,) + cd["a"], "b": (node,) + cd["b"]}, lay.fm[:, :lay.n], g, h,
                                 nb, (sg, sh), lam=float(inp["lam"]), gamma=float(inp["gamma"]),
                                 boost_of=None if imat is None else
                                 (lambda k: D.path_boost(b, k, imat, float(inp["ib"]))))
            rec.update(rows=gap["rows"], gain_exact=round(gap["exact"]["gain"], 6),
                       gain_reference=round(gap["reference"]["gain"], 6),
                       gap_rel=float(f"{gap['gap'] / max(abs(gap['exact']['gain']), 1e-300):.3g}"),
                       bound_rel=float(f"{gap['bound'] / max(abs(gap['exact']['gain']), 1e-300):.3g}"),
                       explained=bool(gap["explained"]))
        diffs.append(rec)

    est = YABTClassifier(n_estimators=n_trees, max_leaves=256, max_depth=8, max_bins=28, neural_leaves=False,
                         grower_arithmetic="reference")
    Booster(est._boost_params(), LogLoss()).fit(X, y, on_tree=on_tree)
    return {"trees": n_trees, "differing_split_sets": len(diffs),
            "all_explained": all(d.get("explained", False) for d in diffs), "differences": diffs}


def boosting_fits(torch) -> dict:
    """Wall time of whole estimator fits (binning included, after one warm-up
    fit) in both grower arithmetics:
      * regression: X ~ N(0,1) 20 000 x 20, y = sin x0 + 0.5 x1 x2 + x3^2 +
        0.3 sum x4..x9 + N(0, 0.1^2); 25 trees, 31 leaves, lr 0.1, linear
        leaves, 255 bins;
      * binary: X ~ N(0,1) 1 000 000 x 28, y ~ Bernoulli(sigmoid(X w)),
        w ~ N(0,1); 100 trees of depth 8 (256 leaves), 28 bins, no leaf models."""
    from yabt_amd import YABTClassifier, YABTRegressor
    out = {}
    rng = np.random.default_rng(0)
    X = rng.normal(size=(20_000, 20)).astype(np.float32)
    y = (np.sin(X[:, 0]) + 0.5 * X[:, 1] * X[:, 2] + X[:, 3] ** 2 + 0.3 * X[:, 4:10].sum(axis=1)
         + rng.normal(scale=0.1, size=20_000)).astype(np.float32)
    for arith in ("exact", "reference"):
        mk = lambda: YABTRegressor(n_estimators=25, max_leaves=31, learning_rate=0.1, max_bins=255,
                                   grower_arithmetic=arith)
        mk().fit(X, y)
        t0 = time.perf_counter()
        mk().fit(X, y)
        torch.cuda.synchronize()
        out[f"regression_20kx20_25trees_s_{arith}"] = round(time.perf_counter() - t0, 3)
    log("[bench] depth-6 trees on 4M x 500 mostly-zero bins")
    out.update(depthwise_trees(torch))
    log("[bench] 10-class fits with linear leaves")
    out.update(multiclass_fit(torch))
    log("[bench] binary classifier fits")
    rng = np.random.default_rng(0)
    X = rng.normal(size=(1_000_000, 28)).astype(np.float32)
    w = rng.normal(size=28)
    y = (rng.random(1_000_000) < 1 / (1 + np.exp(-(X @ w)))).astype(np.float32)
    for arith in ("exact", "reference"):
        mk = lambda: YABTClassifier(n_estimators=100, max_leaves=256, max_depth=8, max_bins=28,
                                    neural_leaves=False, grower_arithmetic=arith)
        if arith == "exact":
            mk().fit(X[:50_000], y[:50_000])
        t0 = time.perf_counter()
        mk().fit(X, y)
        torch.cuda.synchronize()
        out[f"binary_1Mx28_100trees_s_{arith}"] = round(time.perf_counter() - t0, 2)
    log("[bench] exact vs reference arithmetic along the binary fit's trajectory (untimed)")
    out["binary_1Mx28_exact_vs_reference"] = exact_departures(torch, X, y)
    return out


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--rows", type=int, default=N_ROWS)
    ap.add_argument("--no-neural", action="store_true", help="time the grower only")
    ap.add_argument("--ref-steps", type=int, default=1,
                    help="trees grown with the reference arithmetic (0: skip)")
    ap.add_argument("--no-boosting", action="store_true", help="skip the estimator fits")
    ap.add_argument("--boosting-only", action="store_true",
                    help="only the estimator fits and depth-6 trees (one JSON line of their timings)")
    ap.add_argument("--counters", action="store_true",
                    help="only launch the copy and root-histogram kernels for rocprofv3 --pmc")
    ap.add_argument("--leaf-compare", action="store_true",
                    help="only the linear-leaf step in both Gram modes (one JSON line)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (got --gpus {args.gpus}); the tree-growing path "
              "runs on a single device", file=sys.stderr)
        sys.exit(2)

    import torch
    from yabt_amd import grow_hip as G

    if args.boosting_only:
        print(json.dumps({"boosting": boosting_fits(torch)}), flush=True)
        return

    n, F = args.rows, N_FEAT
    log(f"[bench] generating {n} x {F} inputs on cuda:0")
    lay, g, h = gpu_inputs(torch, n, F)
    nbins = np.full(F, 256, np.int32)
    if args.counters:
        log("[bench] copy and root-histogram kernels for counter passes")
        counter_launches(torch, lay, g, h)
        log("[bench] done")
        return
    if args.leaf_compare:
        log("[bench] linear-leaf step, exact and fp64 MFMA Gram sums")
        print(json.dumps({"leaf_gram": leaf_gram_compare(torch, lay, g, h, nbins)}), flush=True)
        return

    log("[bench] root histogram kernel")
    ms_counts = time_bin_counts(torch, lay)
    root_mean_ms, root_med_ms = time_root_hist(torch, lay, g, h)

    from yabt_amd.neural_leaves import fit_leaf_networks_binned
    from yabt_amd.tree import Tree

    def step(neural: bool):
        res = G.grow_device(lay, g, h, nbins, sync=False, **PARAMS)
        if not neural:
            return res, None
        # node arrays are full length (2L + 1); unused slots are empty leaves
        leaf = G.leaf_ids(res, n, F, MAX_LEAVES)
        tree = Tree(res.feature, res.thr_bin.float(), res.left, res.right, res.value, 0)
        g2 = torch.addcmul(g, h, res.value[leaf])   # g + h * value[leaf], one pass
        return res, fit_leaf_networks_binned(tree, lay.fm, g2, h, leaf, LeafNetParams, n=n)

    def timed(neural: bool, steps: int) -> float:
        stream = torch.cuda.current_stream()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        e0.record(stream)
        for _ in range(steps):
            step(neural)
        e1.record(stream)
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / steps

    neural = not args.no_neural
    log(f"[bench] warm-up trees: {args.warmup}")
    for _ in range(args.warmup):
        step(neural)
    torch.cuda.synchronize()
    log(f"[bench] timed trees: {args.steps} (grower only)")
    ms_grow = timed(False, args.steps)
    ms_per_tree = ms_grow
    if neural:
        log(f"[bench] timed trees: {args.steps} (grower + leaf models)")
        ms_per_tree = timed(True, args.steps)
    res, net = step(neural)
    torch.cuda.synchronize()
    if res.n_nodes is None:
        res.n_nodes = int(res._status[0].item())

    nn = res.n_nodes
    feat = res.feature[:nn].cpu().numpy()
    left = res.left[:nn].cpu().numpy()
    right = res.right[:nn].cpu().numpy()
    leaf = G.leaf_ids(res, n, F, MAX_LEAVES).cpu().numpy()
    sizes = node_sizes(feat, left, right, leaf)
    upd = tree_updates(feat, left, right, sizes, F)
    value = upd / (ms_per_tree * 1e-3) / 1e9

    root_bytes = n * F + 8 * n
    achieved = root_bytes / (root_mean_ms * 1e-3) / 1e9
    line = {
        "metric": METRIC, "value": round(value, 3), "unit": "G row·feature updates/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": round(ms_per_tree, 3), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "int64",
        "data": "synthetic (device RNG, seed 0)",
        "config": {"workload": "best-first tree, 10M rows x 100 features x 256 uint8 bins, 255 leaves"
                               + (", linear leaf models (K=8)" if neural else ""),
                   "rows": n, "features": F, "bins": 256, "max_leaves": MAX_LEAVES,
                   "min_samples_leaf": 20, "leaves_grown": int((feat == -1).sum()),
                   "tree_updates": upd, "growth": growth_of(res)},
        "ms_per_tree": round(ms_per_tree, 3), "ms_grow": round(ms_grow, 3),
        "leaf_models_fitted": (int((net.leaf_net_linear.abs().sum(dim=1) > 0).sum()) if neural else 0),
        "root_hist": {"ms": round(root_mean_ms, 4), "ms_median": round(root_med_ms, 4),
                      "updates_per_s": round(n * F / (root_mean_ms * 1e-3) / 1e9, 3),
                      "unit": "G updates/s", "GBps": round(achieved, 1),
                      "frac_hbm": round(achieved / HBM_PEAK_GBS, 4)},
        "fit_setup": {"bin_counts_ms": round(ms_counts, 4),
                      "note": "per-fit count plane of the root histogram (yabt_bin_counts), outside the step"},
        "roofline": {"kernel": "k_hist_root<false, true> (streaming root histogram)", "bound": "hbm",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": committed_traffic()},
    }
    ref_tree = None
    if args.ref_steps > 0:
        line["reference_arithmetic"], ref_tree = reference_arithmetic(torch, lay, g, h, nbins, args.ref_steps, res,
                                                                      neural)
    # the CPU baseline grows its tree on these same inputs
    host_inputs = None
    if not args.no_cpu:
        host_inputs = (np.ascontiguousarray(lay.fm[:, :n].cpu().numpy()), g.cpu().numpy(), h.cpu().numpy())
    if neural:
        log("[bench] linear-leaf step, exact and fp64 MFMA Gram sums")
        line["leaf_gram"] = leaf_gram_compare(torch, lay, g, h, nbins)
    if not args.no_boosting:
        del lay, g, h
        torch.cuda.empty_cache()
        line["boosting"] = boosting_fits(torch)
    if not args.no_cpu:
        log("[bench] CPU baseline")
        line["cpu_baseline"] = cpu_baseline(host_inputs, ref_tree)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
