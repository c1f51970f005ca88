// Stand-alone per-stage entry points of the gfx950 library: one histogram,
// one split scan, one stable partition, routing and the bin transpose.  They
// run the same device code as the grower (hist.h, scan.h) so each stage can be
// checked and timed alone.

#include "common.h"
#include "hist.h"
#include "host.h"
#include "scan.h"
#include "yabt_hip.h"

#include <string.h>

#include <mutex>
#include <vector>

namespace yabt {

char* error_buffer() {
    static thread_local char buf[ERROR_LEN] = "";
    return buf;
}

namespace {
struct PinnedEntry {
    void* p;
    size_t bytes;
    unsigned flags;
    int device;
};
std::mutex g_pinned_mu;
std::vector<PinnedEntry>& pinned_free() {
    static std::vector<PinnedEntry>* v = new std::vector<PinnedEntry>();   // never destroyed: kept to exit
    return *v;
}
}  // namespace

int pinned_take(size_t bytes, unsigned flags, void** out, int* device) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return hip_fail(e, "pinned host buffer");
    *device = dev;
    {
        std::lock_guard<std::mutex> lk(g_pinned_mu);
        auto& v = pinned_free();
        for (size_t i = 0; i < v.size(); ++i) {
            if (v[i].bytes == bytes && v[i].flags == flags && v[i].device == dev) {
                *out = v[i].p;
                v[i] = v.back();
                v.pop_back();
                return 0;
            }
        }
    }
    e = hipHostMalloc(out, bytes, flags);
    if (e != hipSuccess) {
        *out = nullptr;
        return hip_fail(e, "pinned host buffer");
    }
    return 0;
}

void pinned_give(void* p, size_t bytes, unsigned flags, int device) {
    std::lock_guard<std::mutex> lk(g_pinned_mu);
    pinned_free().push_back(PinnedEntry{p, bytes, flags, device});
}

constexpr int OB = 256;
constexpr int SPART_IPT = 16;
constexpr int SPART_TILE = OB * SPART_IPT;
constexpr int SPART_MAX_BLOCKS = 1024;

__global__ void __launch_bounds__(OB) k_quant(const float* grad, const float* hess, int64_t n, Quant* q) {
    quant_reduce<OB>(grad, hess, n, q);
}

__global__ void k_fill_i64(int64_t* p, int64_t v, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * OB + threadIdx.x; i < count; i += (int64_t)gridDim.x * OB) p[i] = v;
}

__global__ void k_fill_u32(uint32_t* p, uint32_t v, int64_t count) {
    for (int64_t i = (int64_t)blockIdx.x * OB + threadIdx.x; i < count; i += (int64_t)gridDim.x * OB) p[i] = v;
}

__global__ void k_set_hist_job(HistJob* j, const uint32_t* rows, int64_t lo, int64_t hi, int64_t* out) {
    j->active = 1;
    j->pad = 0;
    j->rows = rows;
    j->lo = lo;
    j->hi = hi;
    j->out = out;
}

__global__ void k_copy_shifts(const Quant* q, int32_t* out) {
    out[0] = q->sg;
    out[1] = q->sh;
    out[2] = q->wide;
}

// ---- stable two-pass partition (input order kept on each side) ----

struct PartRange {
    int nblk;
    int64_t lo, hi;
};

__device__ __forceinline__ PartRange part_range(int64_t m) {
    PartRange r;
    const int64_t tiles = (m + SPART_TILE - 1) / SPART_TILE;
    r.nblk = (int)min((int64_t)gridDim.x, max(tiles, (int64_t)1));
    const int64_t tpb = (tiles + r.nblk - 1) / r.nblk;
    r.lo = min(m, (int64_t)blockIdx.x * tpb * SPART_TILE);
    r.hi = min(m, r.lo + tpb * SPART_TILE);
    return r;
}

__global__ void __launch_bounds__(OB) k_part_count(const uint8_t* __restrict__ col, const uint32_t* rows_in,
                                                   int64_t m, int b, uint32_t* cnt) {
    const PartRange R = part_range(m);
    if ((int)blockIdx.x >= R.nblk) return;
    uint32_t c = 0;
    for (int64_t i = R.lo + threadIdx.x; i < R.hi; i += OB) c += (int)col[rows_in ? rows_in[i] : (uint32_t)i] <= b;
    __shared__ uint32_t s_red[OB / WAVE];
    c = block_sum<OB, uint32_t>(c, s_red);
    if (threadIdx.x == 0) cnt[blockIdx.x] = c;
}

__global__ void __launch_bounds__(OB) k_part_scatter(const uint8_t* __restrict__ col, const uint32_t* rows_in,
                                                     int64_t m, int b, const uint32_t* cnt, uint32_t* rows_out,
                                                     int64_t* out_mid) {
    const PartRange R = part_range(m);
    if ((int)blockIdx.x >= R.nblk) return;
    __shared__ uint64_t s_red64[OB / WAVE];
    __shared__ uint32_t s_wave[OB / WAVE];
    uint64_t before = 0, total = 0;
    for (int j = threadIdx.x; j < R.nblk; j += OB) {
        const uint64_t c = cnt[j];
        total += c;
        if (j < (int)blockIdx.x) before += c;
    }
    before = block_sum<OB, uint64_t>(before, s_red64);
    total = block_sum<OB, uint64_t>(total, s_red64);
    const int64_t mid = (int64_t)total;
    if (blockIdx.x == 0 && threadIdx.x == 0) out_mid[0] = mid;
    int64_t run_l = (int64_t)before, run_r = R.lo - (int64_t)before;
    for (int64_t t0 = R.lo; t0 < R.hi; t0 += SPART_TILE) {
        const int64_t a = t0 + (int64_t)threadIdx.x * SPART_IPT;
        uint32_t rid[SPART_IPT];
        uint32_t flags = 0, nv = 0;
#pragma unroll
        for (int j = 0; j < SPART_IPT; ++j) {
            const int64_t i = a + j;
            if (i < R.hi) {
                rid[j] = rows_in ? rows_in[i] : (uint32_t)i;
                flags |= ((int)col[rid[j]] <= b ? 1u : 0u) << j;
                ++nv;
            }
        }
        const uint32_t nl = __popc(flags), nr = nv - nl;
        uint32_t tl, tr;
        const uint32_t ol = block_excl_scan<OB, uint32_t>(nl, s_wave, &tl);
        const uint32_t orr = block_excl_scan<OB, uint32_t>(nr, s_wave, &tr);
        int64_t pl = run_l + ol, pr = mid + run_r + orr;
#pragma unroll
        for (int j = 0; j < SPART_IPT; ++j) {
            if ((uint32_t)j < nv) {
                if ((flags >> j) & 1u) rows_out[pl++] = rid[j];
                else rows_out[pr++] = rid[j];
            }
        }
        run_l += tl;
        run_r += tr;
    }
}

// ---- one split scan ----

__global__ void __launch_bounds__(OB) k_scan_one(const int64_t* hist, int F, const int32_t* nbins,
                                                 const uint8_t* fmask, const float* boost, int sg, int sh,
                                                 ScanParams sp, ScanRec* rec, uint32_t* ticket, double* out_gain,
                                                 int32_t* out_fb) {
    const int lane = threadIdx.x & (WAVE - 1), w = threadIdx.x / WAVE;
    const int f = blockIdx.x * (OB / WAVE) + w;
    if (f < F) {
        int64_t g4[4], h4[4], c4[4], t256[3];
        load_bins(hist, F, f, lane, g4, h4, c4, true);
        const int nb = max(0, min(NB, nbins[f]));
        ScanRec r = scan_feature(g4, h4, c4, nb, ldexp(1.0, -sg), ldexp(1.0, -sh), sp,
                                 (double)(boost ? boost[f] : 1.0f), lane, t256);
        if (!fmask[f]) no_split(r);
        if (lane == 0) rec[f] = r;
    }
    if (!last_block(ticket)) return;
    const int bf = reduce_records<OB>(rec, F);
    if (threadIdx.x == 0) {
        out_gain[0] = bf >= 0 ? rec[bf].gain : -INFINITY;
        out_fb[0] = bf;
        out_fb[1] = bf >= 0 ? rec[bf].b : -1;
    }
}

__global__ void k_zero_u32(uint32_t* p) { *p = 0; }

// ---- routing and layout ----

// Leaf index per row of raw X (n, ldx) row-major: x[f] <= threshold goes left
// (grow.c:223-239); at most max_steps steps (a malformed tree cannot loop).
__global__ void __launch_bounds__(OB) k_apply(const float* __restrict__ X, int64_t ldx, int F,
                                              const int64_t* __restrict__ feature,
                                              const float* __restrict__ threshold, const int64_t* __restrict__ left,
                                              const int64_t* __restrict__ right, int64_t n, int n_nodes,
                                              int64_t* out) {
    for (int64_t r = (int64_t)blockIdx.x * OB + threadIdx.x; r < n; r += (int64_t)gridDim.x * OB) {
        const float* x = X + (size_t)r * ldx;
        int64_t node = 0;
        for (int s = 0; s < n_nodes; ++s) {
            const int64_t f = feature[node];
            if (f < 0 || f >= F) break;
            const int64_t nxt = (x[f] <= threshold[node]) ? left[node] : right[node];
            if (nxt < 0 || nxt >= n_nodes) break;
            node = nxt;
        }
        out[r] = node;
    }
}

// (F, ld_src) feature-major -> (n, ld_dst) row-major, 64x64 byte tiles via LDS.
__global__ void __launch_bounds__(OB) k_transpose(const uint8_t* __restrict__ src, int64_t ld_src, int64_t n, int F,
                                                  uint8_t* __restrict__ dst, int64_t ld_dst) {
    __shared__ uint8_t t[64][65];
    const int64_t r0 = (int64_t)blockIdx.x * 64;
    const int f0 = blockIdx.y * 64;
    for (int i = threadIdx.x; i < 64 * 64; i += OB) {
        const int fi = i / 64, ri = i % 64;
        const int64_t r = r0 + ri;
        const int f = f0 + fi;
        t[fi][ri] = (r < n && f < F) ? src[(size_t)f * ld_src + r] : (uint8_t)0;
    }
    __syncthreads();
    for (int i = threadIdx.x; i < 64 * 64; i += OB) {
        const int ri = i / 64, fi = i % 64;
        const int64_t r = r0 + ri;
        const int f = f0 + fi;
        if (r < n && f < ld_dst) dst[(size_t)r * ld_dst + f] = t[fi][ri];
    }
}

static int check_hist_layout(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                             const float* grad, const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m,
                             const char* who) {
    static thread_local char msg[160];
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll || !grad || !hess) {
        snprintf(msg, sizeof msg, "%s: bad arguments", who);
        return fail(-2, msg);
    }
    if (rows ? (!bins_rm || ld_rm < F || ld_rm % 16 || !aligned16(bins_rm) || m < 0)
             : (!bins_fm || ld_fm < n || ld_fm % 16 || !aligned16(bins_fm))) {
        snprintf(msg, sizeof msg, "%s: bins layout (pointer, alignment or leading dimension) invalid", who);
        return fail(-2, msg);
    }
    if (!aligned16(grad) || !aligned16(hess)) {
        snprintf(msg, sizeof msg, "%s: grad and hess must be 16-byte aligned", who);
        return fail(-2, msg);
    }
    return 0;
}

// yabt_hist's work on a workspace of yabt_hist_workspace_bytes() (the
// quantisation record, then the gather job); shared with yabt_hist_noalloc.
int hist_enqueue(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
                 const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m, void* workspace, int64_t* out,
                 int32_t* out_shifts, hipStream_t stream, const char* who) {
    static thread_local char msg[160];
    if (!out || !workspace || !out_shifts) {
        snprintf(msg, sizeof msg, "%s: bad arguments", who);
        return fail(-2, msg);
    }
    const int rc0 = check_hist_layout(bins_fm, ld_fm, bins_rm, ld_rm, grad, hess, n, F, rows, m, who);
    if (rc0) return rc0;
    Carve c{(char*)workspace, 0};
    Quant* q = c.take<Quant>(1);
    HistJob* job = c.take<HistJob>(1);
    k_quant_clear<<<1, 1, 0, stream>>>(q);
    k_quant<<<launch_grid(n, OB * 16, 1024), OB, 0, stream>>>(grad, hess, n, q);
    launch_quant_resid(stream, grad, hess, n, q);
    const int64_t ne = 3 * (int64_t)F * NB;
    k_fill_i64<<<launch_grid(ne, OB, 1024), OB, 0, stream>>>(out, 0, ne);
    const int tiles = (F + HFL - 1) / HFL;
    if (!rows) {
        if (n > 0) {
            launch_hist_root(stream, bins_fm, ld_fm, grad, hess, n, F, q, 0.0, 0.0, 0, nullptr, nullptr, nullptr, out, 0,
                             nullptr);
        }
    } else if (m > 0) {
        k_set_hist_job<<<1, 1, 0, stream>>>(job, rows, 0, m, out);
        k_hist_gather<<<tiles * GATHER_MAX_CHUNKS, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, q, 0.0, 0.0,
                                                                        nullptr, job, 0, nullptr, 0);
    }
    k_copy_shifts<<<1, 1, 0, stream>>>(q, out_shifts);
    snprintf(msg, sizeof msg, "%s launch", who);
    return launch_status(msg);
}

}  // namespace yabt

using namespace yabt;

extern "C" {

const char* yabt_last_error(void) { return error_buffer(); }

int yabt_transpose_bins(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int F, uint8_t* bins_rm, int64_t ld_rm,
                        hipStream_t stream) {
    if (!bins_fm || !bins_rm || n < 0 || F < 1 || ld_fm < n || ld_rm < F)
        return fail(-2, "yabt_transpose_bins: bad arguments");
    if (n == 0) return 0;
    dim3 grid((unsigned)((n + 63) / 64), (unsigned)((ld_rm + 63) / 64));
    k_transpose<<<grid, OB, 0, stream>>>(bins_fm, ld_fm, n, F, bins_rm, ld_rm);
    return launch_status("yabt_transpose_bins launch");
}

int yabt_apply(const float* X, int64_t ldx, int64_t n, int F, const int64_t* feature, const float* threshold,
               const int64_t* left, const int64_t* right, int n_nodes, int64_t* out_node, hipStream_t stream) {
    if (!X || ldx < F || n < 0 || F < 1 || !feature || !threshold || !left || !right || n_nodes < 1 || !out_node)
        return fail(-2, "yabt_apply: bad arguments");
    if (n == 0) return 0;
    k_apply<<<launch_grid(n, OB, 4096), OB, 0, stream>>>(X, ldx, F, feature, threshold, left, right, n, n_nodes,
                                                         out_node);
    return launch_status("yabt_apply launch");
}

size_t yabt_hist_workspace_bytes(void) { return align_up(sizeof(Quant), 256) + align_up(sizeof(HistJob), 256); }

int yabt_hist(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm, const float* grad,
              const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m, void* workspace, int64_t* out,
              int32_t* out_shifts, hipStream_t stream) {
    if (!workspace) return fail(-2, "yabt_hist: bad arguments");
    return hist_enqueue(bins_fm, ld_fm, bins_rm, ld_rm, grad, hess, n, F, rows, m, workspace, out, out_shifts, stream,
                        "yabt_hist");
}

int yabt_hist_accumulate(const uint8_t* bins_fm, int64_t ld_fm, const uint8_t* bins_rm, int64_t ld_rm,
                         const float* grad, const float* hess, int64_t n, int F, const uint32_t* rows, int64_t m,
                         int sg, int sh, int wide, void* workspace, int64_t* out, hipStream_t stream) {
    if (!out || (rows && !workspace)) return fail(-2, "yabt_hist_accumulate: bad arguments");
    const int rc0 =
        check_hist_layout(bins_fm, ld_fm, bins_rm, ld_rm, grad, hess, n, F, rows, m, "yabt_hist_accumulate");
    if (rc0) return rc0;
    const double scg = ldexp(1.0, sg), sch = ldexp(1.0, sh);
    const int tiles = (F + HFL - 1) / HFL;
    if (!rows) {
        if (n > 0) {
            launch_hist_root(stream, bins_fm, ld_fm, grad, hess, n, F, nullptr, scg, sch, wide, nullptr, nullptr,
                             nullptr, out, 0, nullptr);
        }
    } else if (m > 0) {
        Carve c{(char*)workspace, 0};
        c.take<Quant>(1);
        HistJob* job = c.take<HistJob>(1);
        k_set_hist_job<<<1, 1, 0, stream>>>(job, rows, 0, m, out);
        k_hist_gather<<<tiles * GATHER_MAX_CHUNKS, HBLOCK, 0, stream>>>(bins_rm, ld_rm, grad, hess, F, nullptr, scg,
                                                                        sch, nullptr, job, 0, nullptr,
                                                                        window_log2(n, wide != 0));
    }
    return launch_status("yabt_hist_accumulate launch");
}

size_t yabt_bin_counts_words(int64_t n, int F) {
    if (F < 1 || n < 0 || n > 0xFFFFFFFFll) return 0;
    return (size_t)F * NB + (size_t)F * (size_t)count_segments(n);
}

int yabt_bin_counts(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int F, uint32_t* out_counts,
                    hipStream_t stream) {
    if (!bins_fm || !out_counts || F < 1 || n < 0 || n > 0xFFFFFFFFll || ld_fm < n || ld_fm % 16 ||
        !aligned16(bins_fm))
        return fail(-2, "yabt_bin_counts: bad arguments");
    const int64_t ne = (int64_t)F * NB;
    k_fill_u32<<<launch_grid(ne, OB, 1024), OB, 0, stream>>>(out_counts, 0, ne);
    if (n > 0) {
        const int64_t blocks = (int64_t)((F + HFL - 1) / HFL) * count_segments(n);
        k_bin_count_seg<<<(unsigned)blocks, HBLOCK, 0, stream>>>(bins_fm, ld_fm, n, F, out_counts);
    }
    return launch_status("yabt_bin_counts launch");
}

int yabt_hist_root(const uint8_t* bins_fm, int64_t ld_fm, const float* grad, const float* hess, int64_t n, int F,
                   const uint32_t* bin_counts, int sg, int sh, int wide, int64_t* out, hipStream_t stream) {
    if (!out) return fail(-2, "yabt_hist_root: bad arguments");
    const int rc0 = check_hist_layout(bins_fm, ld_fm, nullptr, 0, grad, hess, n, F, nullptr, 0, "yabt_hist_root");
    if (rc0) return rc0;
    if (n > 0) {
        launch_root_kernel(stream, root_grid(n, F, grad, hess), bins_fm, ld_fm, grad, hess, n, F, nullptr,
                           ldexp(1.0, sg), ldexp(1.0, sh), wide, nullptr, bin_counts, nullptr, out, 0, nullptr);
    }
    return launch_status("yabt_hist_root launch");
}

size_t yabt_best_split_workspace_bytes(int F) {
    return F < 1 ? 0 : align_up((size_t)F * sizeof(ScanRec), 256) + 256;
}

int yabt_best_split(const int64_t* hist, int F, const int32_t* nbins, const uint8_t* fmask, const float* boost, int sg,
                    int sh, double lam, double gamma, double mcw, int msl, void* workspace, double* out_gain,
                    int32_t* out_fb, hipStream_t stream) {
    if (!hist || F < 1 || !nbins || !fmask || !workspace || !out_gain || !out_fb)
        return fail(-2, "yabt_best_split: bad arguments");
    Carve c{(char*)workspace, 0};
    ScanRec* rec = c.take<ScanRec>((size_t)F);
    uint32_t* ticket = c.take<uint32_t>(1);
    k_zero_u32<<<1, 1, 0, stream>>>(ticket);
    const ScanParams sp = {lam, gamma, mcw, msl};
    k_scan_one<<<(F + 3) / 4, OB, 0, stream>>>(hist, F, nbins, fmask, boost, sg, sh, sp, rec, ticket, out_gain, out_fb);
    return launch_status("yabt_best_split launch");
}

size_t yabt_partition_workspace_bytes(void) { return align_up(SPART_MAX_BLOCKS * sizeof(uint32_t), 256); }

int yabt_partition(const uint8_t* bins_fm, int64_t ld_fm, int64_t n, int f, int b, const uint32_t* rows_in,
                   int64_t m, uint32_t* rows_out, void* workspace, int64_t* out_mid, hipStream_t stream) {
    if (!bins_fm || !rows_out || !workspace || !out_mid || m < 0 || f < 0 || ld_fm < n || m > 0xFFFFFFFFll ||
        (!rows_in && m > n))
        return fail(-2, "yabt_partition: bad arguments");
    uint32_t* cnt = reinterpret_cast<uint32_t*>(workspace);
    const uint8_t* col = bins_fm + (size_t)f * ld_fm;
    if (m == 0) {
        k_fill_i64<<<1, OB, 0, stream>>>(out_mid, 0, 1);
    } else {
        const int g = launch_grid(m, SPART_TILE, SPART_MAX_BLOCKS);
        k_part_count<<<g, OB, 0, stream>>>(col, rows_in, m, b, cnt);
        k_part_scatter<<<g, OB, 0, stream>>>(col, rows_in, m, b, cnt, rows_out, out_mid);
    }
    return launch_status("yabt_partition launch");
}

}  // extern "C"
