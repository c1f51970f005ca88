// Node-histogram kernels (exact int64 fixed point), shared by the grower and
// the stand-alone entry points.
//
// A block owns a tile of HFL = 16 features and a chunk of rows; its LDS
// histogram is laid out [bin][feature] (cell bin * 16 + fl).  An LDS atomic
// instruction of a wave is processed a quarter wave at a time, and every
// layout below sends the 16 lanes of a quarter wave to 16 different features
// (16 different bank pairs) whatever the bins are; a row-per-lane layout
// without that would send 64 lanes to random bins of one feature.
//   * streaming root (feature-major bins): lane 16 q + fl handles feature
//     f0 + fl for row group q, loads 16 consecutive bins of its feature with
//     one 16-byte load, and gets each row's words from the lane that loaded
//     them with DPP row_newbcast;
//   * gathered children (row-major bins): each lane takes one row, loads its
//     16 bins of the tile with one 16-byte load, and rotates them by lane % 16
//     so that its J-th add goes to feature (J + lane) % 16.
//
// Optional skips, both exact because the sums are integers:
//   * dflt[f] (may be NULL): rows whose bin equals dflt[f] are not added; the
//     caller restores that bin as node total minus the other bins (the
//     default-bin fill of grow.c:101-106, here exact);
//   * HCH = false: no h channel (every h equal): sum q(h) = count * q(h), and
//     the h plane of the output is left untouched.
#pragma once

#include "common.h"

namespace yabt {

constexpr int HFL = 16;                       // features per tile
constexpr int HBLOCK = 1024;                  // threads per histogram block
constexpr int HWAVES = HBLOCK / WAVE;
constexpr int HSTEP = HWAVES * WAVE;          // rows per block step (64 per wave)
constexpr int GATHER_MAX_CHUNKS = 64;         // chunk slots per tile in a gather launch
constexpr int GATHER_MIN_ROWS = 8192;         // rows per gather chunk, at least

struct HistLds {
    unsigned long long g[NB * HFL];           // [bin][fl]
    unsigned long long h[NB * HFL];
    uint32_t c[NB * HFL];
};

// Rows per block chunk for the streaming kernel: about two resident blocks
// per CU on 256 CUs, chunks a multiple of 8 so that all tiles of a row chunk
// run on one XCD (block id % 8) and share its L2 for the chunk's g and h.
inline int root_chunks(int64_t n, int tiles) {
    int want = 512 / tiles;
    const int64_t useful = (n + HSTEP - 1) / HSTEP;
    if (want > useful) want = (int)useful;
    want = want / 8 * 8;
    return want < 8 ? 8 : want;
}

// ---------------------------------------------------------------------------
// Packed count channel.  The count rides in the low bits of one 64-bit LDS
// word next to q (q(h), or q(g) without the h channel): every row adds
// (q << cb) + 1, so a sum over R rows is (sum q) << cb + R, exact while
// R < 2^cb and |sum q| < 2^(63 - cb).  With |q| <= 2^(61 - k) (n <= 2^k, the
// standard shift) both hold for windows of R <= 2^w rows, w = (k + 1) / 2,
// cb = w + 1; after each window every thread moves its 4 entries into
// registers (exact integer unpack) and clears them.  Two LDS atomics per
// update instead of three (one without the h channel).
// ---------------------------------------------------------------------------

constexpr int HENT = NB * HFL / HBLOCK;       // entries per thread in an unpack

// Packed-word LDS of the gather (see hist_gather_packed); its callers keep it
// in a union with HistLds, which the final flush reuses.
struct HistLdsP {
    unsigned long long g[NB * HFL];           // sum q(g) (with the h channel)
    unsigned long long p[NB * HFL];           // packed (q << cb) + 1
};
// The gather's LDS: the packed words, then the final flush's HistLds.
union GatherLds {
    HistLds u;
    HistLdsP p;
};

// Final flush of the packed kernels: thread t holds cells i = t + k HBLOCK
// (bin i / HFL, feature f0 + i % HFL) with sums g, h and counts c.  They go
// through the block's LDS (a HistLds, 80 KB, which the kernels' LDS unions
// hold) transposed to [feature][bin], so that a wave's global atomics cover
// 64 consecutive bins of one feature: four 128-byte lines per instruction
// instead of sixteen.  Feature fl's bin b sits at fl NB + (b ^ 2 fl): the
// swizzle spreads the 16 features a half-wave writes for two bins over 32
// distinct bank pairs (unswizzled they share one), and stays inside each
// aligned group of 64 bins, so a wave's reads still cover 64 consecutive
// bins.  The caller has finished with its own LDS layout (a barrier before
// the call).  Features >= F are skipped; cells without rows are skipped when
// adding (STORE false: global atomics into out's sums so far) and written as
// zeros when storing (STORE true: out is this block's own piece).
template <bool HCH, bool STORE = false>
__device__ __forceinline__ void flush_cells(HistLds& T, const uint64_t (&g)[HENT], const int64_t (&h)[HENT],
                                            const uint32_t (&c)[HENT], int64_t* out, int F, int f0) {
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        const int i = threadIdx.x + k * HBLOCK;
        const int fl = i % HFL;
        const int j = fl * NB + ((i / HFL) ^ (2 * fl));
        T.g[j] = g[k];
        if (HCH) T.h[j] = (unsigned long long)h[k];
        T.c[j] = c[k];
    }
    __syncthreads();
    const size_t plane = (size_t)F * NB;
#pragma unroll
    for (int k = 0; k < HENT; ++k) {
        const int j = threadIdx.x + k * HBLOCK;
        const int fl = j / NB;
        const int fi = f0 + fl;
        const uint32_t cj = T.c[j];
        if (fi >= F || (!STORE && cj == 0)) continue;
        const size_t at = (size_t)fi * NB + (size_t)((j % NB) ^ (2 * fl));
        if (STORE) {
            out[at] = (int64_t)T.g[j];
            if (HCH) out[plane + at] = (int64_t)T.h[j];
            out[2 * plane + at] = (int64_t)cj;
        } else {
            atomicAdd((unsigned long long*)(out + at), T.g[j]);
            if (HCH) atomicAdd((unsigned long long*)(out + plane + at), T.h[j]);
            atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)cj);
        }
    }
}

// LDS of the streaming root histogram: 256 bins x 32 words of 8 bytes, of
// which words 0..15 of a bin are the cells of features f0 .. f0 + 15 in one
// buffer and words 16..31 in the other.  The byte address of a cell is then
// (bin << 8) | (buffer << 7) | (fl << 3): one byte permute of the loaded bin
// word builds it.
// Within the 16 lanes of a row group the 16 features hit 16 distinct bank
// pairs whatever the bins are.
struct HistLdsR {
    unsigned long long w[NB * 2 * HFL];
};

// Byte J of `word` placed in bits 8..15 over `lo` (bits 0..7).
template <int J>
__device__ __forceinline__ uint32_t bin_addr(uint32_t word, uint32_t lo) {
    return __builtin_amdgcn_perm(word, lo, 0x0c0c0000u | ((4u + J) << 8));
}

// bin_addr with J a compile-time constant of an unrolled loop.
__device__ __forceinline__ uint32_t bin_addr_rt(uint32_t word, uint32_t lo, int j) {
    return __builtin_amdgcn_perm(word, lo, 0x0c0c0000u | ((4u + (uint32_t)j) << 8));
}

// ---------------------------------------------------------------------------
// Streaming root histogram: one LDS atomic per (row, feature).
//
// The count plane never needs the stream: it depends only on the bins, which
// stay the same over a whole fit, so it comes from the per-fit counts
// (F, 256) (k_bin_count, yabt_bin_counts), which each tile's chunk-0 block
// adds at its flush.  The stream carries g and h only:
//   ROOT_PACKED (h varies, narrow contract): each update adds the word
//     (q(g) << 32) + q(h) (mod 2^64)
//     into the cell [bin][feature]; each thread then reads its 4 cells and
//     unpacks them -- lo, the
//     sign-extended low 32 bits, is the h sum; (cell - lo) >> 32 the g sum.
//     The cells come in two buffers that alternate every epoch of
//     ROOT_DEPTH = 3 steps: after the barrier that ends an epoch, each thread
//     reads and clears its cells of that epoch's buffer while the waves add
//     the next epoch into the other one.  A cell so takes the rows of one
//     epoch (3072, or n when smaller) between two reads, and no atomic
//     targets it while it is read; with hist_shift's |q| <= 2^(30 -
//     min(k, 11)) each half's sum stays within 3 * 2^29 < 2^31 (2^30 for
//     n <= 2048), so both are exact.
//   ROOT_WIDE (h varies, wide contract): q(g) and q(h) go to a 64-bit cell
//     each (the two buffers), two atomics per update, no unpacking.
//   ROOT_G (every h equal): the word is q(g) itself; no unpacking, and the h
//     plane is left to the caller (count * q(h)).
// Invalid rows of a step add zero words (their q is 0), so the loop needs no
// per-row tail test; only the loads are bounded.  Each wave keeps the loads
// of the next ROOT_DEPTH steps in flight (the adds of one step take far less
// than a load's latency).
//
// SKIP: dflt is given (rows in a feature's default bin are not added, and
// the chunk-0 block leaves that bin's count out too: the caller restores the
// whole bin as node total minus the other bins).  Lanes of features >= F
// read feature f0's column and add into their own LDS columns, which the
// flush ignores.
// ---------------------------------------------------------------------------

// The streaming root kernel's blocks: 1024 threads (16 waves, 1024 rows per
// step) and 64 KB of LDS.
constexpr int RBLOCK = 1024;
constexpr int RSTEP = RBLOCK;                  // rows per block step (64 per wave)
constexpr int RENT = NB * HFL / RBLOCK;        // cells per thread in an unpack and the flush

// LDS of the root kernel's flush: the block's cells transposed to
// [feature][bin] (see flush_cells); shares the space of HistLdsR.
struct RootFlushLds {
    unsigned long long g[NB * HFL];
    unsigned long long h[NB * HFL];
};

// Final flush of the streaming root kernel: as flush_cells, with the counts
// read from the per-fit table (chunk-0 blocks only, `counts` may be NULL;
// a feature's default bin, dflt[f] when dflt is given, is left out) and
// cells whose g and h sums are zero skipped (adding zero changes nothing).
template <bool HCH>
__device__ __forceinline__ void flush_cells_gh(RootFlushLds& T, const int64_t (&g)[RENT], const int64_t (&h)[RENT],
                                               const uint32_t* __restrict__ counts,
                                               const int32_t* __restrict__ dflt, int64_t* out, int F, int f0) {
#pragma unroll
    for (int k = 0; k < RENT; ++k) {
        const int i = threadIdx.x + k * RBLOCK;
        const int fl = i % HFL;
        const int j = fl * NB + ((i / HFL) ^ (2 * fl));
        T.g[j] = (unsigned long long)g[k];
        if (HCH) T.h[j] = (unsigned long long)h[k];
    }
    __syncthreads();
    const size_t plane = (size_t)F * NB;
#pragma unroll
    for (int k = 0; k < RENT; ++k) {
        const int j = threadIdx.x + k * RBLOCK;
        const int fl = j / NB;
        const int fi = f0 + fl;
        if (fi >= F) continue;
        const int b = (j % NB) ^ (2 * fl);
        const size_t at = (size_t)fi * NB + (size_t)b;
        const unsigned long long gj = T.g[j];
        if (gj) atomicAdd((unsigned long long*)(out + at), gj);
        if (HCH) {
            const unsigned long long hj = T.h[j];
            if (hj) atomicAdd((unsigned long long*)(out + plane + at), hj);
        }
        if (counts) {
            const uint32_t cj = counts[at];
            const int d = dflt ? dflt[fi] : -1;   // the default bin's count is left to the caller's fill
            if (cj && b != d) atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)cj);
        }
    }
}

// Rows per chunk of the streaming root kernel's full tiles (whole block steps).
__host__ __device__ inline int64_t root_chunk_rows(int64_t n, int chunks) {
    return ((n + chunks - 1) / chunks + RSTEP - 1) / RSTEP * RSTEP;
}

constexpr int TAILF = 4;                 // features of a tail tile, at most
constexpr int TSTEP = 2 * RBLOCK;        // rows per tail block step (128 per wave)

// Grid of the streaming root kernel: `tiles` full 16-feature tiles of
// `chunks` row chunks each, and `tail` blocks of tail_rows rows for the tail
// tile.  The last tile is a tail tile when it holds 1..TAILF features and g
// and h can be read in aligned pairs (8-byte aligned, n >= 2).  One
// 1024-thread block runs per CU, so the grid is one wave: RXCD dies of RSLOTS
// CUs, block id b on die b % RXCD (the dispatcher's round robin).  Die x
// runs the full tiles of chunks x, x + RXCD, ... -- every tile of a chunk on
// one die, sharing its L2 for the chunk's g and h -- and tail blocks in its
// remaining slots (root_block); chunks is chosen so that the slowest block is
// as short as it can be: a full block costs 16 per row and a tail block
// TAIL_COST (its quarter of the LDS atomics comes with more VALU work and
// loads of g and h of its own: 7 per row, measured against the full
// blocks' 16).  At 10M x 100: 39 chunks (234 full blocks of 257 024 rows)
// and 22 tail blocks (454 656 rows); with chunks a multiple of 8 it was 40
// and 16 (626 688 rows), and the tail blocks ended 15-20 µs after the full
// ones.  With more than RSLOTS tiles a chunk cannot fit one die and the
// tiles go in order (tile-major, chunks a multiple of 8, tail blocks first).
constexpr int RXCD = 8, RSLOTS = 32;   // dies, one-block-per-CU slots per die
constexpr int TAIL_COST = 7;           // a tail block's cost per row, a full block's being 16

struct RootGrid {
    int tiles, chunks, tail, blocks;
    int xcd;                           // 1: die-aware layout (root_block); 0: tail blocks, then tile-major
    int64_t tail_rows;
};

// Chunks whose full tiles die x runs in the die-aware layout.
__host__ __device__ inline int xcd_chunks(int chunks, int x) { return chunks > x ? (chunks - x + RXCD - 1) / RXCD : 0; }

inline RootGrid root_grid(int64_t n, int F, const void* grad, const void* hess) {
    constexpr int SLOTS = RXCD * RSLOTS;
    const int rem = F % HFL;
    const bool tail = rem >= 1 && rem <= TAILF && n >= 2 && (uintptr_t)grad % 8 == 0 && (uintptr_t)hess % 8 == 0;
    RootGrid g;
    g.tiles = tail ? F / HFL : (F + HFL - 1) / HFL;
    g.xcd = g.tiles <= RSLOTS ? 1 : 0;
    const int64_t useful = max((int64_t)1, (n + RSTEP - 1) / RSTEP);   // chunks with rows
    const int64_t tail_useful = (n + TSTEP - 1) / TSTEP;               // tail blocks with rows
    g.chunks = 0;
    int T = 0;
    if (g.xcd) {
        if (g.tiles > 0) {
            const int cmax = (int)min((int64_t)(RSLOTS / g.tiles * RXCD), useful);
            g.chunks = cmax;
            if (tail) {
                // the chunk count whose slowest block is shortest: full blocks
                // cost 16 / c of the rows each, tail blocks TAIL_COST / T
                int64_t best_num = -1, best_den = 1;
                for (int c = 1; c <= cmax; ++c) {
                    const int t = (int)min((int64_t)(SLOTS - g.tiles * c), tail_useful);
                    if (t < 1) break;
                    // max(16 / c, TAIL_COST / t) as a fraction num / den
                    const int64_t a_num = 16 * (int64_t)t, b_num = (int64_t)TAIL_COST * c, den = (int64_t)c * t;
                    const int64_t num = a_num > b_num ? a_num : b_num;
                    if (best_num < 0 || num * best_den < best_num * den) {
                        best_num = num;
                        best_den = den;
                        g.chunks = c;
                    }
                }
                T = (int)min((int64_t)(SLOTS - g.tiles * g.chunks), tail_useful);
            }
        } else {
            T = (int)min((int64_t)SLOTS, tail_useful);
        }
    } else {
        int want = tail ? 8 * SLOTS / (8 * g.tiles + 3) : SLOTS / g.tiles;
        if (want > useful) want = (int)useful;
        want = want / 8 * 8;
        g.chunks = want < 8 ? 8 : want;
        if (tail) T = (int)min((int64_t)max(SLOTS - g.tiles * g.chunks, (3 * g.chunks + 7) / 8), tail_useful);
    }
    g.tail = 0;
    g.tail_rows = 0;
    if (tail && T > 0) {
        g.tail_rows = ((n + T - 1) / T + TSTEP - 1) / TSTEP * TSTEP;
        g.tail = (int)((n + g.tail_rows - 1) / g.tail_rows);   // no empty tail block
    }
    g.blocks = g.xcd ? (g.tiles > 0 ? SLOTS : g.tail) : g.tail + g.tiles * g.chunks;
    return g;
}

// Block bid of a root grid: a full block (tile, chunk) with tb = -1, or tail
// block tb; false for an idle slot.
__host__ __device__ __forceinline__ bool root_block(int bid, int tiles, int chunks, int tail, int xcd, int& tile,
                                                    int& chunk, int& tb) {
    tile = chunk = 0;
    tb = -1;
    if (!xcd) {
        if (bid < tail) {
            tb = bid;
            return true;
        }
        tile = (bid - tail) / chunks;
        chunk = (bid - tail) % chunks;
        return true;
    }
    if (tiles == 0) {
        tb = bid;
        return bid < tail;
    }
    const int x = bid % RXCD, k = bid / RXCD;
    const int nx = xcd_chunks(chunks, x) * tiles;
    if (k < nx) {
        tile = k % tiles;
        chunk = (k / tiles) * RXCD + x;
        return true;
    }
    int pre = 0;   // tail slots of the dies before x
    for (int y = 0; y < x; ++y) pre += RSLOTS - xcd_chunks(chunks, y) * tiles;
    tb = pre + (k - nx);
    return tb < tail;
}

constexpr int ROOT_G = 0, ROOT_PACKED = 1, ROOT_WIDE = 2;   // modes of the streaming root kernels
constexpr int ROOT_DEPTH = 3;    // steps of inputs loaded ahead of the adds: one epoch
// A packed cell stays exact while it takes fewer than PACKED_CELL_ROWS rows:
// with hist_shift's |q| <= 2^19 (n > 2048; below, |q| <= 2^30 / n) each half
// then stays below 2^31.
constexpr int64_t PACKED_CELL_ROWS = 4096;
// Rows of a count segment: the per-fit count table also holds, per feature
// and segment, the largest count of any bin in the segment (yabt_bin_counts),
// which bounds the rows any cell of a root chunk can take.
constexpr int64_t SEG_ROWS = 65536;
__host__ __device__ inline int64_t count_segments(int64_t n) { return (n + SEG_ROWS - 1) / SEG_ROWS; }
constexpr int TAIL_DEPTH = 4;    // the same in a tail block (4 steps of 512 rows per column)
// A cell takes the rows of one epoch between two unpacks: ROOT_DEPTH block
// steps of RSTEP rows (3072), and with hist_shift's |q| <= 2^19 each half of
// the packed cell then stays within 3072 * 2^19 < 2^31.
static_assert((int64_t)ROOT_DEPTH * RSTEP * (1 << 19) < (1ll << 31), "an epoch's sums fit 32-bit halves");
static_assert(PACKED_CELL_ROWS * (1 << 19) <= (1ll << 31) && ROOT_DEPTH * RSTEP <= PACKED_CELL_ROWS,
              "a cell below PACKED_CELL_ROWS rows is exact");
static_assert((int64_t)TAIL_DEPTH * TSTEP / 4 * (1 << 19) < (1ll << 31), "a tail epoch's sums fit 32-bit halves");

// Whether root chunks (or tail spans) of up to `per` rows over bins of
// leading dimension ld can be read through buffer resources: every 32-bit
// offset of a tile's loads (a lane's column, fl ld, plus the row of a step,
// the ring's steps past the chunk included) and of the chunk's g and h (4
// bytes a row) fits 32 bits.
__host__ __device__ inline bool root_buffers(int64_t ld, int64_t per) {
    const int64_t rows = per + 8 * RSTEP;
    return (int64_t)HFL * ld + rows < (1ll << 32) && 4 * rows < (1ll << 32);
}

// MODE: ROOT_G (every h equal: the word is q(g), never unpacked), ROOT_PACKED
// (narrow contract: (q(g) << 32) + q(h) in one cell, epochs), ROOT_WIDE (wide
// contract: q(g) and q(h) in a cell each -- the two buffers of the layout --
// with one atomic per channel; 64-bit cells never need an unpack).
// BUF (root_buffers holds): the loads go through buffer resources bounded at
// the chunk's end -- g and h past it read as 0, so their words are 0 and no
// row needs a test, and the steps' offsets are scalar -- else through global
// pointers with each row clamped into the chunk and its word masked.
// The root totals (q_tot, tile 0) are the sums of feature 0's cells (every
// row has one bin of feature 0), or with SKIP (default bins left out) the
// per-row sums.
template <int MODE, bool SKIP, bool BUF>
__device__ __forceinline__ void hist_root_gh(HistLdsR& L, const uint8_t* __restrict__ bins_fm, int64_t ld,
                                             const float* __restrict__ grad, const float* __restrict__ hess,
                                             int64_t n, int F, double scg, double sch,
                                             const int32_t* __restrict__ dflt, const uint32_t* __restrict__ counts,
                                             Quant* q_tot, int64_t* out, int chunks, int tile, int chunk) {
    constexpr bool HCH = MODE != ROOT_G, PACK = MODE == ROOT_PACKED;
    const int f0 = tile * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int64_t per = root_chunk_rows(n, chunks);
    const int64_t lo = (int64_t)chunk * per, hi = min(n, lo + per);
    if (f0 >= F || lo >= hi) return;
    const int d = (SKIP && fok) ? dflt[f] : -1;
    const bool totals = q_tot != nullptr && tile == 0;
    for (int i = threadIdx.x; i < NB * 2 * HFL; i += RBLOCK) L.w[i] = 0;
    const uint32_t lbase = (uint32_t)fl << 3;
    char* const lds = reinterpret_cast<char*>(L.w);
    int64_t ag[RENT], ah[RENT];   // unpacked sums of this thread's cells
#pragma unroll
    for (int k = 0; k < RENT; ++k) {
        ag[k] = 0;
        ah[k] = 0;
    }
    // the cell a thread unpacks: cell i = t + k RBLOCK is bin i / HFL, feature i % HFL
    auto cell = [](int k) { const int i = threadIdx.x + k * RBLOCK; return (i / HFL) * (2 * HFL) + (i % HFL); };
    // add buffer p's cells to the sums and clear them (no atomic targets p
    // meanwhile: the other buffer takes the current epoch)
    auto unpack = [&](int p) {
#pragma unroll
        for (int k = 0; k < RENT; ++k) {
            const int c = cell(k) + p * HFL;
            const uint64_t v = L.w[c];
            L.w[c] = 0;
            const int64_t hs = (int64_t)(int32_t)(uint32_t)v;
            ah[k] += hs;
            ag[k] += (int64_t)(v - (uint64_t)hs) >> 32;
        }
    };
    // Inputs of step s: this lane's row's g and h, and 16 rows of its
    // feature's bins.
    //   BUF: offsets from the chunk's first row; the bins' resource starts at
    //   row lo of feature f0 and ends with the tile's last feature below F, so
    //   lanes of features >= F read zeros (their columns are never flushed).
    //   Otherwise the loads are unconditional: a row past hi reads row hi - 1
    //   (its word is masked to zero below), and a row group past hi reads the
    //   chunk's first 16 rows (their rows' words are zero); r0 % 64 == 0 and
    //   lo % 16 == 0, so the bins base is a multiple of 16 below hi <= n <= ld
    //   (ld % 16 == 0): the 16-byte load stays inside the row.
    const int nf = min(HFL, F - f0);
    const __amdgpu_buffer_rsrc_t rsg = raw_rsrc(grad + lo, BUF ? (uint32_t)((hi - lo) * 4) : 0u);
    const __amdgpu_buffer_rsrc_t rsh = raw_rsrc(hess + lo, (BUF && HCH) ? (uint32_t)((hi - lo) * 4) : 0u);
    const __amdgpu_buffer_rsrc_t rsb =
        raw_rsrc(bins_fm + (size_t)f0 * ld + lo, BUF ? (uint32_t)((int64_t)nf * ld - lo) : 0u);
    const uint32_t vg = (uint32_t)(wave * WAVE + lane) * 4u;
    const uint32_t vb = (uint32_t)((int64_t)fl * ld) + (uint32_t)(wave * WAVE + HFL * rg);
    const uint8_t* col = bins_fm + (size_t)(fok ? f : f0) * ld;
    auto load = [&](int64_t s, float& gv, float& hv, uint4& bw) {
        if (BUF) {
            typedef int v4i __attribute__((ext_vector_type(4)));
            const int so = (int)(s * RSTEP);
            // issued in this order wherever load runs (see the ring below)
            gv = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsg, (int)vg, so * 4, 0));
            __builtin_amdgcn_sched_barrier(0);
            if (HCH) hv = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsh, (int)vg, so * 4, 0));
            __builtin_amdgcn_sched_barrier(0);
            const v4i b = __builtin_amdgcn_raw_buffer_load_b128(rsb, (int)vb, so, 0);
            __builtin_amdgcn_sched_barrier(0);
            bw = make_uint4((uint32_t)b.x, (uint32_t)b.y, (uint32_t)b.z, (uint32_t)b.w);
        } else {
            const int64_t r0 = lo + s * RSTEP + (int64_t)wave * WAVE;
            const int64_t r = min(r0 + lane, hi - 1);
            gv = grad[r];
            if (HCH) hv = hess[r];
            const int64_t base = r0 + HFL * rg;
            bw = *reinterpret_cast<const uint4*>(col + (base < hi ? base : lo));
        }
    };
    const int64_t steps = (hi - lo + RSTEP - 1) / RSTEP;   // the same in every wave: barriers below
    // Packed cells need epochs only when one of them could take
    // PACKED_CELL_ROWS rows of the chunk: the per-fit table bounds a cell's
    // rows by the sum, over the count segments the chunk touches, of its
    // feature's largest bin count in each (uniform over the block; no table:
    // epochs).  Without epochs every row goes to buffer 0, unpacked once at
    // the end.
    bool epochs = PACK;
    if (PACK && counts) {
        const uint32_t* segmax = counts + (size_t)F * NB;
        const int64_t nseg = count_segments(n);
        uint32_t bound = 0;
        if (fok)
            for (int64_t sg = lo / SEG_ROWS; sg <= (hi - 1) / SEG_ROWS; ++sg) bound += segmax[(size_t)f * nseg + sg];
        bound = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_max_u32_v(bound));
        epochs = (int64_t)bound >= PACKED_CELL_ROWS;
    }
    // Ring of ROOT_DEPTH stages: stage j holds step s0 + j and is then refilled
    // with step s0 + j + ROOT_DEPTH (the ring is unrolled: no register moves).
    // A round of the ring is one epoch; its cells are one of two buffers,
    // which alternate by round.  The first round's loads are issued before
    // the loop, in the loop's own order (scheduling barriers between them),
    // so that the compiler's waits at the loop's head, which must hold for
    // the entry as well as the back edge, wait only for the stage's own
    // loads.
    float gs[ROOT_DEPTH], hs[ROOT_DEPTH];
    uint4 bs[ROOT_DEPTH];
#pragma unroll
    for (int j = 0; j < ROOT_DEPTH; ++j) {
        hs[j] = 0.0f;
        __builtin_amdgcn_sched_barrier(0);
        load(j, gs[j], hs[j], bs[j]);
    }
    __syncthreads();
    int64_t sum_g = 0, sum_h = 0;
    uint32_t buf = 0;   // the cell buffer of this round's epoch
    for (int64_t s0 = 0; s0 < steps; s0 += ROOT_DEPTH) {
        const uint32_t lb = PACK ? (lbase | (buf << 7)) : lbase;
#pragma unroll
        for (int j = 0; j < ROOT_DEPTH; ++j) {
            const int64_t s = s0 + j;
            // keep the scheduler from hoisting a later stage's use of its
            // loads above this stage's work (that would wait for them early);
            // every stage runs, a step past the last being all invalid rows
            __builtin_amdgcn_sched_barrier(0);
            const bool rok = BUF || lo + s * RSTEP + (int64_t)wave * WAVE + lane < hi;
            int64_t gq, hq;
            uint64_t word;
            if (PACK) {
                // |q| <= 2^30 (hist_shift): 32-bit halves, the word's high half
                // borrowing one from it when q(h) is negative
                const int32_t g32 = rok ? (int32_t)quantise_node(gs[j], scg) : 0;
                const int32_t h32 = rok ? (int32_t)quantise_node(hs[j], sch) : 0;
                gq = g32;
                hq = h32;
                word = ((uint64_t)((uint32_t)g32 + (uint32_t)(h32 >> 31)) << 32) | (uint32_t)h32;
            } else {
                gq = rok ? quantise_wide(gs[j], scg) : 0;
                hq = (HCH && rok) ? quantise_wide(hs[j], sch) : 0;
                word = (uint64_t)gq;
            }
            // the 16 cell addresses (and, with SKIP, which rows are not added)
            // come out of this stage's bins before its registers are refilled,
            // so the old and new values are never live at once (else the refill
            // lands in other registers and a copy at the loop's end waits for it)
            const uint32_t wv[4] = {bs[j].x, bs[j].y, bs[j].z, bs[j].w};
            uint32_t at[HFL];
            uint32_t keep = 0xffffu;
#pragma unroll
            for (int J = 0; J < HFL; ++J) {
                at[J] = bin_addr_rt(wv[J >> 2], lb, J & 3);
                if (SKIP && (int)((wv[J >> 2] >> (8 * (J & 3))) & 0xffu) == d) keep &= ~(1u << J);
            }
            load(s + ROOT_DEPTH, gs[j], hs[j], bs[j]);
            if (SKIP) {
                sum_g += gq;
                sum_h += hq;
            }
            // ROOT_WIDE: the h cell is the g cell's twin in the other buffer
            // (16 words, 128 bytes, further)
#define YABT_GH_ADD(J)                                                           \
            {                                                                    \
                const uint64_t wj = row_bcast64<J>(word);                        \
                unsigned long long* const cp = reinterpret_cast<unsigned long long*>(lds + at[J]); \
                if (!SKIP || ((keep >> (J)) & 1u)) {                             \
                    atomicAdd(cp, (unsigned long long)wj);                       \
                    if (MODE == ROOT_WIDE)                                       \
                        atomicAdd(cp + HFL, (unsigned long long)row_bcast64<J>((uint64_t)hq)); \
                }                                                                \
            }
            YABT_GH_ADD(0) YABT_GH_ADD(1) YABT_GH_ADD(2) YABT_GH_ADD(3)
            YABT_GH_ADD(4) YABT_GH_ADD(5) YABT_GH_ADD(6) YABT_GH_ADD(7)
            YABT_GH_ADD(8) YABT_GH_ADD(9) YABT_GH_ADD(10) YABT_GH_ADD(11)
            YABT_GH_ADD(12) YABT_GH_ADD(13) YABT_GH_ADD(14) YABT_GH_ADD(15)
#undef YABT_GH_ADD
        }
        if (epochs) {
            // end of the epoch: once every wave's adds into its buffer are
            // done, read it while the next epoch adds into the other one
            __syncthreads();
            unpack((int)buf);
            buf ^= 1u;
        }
    }
    __syncthreads();
    if (PACK && !epochs) unpack(0);
    if (!PACK) {   // never unpacked: the cells are the g sums (and the h sums)
#pragma unroll
        for (int k = 0; k < RENT; ++k) {
            ag[k] = (int64_t)L.w[cell(k)];
            if (HCH) ah[k] = (int64_t)L.w[cell(k) + HFL];
        }
    }
    if (totals) {
        if (!SKIP) {   // thread t's cells are of feature t % HFL
            sum_g = 0;
            sum_h = 0;
            if (threadIdx.x % HFL == 0) {
#pragma unroll
                for (int k = 0; k < RENT; ++k) {
                    sum_g += ag[k];
                    sum_h += ah[k];
                }
            }
        }
        sum_g = wave_sum<int64_t>(sum_g);
        sum_h = wave_sum<int64_t>(sum_h);
        if (lane == 0) {
            atomicAdd((unsigned long long*)&q_tot->tot_g, (unsigned long long)sum_g);
            atomicAdd((unsigned long long*)&q_tot->tot_h, (unsigned long long)sum_h);
        }
    }
    __syncthreads();   // every cell read before the LDS is rewritten
    flush_cells_gh<HCH>(*reinterpret_cast<RootFlushLds*>(&L), ag, ah, chunk == 0 ? counts : nullptr,
                        SKIP ? dflt : nullptr, out, F, f0);
}

// ---------------------------------------------------------------------------
// Streaming root histogram of a tail tile: the last tile when it holds at
// most TAILF = 4 features (F % 16 in 1..4), where the full kernel's lanes of
// 12 or more of the 16 columns would add into cells the flush ignores.  Here
// the 16 columns hold the tail's 4 features 4 times over (column 4 a + c:
// feature f0 + c, replica a), lane 16 qw + 4 a + c adds feature c for
// replica a, and the replicas take different rows, so every lane adds a live
// feature and the 16 lanes of a quarter wave still hit 16 distinct columns
// (bank pairs).  A wave step covers 128 rows: replica a of quarter qw takes
// rows rA = r0 + 32 qw + 8 a .. rA + 7 (one 8-byte load of the lane's
// feature's bins); lane (a, c) loads g and h of rows rA + 2 c and rA + 2 c + 1
// (8-byte loads), and the J-th add of a replica's lanes takes row rA + J's
// word from lane (a, J / 2) of the quad with a DPP quad_perm.  A block step
// is 2048 rows, 512 per column, so an epoch (2048 rows of a cell between two
// unpacks) is 4 steps: one round of the ring, whose cell buffer alternates by
// round.  The flush sums a feature's 4 replicas before its global atomics.
// Block tb takes rows [tb span, (tb + 1) span), span a multiple of 2048.  The
// loop adds rows below n rounded down to even (the pairs); an odd n's last
// row is added after it.
// ---------------------------------------------------------------------------

// This lane's copy of the 64-bit word of lane S of its quad (DPP quad_perm).
template <int S>
__device__ __forceinline__ uint64_t quad_bcast64(uint64_t v) {
    constexpr int CTRL = S * 0x55;   // quad_perm [S, S, S, S]
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)hi << 32) | lo;
}

// Final flush of a tail block: as flush_cells_gh, with each feature's 4
// replica columns summed first (thread j: feature f0 + j / 256, bin j % 256).
template <bool HCH>
__device__ __forceinline__ void flush_tail_gh(RootFlushLds& T, const int64_t (&g)[RENT], const int64_t (&h)[RENT],
                                              const uint32_t* __restrict__ counts,
                                              const int32_t* __restrict__ dflt, int64_t* out, int F, int f0) {
    static_assert(TAILF * NB == RBLOCK, "one thread per (tail feature, bin)");
#pragma unroll
    for (int k = 0; k < RENT; ++k) {
        const int i = threadIdx.x + k * RBLOCK;
        const int fl = i % HFL;
        const int j = fl * NB + ((i / HFL) ^ (2 * fl));
        T.g[j] = (unsigned long long)g[k];
        if (HCH) T.h[j] = (unsigned long long)h[k];
    }
    __syncthreads();
    const int c = threadIdx.x / NB, b = threadIdx.x % NB;
    const int fi = f0 + c;
    if (fi >= F) return;
    unsigned long long sg = 0, sh = 0;
#pragma unroll
    for (int a = 0; a < HFL / TAILF; ++a) {
        const int fl = c + TAILF * a;
        const int j = fl * NB + (b ^ (2 * fl));
        sg += T.g[j];
        if (HCH) sh += T.h[j];
    }
    const size_t plane = (size_t)F * NB;
    const size_t at = (size_t)fi * NB + (size_t)b;
    if (sg) atomicAdd((unsigned long long*)(out + at), sg);
    if (HCH && sh) atomicAdd((unsigned long long*)(out + plane + at), sh);
    if (counts) {
        const uint32_t cj = counts[at];
        const int d = dflt ? dflt[fi] : -1;   // the default bin's count is left to the caller's fill
        if (cj && b != d) atomicAdd((unsigned long long*)(out + 2 * plane + at), (unsigned long long)cj);
    }
}

// MODE as in hist_root_gh; BUF: root_buffers holds for the tail's spans
// (loads through buffer resources bounded at the span's last whole pair).
template <int MODE, bool SKIP, bool BUF>
__device__ __forceinline__ void hist_root_tail(HistLdsR& L, const uint8_t* __restrict__ bins_fm, int64_t ld,
                                               const float* __restrict__ grad, const float* __restrict__ hess,
                                               int64_t n, int F, double scg, double sch,
                                               const int32_t* __restrict__ dflt,
                                               const uint32_t* __restrict__ counts, Quant* q_tot, int64_t* out,
                                               int64_t span, int tb) {
    constexpr bool HCH = MODE != ROOT_G, PACK = MODE == ROOT_PACKED;
    const int f0 = F / HFL * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int col = lane & (HFL - 1), c = lane & (TAILF - 1), a = col / TAILF, qw = lane / HFL;
    const int f = f0 + c;
    const bool fok = f < F;
    const int64_t lo = (int64_t)tb * span, hi = min(n, lo + span);
    if (lo >= hi) return;
    const int64_t n2 = n & ~(int64_t)1;   // the loop adds rows [lo, hi2): whole pairs
    const int64_t hi2 = min(hi, n2);
    const int d = (SKIP && fok) ? dflt[f] : -1;
    const bool totals = q_tot != nullptr && f0 == 0;
    for (int i = threadIdx.x; i < NB * 2 * HFL; i += RBLOCK) L.w[i] = 0;
    const uint32_t lbase = (uint32_t)col << 3;
    char* const lds = reinterpret_cast<char*>(L.w);
    int64_t ag[RENT], ah[RENT];
#pragma unroll
    for (int k = 0; k < RENT; ++k) ag[k] = ah[k] = 0;
    auto cell = [](int k) { const int i = threadIdx.x + k * RBLOCK; return (i / HFL) * (2 * HFL) + (i % HFL); };
    auto unpack = [&](int p) {
#pragma unroll
        for (int k = 0; k < RENT; ++k) {
            const int cc = cell(k) + p * HFL;
            const uint64_t v = L.w[cc];
            L.w[cc] = 0;
            const int64_t hs = (int64_t)(int32_t)(uint32_t)v;
            ah[k] += hs;
            ag[k] += (int64_t)(v - (uint64_t)hs) >> 32;
        }
    };
    const uint8_t* colp = bins_fm + (size_t)(fok ? f : f0) * ld;
    // Inputs of step s: g and h of this lane's row pair, and 8 rows of its
    // feature's bins.
    //   BUF: offsets from the span's first row (even, like the pairs, so no
    //   8-byte load straddles the end hi2 of the resources: pairs past it
    //   read zeros); the bins' resource ends with the last feature below F.
    //   Otherwise unconditional loads: the pair clamped to the last whole
    //   pair (n2 >= 2, so the 8-byte loads stay inside the arrays; its words
    //   are masked below), and the bins at rA % 8 == 0 with rA < hi <= n <=
    //   ld (ld % 16 == 0), or at lo when past hi.
    const int nf = F - f0;
    const uint32_t rpos = (uint32_t)(wave * (2 * WAVE) + 32 * qw + 8 * a);
    const __amdgpu_buffer_rsrc_t rsg = raw_rsrc(grad + lo, BUF ? (uint32_t)((hi2 - lo) * 4) : 0u);
    const __amdgpu_buffer_rsrc_t rsh = raw_rsrc(hess + lo, (BUF && HCH) ? (uint32_t)((hi2 - lo) * 4) : 0u);
    const __amdgpu_buffer_rsrc_t rsb =
        raw_rsrc(bins_fm + (size_t)f0 * ld + lo, BUF ? (uint32_t)((int64_t)nf * ld - lo) : 0u);
    const uint32_t vg = (rpos + 2u * (uint32_t)c) * 4u;
    const uint32_t vb = (uint32_t)((int64_t)c * ld) + rpos;
    auto load = [&](int64_t s, float2& gv, float2& hv, uint2& bw) {
        if (BUF) {
            typedef int v2i __attribute__((ext_vector_type(2)));
            const int so = (int)(s * TSTEP);
            // issued in this order wherever load runs (see the ring below)
            const v2i gw = __builtin_amdgcn_raw_buffer_load_b64(rsg, (int)vg, so * 4, 0);
            gv = make_float2(__int_as_float(gw.x), __int_as_float(gw.y));
            __builtin_amdgcn_sched_barrier(0);
            if (HCH) {
                const v2i hw = __builtin_amdgcn_raw_buffer_load_b64(rsh, (int)vg, so * 4, 0);
                hv = make_float2(__int_as_float(hw.x), __int_as_float(hw.y));
            }
            __builtin_amdgcn_sched_barrier(0);
            const v2i b = __builtin_amdgcn_raw_buffer_load_b64(rsb, (int)vb, so, 0);
            bw = make_uint2((uint32_t)b.x, (uint32_t)b.y);
            __builtin_amdgcn_sched_barrier(0);
        } else {
            const int64_t rA = lo + s * TSTEP + rpos;
            const int64_t p = min(rA + 2 * c, n2 - 2);
            gv = *reinterpret_cast<const float2*>(grad + p);
            if (HCH) hv = *reinterpret_cast<const float2*>(hess + p);
            bw = *reinterpret_cast<const uint2*>(colp + (rA < hi ? rA : lo));
        }
    };
    const int64_t steps = (hi - lo + TSTEP - 1) / TSTEP;
    // Packed cells need epochs only where the per-fit table's bound over the
    // span (each column takes a quarter of its rows, at most) reaches
    // PACKED_CELL_ROWS, as in hist_root_gh.
    bool epochs = PACK;
    if (PACK && counts) {
        const uint32_t* segmax = counts + (size_t)F * NB;
        const int64_t nseg = count_segments(n);
        uint32_t bound = 0;
        if (fok)
            for (int64_t sg = lo / SEG_ROWS; sg <= (hi - 1) / SEG_ROWS; ++sg) bound += segmax[(size_t)f * nseg + sg];
        bound = (uint32_t)__builtin_amdgcn_readfirstlane((int)wave_max_u32_v(bound));
        epochs = (int64_t)bound >= PACKED_CELL_ROWS;
    }
    // The ring as in hist_root_gh: TAIL_DEPTH stages, the first round's loads
    // issued before the loop in the loop's order.
    float2 gs[TAIL_DEPTH], hs[TAIL_DEPTH];
    uint2 bs[TAIL_DEPTH];
#pragma unroll
    for (int j = 0; j < TAIL_DEPTH; ++j) {
        hs[j] = make_float2(0.0f, 0.0f);
        __builtin_amdgcn_sched_barrier(0);
        load(j, gs[j], hs[j], bs[j]);
    }
    __syncthreads();
    int64_t sum_g = 0, sum_h = 0;
    uint32_t buf = 0;   // the cell buffer of this ring round's epoch
    for (int64_t s0 = 0; s0 < steps; s0 += TAIL_DEPTH) {
        const uint32_t lb = PACK ? (lbase | (buf << 7)) : lbase;
#pragma unroll
        for (int j = 0; j < TAIL_DEPTH; ++j) {
            const int64_t s = s0 + j;
            __builtin_amdgcn_sched_barrier(0);
            const int64_t p = lo + s * TSTEP + rpos + 2 * c;
            const bool ok0 = BUF || p < hi2, ok1 = BUF || p + 1 < hi2;
            const int64_t g0 = ok0 ? (PACK ? quantise_node(gs[j].x, scg) : quantise_wide(gs[j].x, scg)) : 0;
            const int64_t g1 = ok1 ? (PACK ? quantise_node(gs[j].y, scg) : quantise_wide(gs[j].y, scg)) : 0;
            const int64_t h0 = (HCH && ok0) ? (PACK ? quantise_node(hs[j].x, sch) : quantise_wide(hs[j].x, sch)) : 0;
            const int64_t h1 = (HCH && ok1) ? (PACK ? quantise_node(hs[j].y, sch) : quantise_wide(hs[j].y, sch)) : 0;
            const uint32_t wv[2] = {bs[j].x, bs[j].y};
            uint32_t at[8];
            uint32_t keep = 0xffu;
#pragma unroll
            for (int J = 0; J < 8; ++J) {
                at[J] = bin_addr_rt(wv[J >> 2], lb, J & 3);
                if (SKIP && (int)((wv[J >> 2] >> (8 * (J & 3))) & 0xffu) == d) keep &= ~(1u << J);
            }
            load(s + TAIL_DEPTH, gs[j], hs[j], bs[j]);
            if (SKIP) {
                sum_g += g0 + g1;
                sum_h += h0 + h1;
            }
            const uint64_t w0 = PACK ? ((uint64_t)g0 << 32) + (uint64_t)h0 : (uint64_t)g0;
            const uint64_t w1 = PACK ? ((uint64_t)g1 << 32) + (uint64_t)h1 : (uint64_t)g1;
            // ROOT_WIDE: the h cell is the g cell's twin in the other buffer
#define YABT_TAIL_ADD(J)                                                         \
            {                                                                    \
                const uint64_t wj = quad_bcast64<(J) / 2>(((J) & 1) ? w1 : w0);  \
                unsigned long long* const cp = reinterpret_cast<unsigned long long*>(lds + at[J]); \
                if (!SKIP || ((keep >> (J)) & 1u)) {                             \
                    atomicAdd(cp, (unsigned long long)wj);                       \
                    if (MODE == ROOT_WIDE)                                       \
                        atomicAdd(cp + HFL, (unsigned long long)quad_bcast64<(J) / 2>(  \
                                                ((J) & 1) ? (uint64_t)h1 : (uint64_t)h0)); \
                }                                                                \
            }
            YABT_TAIL_ADD(0) YABT_TAIL_ADD(1) YABT_TAIL_ADD(2) YABT_TAIL_ADD(3)
            YABT_TAIL_ADD(4) YABT_TAIL_ADD(5) YABT_TAIL_ADD(6) YABT_TAIL_ADD(7)
#undef YABT_TAIL_ADD
        }
        if (epochs) {
            // end of the epoch: read this round's buffer while the next round
            // adds into the other one
            __syncthreads();
            unpack((int)buf);
            buf ^= 1u;
        }
    }
    // an odd n's last row, in the block that holds it (a block-uniform test)
    if (n2 < n && hi == n) {
        if (wave == 0 && qw == 0 && a == 0) {   // lanes c = 0 .. 3: one per feature
            const int64_t r = n - 1;
            const int64_t gq = PACK ? quantise_node(grad[r], scg) : quantise_wide(grad[r], scg);
            const int64_t hq = HCH ? (PACK ? quantise_node(hess[r], sch) : quantise_wide(hess[r], sch)) : 0;
            if (SKIP && c == 0) {
                sum_g += gq;
                sum_h += hq;
            }
            const uint32_t b = colp[r];
            const uint64_t word = PACK ? ((uint64_t)gq << 32) + (uint64_t)hq : (uint64_t)gq;
            const uint32_t lb = PACK ? (lbase | (buf << 7)) : lbase;
            if (!SKIP || (int)b != d) {
                unsigned long long* const cp = reinterpret_cast<unsigned long long*>(lds + ((b << 8) | lb));
                atomicAdd(cp, (unsigned long long)word);
                if (MODE == ROOT_WIDE) atomicAdd(cp + HFL, (unsigned long long)hq);
            }
        }
        __syncthreads();
        if (epochs) unpack((int)buf);
    }
    __syncthreads();
    if (PACK && !epochs) unpack(0);
    if (!PACK) {   // never unpacked: the cells are the g sums (and the h sums)
#pragma unroll
        for (int k = 0; k < RENT; ++k) {
            ag[k] = (int64_t)L.w[cell(k)];
            if (HCH) ah[k] = (int64_t)L.w[cell(k) + HFL];
        }
    }
    if (totals) {
        if (!SKIP) {   // thread t's cells are of column t % HFL, feature t % TAILF
            sum_g = 0;
            sum_h = 0;
            if (threadIdx.x % TAILF == 0) {
#pragma unroll
                for (int k = 0; k < RENT; ++k) {
                    sum_g += ag[k];
                    sum_h += ah[k];
                }
            }
        }
        sum_g = wave_sum<int64_t>(sum_g);
        sum_h = wave_sum<int64_t>(sum_h);
        if (lane == 0) {
            atomicAdd((unsigned long long*)&q_tot->tot_g, (unsigned long long)sum_g);
            atomicAdd((unsigned long long*)&q_tot->tot_h, (unsigned long long)sum_h);
        }
    }
    __syncthreads();   // every cell read before the LDS is rewritten
    flush_tail_gh<HCH>(*reinterpret_cast<RootFlushLds*>(&L), ag, ah, tb == 0 ? counts : nullptr,
                       SKIP ? dflt : nullptr, out, F, f0);
}

// Per-fit count table of the feature-major bins (yabt_bin_counts): counts
// (F, 256) -- rows r < n with bin b in feature f, added into (cleared
// beforehand) -- then segmax (F, count_segments(n)): the largest count of any
// bin of feature f among rows [s SEG_ROWS, (s + 1) SEG_ROWS), written.  Block
// (tile, s) counts segment s of its 16 features in LDS (one 32-bit LDS
// atomic per row and feature).
static __global__ __attribute__((unused)) void __launch_bounds__(HBLOCK)
k_bin_count_seg(const uint8_t* __restrict__ bins_fm, int64_t ld, int64_t n, int F, uint32_t* __restrict__ table) {
    __shared__ uint32_t c[NB * HFL];   // [bin][feature]
    __shared__ uint32_t mx[HFL];
    const int64_t nseg = count_segments(n);
    const int tile = (int)(blockIdx.x / nseg);
    const int64_t sg = blockIdx.x % nseg;
    const int f0 = tile * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int64_t lo = sg * SEG_ROWS, hi = min(n, lo + SEG_ROWS);
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) c[i] = 0;
    if (threadIdx.x < HFL) mx[threadIdx.x] = 0;
    __syncthreads();
    const uint8_t* col = bins_fm + (size_t)(fok ? f : f0) * ld;
    for (int64_t r0 = lo + (int64_t)wave * WAVE; r0 < hi; r0 += HSTEP) {
        // base % 16 == 0 and base < hi <= n <= ld (ld % 16 == 0): in the row
        const int64_t base = r0 + HFL * rg;
        if (!fok || base >= hi) continue;
        const uint4 bv = *reinterpret_cast<const uint4*>(col + base);
        const uint32_t w[4] = {bv.x, bv.y, bv.z, bv.w};
        const int nv = (int)min((int64_t)HFL, hi - base);
#pragma unroll
        for (int J = 0; J < HFL; ++J) {
            const int b = (int)((w[J >> 2] >> (8 * (J & 3))) & 0xffu);
            if (J < nv) atomicAdd(&c[b * HFL + fl], 1u);
        }
    }
    __syncthreads();
    // thread t's cells t + k HBLOCK all hold feature t % HFL
    uint32_t m = 0;
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        const int fi = f0 + (i % HFL);
        const uint32_t v = c[i];
        m = max(m, v);
        if (fi < F && v) atomicAdd(table + (size_t)fi * NB + (size_t)(i / HFL), v);
    }
    m = max(m, (uint32_t)__shfl_xor((int)m, HFL, WAVE));
    m = max(m, (uint32_t)__shfl_xor((int)m, 2 * HFL, WAVE));
    if (lane < HFL) atomicMax(&mx[lane], m);
    __syncthreads();
    if (threadIdx.x < HFL && f0 + (int)threadIdx.x < F)
        table[(size_t)F * NB + (size_t)(f0 + threadIdx.x) * nseg + sg] = mx[threadIdx.x];
}

// Bin counts of all n rows of the feature-major bins, per (feature, bin):
// OUT64 false: added into a uint32 (F, 256) table (the per-fit counts);
// OUT64 true: added into an int64 (F, 256) count plane.  dflt (may be NULL):
// bin dflt[f] is not counted.  Same grid and row chunks as k_hist_root; one
// 32-bit LDS atomic per (row, feature).
template <bool OUT64>
static __global__ __attribute__((unused)) void __launch_bounds__(HBLOCK)
k_bin_count(const uint8_t* __restrict__ bins_fm, int64_t ld, int64_t n, int F, const int32_t* __restrict__ dflt,
            void* out, int chunks) {
    __shared__ uint32_t c[NB * HFL];   // [bin][feature]
    const int tile = blockIdx.x / chunks, chunk = blockIdx.x % chunks;
    const int f0 = tile * HFL;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    const int fl = lane & (HFL - 1), rg = lane / HFL;
    const int f = f0 + fl;
    const bool fok = f < F;
    const int64_t per = ((n + chunks - 1) / chunks + HSTEP - 1) / HSTEP * HSTEP;
    const int64_t lo = (int64_t)chunk * per, hi = min(n, lo + per);
    if (f0 >= F || lo >= hi) return;
    const int d = (fok && dflt) ? dflt[f] : -1;
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) c[i] = 0;
    __syncthreads();
    const uint8_t* col = bins_fm + (size_t)(fok ? f : f0) * ld;
    for (int64_t r0 = lo + (int64_t)wave * WAVE; r0 < hi; r0 += HSTEP) {
        // base % 16 == 0 and base < hi <= n <= ld (ld % 16 == 0): in the row
        const int64_t base = r0 + HFL * rg;
        if (!fok || base >= hi) continue;
        const uint4 bv = *reinterpret_cast<const uint4*>(col + base);
        const uint32_t w[4] = {bv.x, bv.y, bv.z, bv.w};
        const int nv = (int)min((int64_t)HFL, hi - base);
#pragma unroll
        for (int J = 0; J < HFL; ++J) {
            const int b = (int)((w[J >> 2] >> (8 * (J & 3))) & 0xffu);
            if (J < nv && b != d) atomicAdd(&c[b * HFL + fl], 1u);
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        const int fi = f0 + (i % HFL);
        const uint32_t v = c[i];
        if (fi >= F || v == 0) continue;
        const size_t at = (size_t)fi * NB + (size_t)(i / HFL);
        if (OUT64)
            atomicAdd(reinterpret_cast<unsigned long long*>(out) + at, (unsigned long long)v);
        else
            atomicAdd(reinterpret_cast<uint32_t*>(out) + at, v);
    }
}

// The streaming root histogram.  count_mode 0: g and h planes; 1: no h plane
// when q->const_h.  counts: the per-fit bin counts, added into the count
// plane by the chunk-0 blocks (NULL: the count plane is not touched).
// SKIP: dflt is given (a separate kernel, so that the loops without the
// default-bin test are compiled on their own).  BUF: root_buffers holds for
// the full tiles' chunks (hist_root_gh).
template <bool SKIP, bool BUF>
static __global__ __attribute__((unused)) void __launch_bounds__(RBLOCK)
k_hist_root(const uint8_t* __restrict__ bins_fm, int64_t ld, const float* __restrict__ grad,
            const float* __restrict__ hess, int64_t n, int F, const Quant* q, double scg_v, double sch_v,
            int wide_v, const int32_t* __restrict__ dflt, const uint32_t* __restrict__ counts, Quant* q_tot,
            int64_t* out, int tiles, int chunks, int tail, int64_t tail_rows, int xcd, int count_mode,
            const int32_t* done) {
    const int32_t dn = done ? *done : 0;
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const bool no_h = count_mode && q && q->const_h;
    const bool wide = q ? q->wide != 0 : wide_v != 0;
    if (dn) return;
    __shared__ HistLdsR L;   // 64 KB, also the flush's RootFlushLds
    static_assert(sizeof(RootFlushLds) <= sizeof(HistLdsR), "the flush reuses the cells' LDS");
    int tile, chunk, tb;
    if (!root_block((int)blockIdx.x, tiles, chunks, tail, xcd, tile, chunk, tb)) return;
    if (tb >= 0) {
        if (no_h)
            hist_root_tail<ROOT_G, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot, out,
                                              tail_rows, tb);
        else if (wide)
            hist_root_tail<ROOT_WIDE, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot,
                                                 out, tail_rows, tb);
        else
            hist_root_tail<ROOT_PACKED, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot,
                                                   out, tail_rows, tb);
        return;
    }
    if (no_h)
        hist_root_gh<ROOT_G, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot, out, chunks,
                                        tile, chunk);
    else if (wide)
        hist_root_gh<ROOT_WIDE, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot, out,
                                           chunks, tile, chunk);
    else
        hist_root_gh<ROOT_PACKED, SKIP, BUF>(L, bins_fm, ld, grad, hess, n, F, scg, sch, dflt, counts, q_tot, out,
                                             chunks, tile, chunk);
}

// One launch of k_hist_root over grid g: the instantiation with the
// default-bin test when dflt is given, with buffer loads when the chunks
// allow them.
static __attribute__((unused)) void launch_root_kernel(hipStream_t stream, const RootGrid& g, const uint8_t* bins_fm,
                                                       int64_t ld, const float* grad, const float* hess, int64_t n,
                                                       int F, const Quant* q, double scg, double sch, int wide,
                                                       const int32_t* dflt, const uint32_t* counts, Quant* q_tot,
                                                       int64_t* out, int count_mode, const int32_t* done) {
    const bool buf = root_buffers(ld, max(g.chunks > 0 ? root_chunk_rows(n, g.chunks) : 0, g.tail_rows));
#define YABT_ROOT_LAUNCH(S, B)                                                                                     \
    k_hist_root<S, B><<<g.blocks, RBLOCK, 0, stream>>>(bins_fm, ld, grad, hess, n, F, q, scg, sch, wide, dflt,   \
                                                       counts, q_tot, out, g.tiles, g.chunks, g.tail, g.tail_rows, \
                                                       g.xcd, count_mode, done)
    if (dflt) {
        if (buf) YABT_ROOT_LAUNCH(true, true);
        else YABT_ROOT_LAUNCH(true, false);
    } else {
        if (buf) YABT_ROOT_LAUNCH(false, true);
        else YABT_ROOT_LAUNCH(false, false);
    }
#undef YABT_ROOT_LAUNCH
}

// Launch the root histogram (grid from root_grid) into the (3, F, 256)
// histogram `out` (cleared beforehand).  With counts == NULL the count plane
// is counted from the bins first (k_bin_count, one more pass over them);
// callers that keep the per-fit counts pass them instead.  The instantiation
// with the default-bin test runs only when dflt is given.
static __attribute__((unused)) void launch_hist_root(hipStream_t stream, const uint8_t* bins_fm, int64_t ld,
                                                     const float* grad, const float* hess, int64_t n, int F,
                                                     const Quant* q, double scg, double sch, int wide,
                                                     const int32_t* dflt, const uint32_t* counts, Quant* q_tot,
                                                     int64_t* out, int count_mode, const int32_t* done) {
    if (!counts) {
        const int tiles = (F + HFL - 1) / HFL;
        const int rc = root_chunks(n, tiles);
        k_bin_count<true><<<tiles * rc, HBLOCK, 0, stream>>>(bins_fm, ld, n, F, dflt, out + (size_t)2 * F * NB, rc);
    }
    launch_root_kernel(stream, root_grid(n, F, grad, hess), bins_fm, ld, grad, hess, n, F, q, scg, sch, wide, dflt,
                       counts, q_tot, out, count_mode, done);
}

// Rows of one node for a gather launch.
struct HistJob {
    int32_t active;
    int32_t pad;
    const uint32_t* rows;      // row ids of the node at positions [lo, hi)
    int64_t lo, hi;
    int64_t* out;              // [3][F][256], cleared beforehand, added into
};

// Chunks of a gather launch over m rows.
__host__ __device__ inline int gather_chunks(int64_t m) {
    const int64_t c = (m + GATHER_MIN_ROWS - 1) / GATHER_MIN_ROWS;
    return (int)(c < GATHER_MAX_CHUNKS ? c : GATHER_MAX_CHUNKS);
}

// The 16 bytes of v rotated by k (0..15): byte j of the result is byte
// (j + k) & 15 of v.
__device__ __forceinline__ uint4 rotate_bytes16(uint4 v, int k) {
    const bool d1 = (k >> 2) & 1, d2 = (k >> 3) & 1;
    const uint32_t b0 = d1 ? v.y : v.x, b1 = d1 ? v.z : v.y, b2 = d1 ? v.w : v.z, b3 = d1 ? v.x : v.w;
    const uint32_t c0 = d2 ? b2 : b0, c1 = d2 ? b3 : b1, c2 = d2 ? b0 : b2, c3 = d2 ? b1 : b3;
    const uint32_t r = (uint32_t)(k & 3);
    return make_uint4(__builtin_amdgcn_alignbyte(c1, c0, r), __builtin_amdgcn_alignbyte(c2, c1, r),
                      __builtin_amdgcn_alignbyte(c3, c2, r), __builtin_amdgcn_alignbyte(c0, c3, r));
}

// Histogram of the rows listed at rows[lo:hi] over features [16 tile,
// 16 tile + 16), bins gathered from the row-major copy, into out (3, F, 256):
// added with global atomics (STORE false: out holds the sums so far) or
// stored (STORE true: out is this block's own piece), with the packed count
// of hist_root's kind: the count rides in the low cb = wlog + 1 bits of one
// 64-bit LDS word, (q << cb) + 1 per row (q = q(h), or q(g) when every h is
// equal), and each window of 2^wlog rows is unpacked into registers; with the
// h channel q(g) has a word of its own.  Two 64-bit LDS atomics per update
// (one without the h channel).  The whole block calls it (barriers inside).
//
// Each lane takes one row per step: its row id, its g and h, and the 16
// bytes of its row's bins for the tile with one 16-byte load, so each lane
// adds its own row's words (no broadcast).  The bytes are rotated by
// k = lane % 16, and the lane's J-th add goes to feature (J + k) % 16: the 16
// lanes of a quarter wave then hit 16 different features (bank pairs) at
// every add, whatever the bins are.  Features >= F are the row-major copy's
// zero padding, added into LDS columns the flush ignores; rows past hi read
// row hi - 1 and add zero words.  A three-stage pipeline per wave: at step s
// the wave adds step s, loads g, h and the bins of step s + 1 (its row ids
// are in registers) and the row ids of step s + 2.
template <bool HCH, bool SKIP, bool STORE = false>
__device__ __forceinline__ void hist_gather_rows(GatherLds& LU, const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                 const float* __restrict__ grad, const float* __restrict__ hess,
                                                 int F, double scg, double sch, const int32_t* __restrict__ dflt,
                                                 const uint32_t* __restrict__ rows, int64_t lo, int64_t hi,
                                                 int64_t* out, int wlog, int tile,
                                                 const float2* __restrict__ gh = nullptr) {
    const int f0 = tile * HFL;
    if (f0 >= F || lo >= hi) return;
    HistLdsP& L = LU.p;
    const int lane = threadIdx.x & (WAVE - 1), wave = threadIdx.x / WAVE;
    int k = lane & (HFL - 1);
    // k is opaque from here: values derived from it are computed per call, not
    // hoisted out of a caller's loop over units and kept live across it
    asm volatile("" : "+v"(k));
    // with SKIP: byte j of dv is the default bin of feature f0 + (j + k) % 16,
    // bit j of dmask says that feature has one
    uint4 dv = make_uint4(0, 0, 0, 0);
    uint32_t dmask = 0;
    if (SKIP) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int j = 0; j < HFL; ++j) {
            const int fj = f0 + ((j + k) & (HFL - 1));
            const int d = fj < F ? dflt[fj] : -1;
            if (d >= 0) {
                w[j >> 2] |= (uint32_t)d << (8 * (j & 3));
                dmask |= 1u << j;
            }
        }
        dv = make_uint4(w[0], w[1], w[2], w[3]);
    }
    const int cb = wlog + 1;
    const uint64_t cmask = ((uint64_t)1 << cb) - 1;
    const int64_t win_steps = (int64_t)1 << (wlog - 10);
    const uint8_t* tb = bins_rm + f0;                // a row's 16 bytes of the tile: tb + r * ld (ld % 16 == 0)
    const int64_t w0 = lo + (int64_t)wave * WAVE;   // this wave's rows at step s: w0 + s * HSTEP + [0, 64)
    auto row_at = [&](int64_t i) { return rows[min(i, hi - 1)]; };
    // stage inputs: row ids of steps 0 and 1, g/h/bins of step 0
    const uint32_t r0 = row_at(w0 + lane);
    uint32_t r1 = row_at(w0 + HSTEP + lane);
    for (int i = threadIdx.x; i < NB * HFL; i += HBLOCK) {
        if (HCH) L.g[i] = 0;
        L.p[i] = 0;
    }
    int64_t qa[HENT];
    uint32_t ca[HENT];
#pragma unroll
    for (int e = 0; e < HENT; ++e) {
        qa[e] = 0;
        ca[e] = 0;
    }
    // a row's g and h: one 8-byte load from the interleaved copy when given
    // (one sector for both), else two
    auto load_gh = [&](uint32_t r, float& g, float& h) {
        if (gh) {
            const float2 v = gh[r];
            g = v.x;
            h = HCH ? v.y : 0.0f;
        } else {
            g = grad[r];
            h = HCH ? hess[r] : 0.0f;
        }
    };
    float gx, hx;
    load_gh(r0, gx, hx);
    uint4 bv = *reinterpret_cast<const uint4*>(tb + (size_t)r0 * ld);
    __syncthreads();
    const int64_t steps = (hi - lo + HSTEP - 1) / HSTEP;   // the same in every wave: barriers below
    for (int64_t s = 0; s < steps; ++s) {
        const int64_t i0 = w0 + s * HSTEP, i1 = i0 + HSTEP, i2 = i1 + HSTEP;
        // stage: row ids of step s + 2; g, h and bins of step s + 1
        const uint32_t r2 = row_at(i2 + lane);
        float gn, hn;
        load_gh(r1, gn, hn);
        const uint4 bn = *reinterpret_cast<const uint4*>(tb + (size_t)r1 * ld);
        // step s
        const bool rok = i0 + lane < hi;
        const int64_t gq = rok ? quantise_wide(gx, scg) : 0;
        const int64_t hq = (HCH && rok) ? quantise_wide(hx, sch) : 0;
        const uint64_t one = rok ? 1 : 0;
        const uint64_t gw = HCH ? (uint64_t)gq : ((uint64_t)gq << cb) + one;
        const uint64_t pw = HCH ? ((uint64_t)hq << cb) + one : 0;
        const uint4 rb = rotate_bytes16(bv, k);
        const uint32_t wv[4] = {rb.x, rb.y, rb.z, rb.w};
        const uint32_t dw[4] = {dv.x, dv.y, dv.z, dv.w};
#pragma unroll
        for (int J = 0; J < HFL; ++J) {
            const uint32_t b = (wv[J >> 2] >> (8 * (J & 3))) & 0xffu;
            const int at = (int)(b * HFL) + ((J + k) & (HFL - 1));
            if (!SKIP || !((dmask >> J) & 1u) || b != ((dw[J >> 2] >> (8 * (J & 3))) & 0xffu)) {
                if (HCH) {
                    atomicAdd(&L.g[at], (unsigned long long)gw);
                    atomicAdd(&L.p[at], (unsigned long long)pw);
                } else {
                    atomicAdd(&L.p[at], (unsigned long long)gw);
                }
            }
        }
        if ((s + 1) % win_steps == 0 || s + 1 == steps) {
            __syncthreads();
#pragma unroll
            for (int e = 0; e < HENT; ++e) {
                const int i = threadIdx.x + e * HBLOCK;
                const uint64_t v = L.p[i];
                L.p[i] = 0;
                const uint64_t c = v & cmask;
                qa[e] += (int64_t)(v - c) >> cb;
                ca[e] += (uint32_t)c;
            }
            __syncthreads();
        }
        r1 = r2;
        gx = gn;
        hx = hn;
        bv = bn;
    }
    uint64_t gv[HENT];
#pragma unroll
    for (int e = 0; e < HENT; ++e) gv[e] = HCH ? L.g[threadIdx.x + e * HBLOCK] : (uint64_t)qa[e];
    __syncthreads();   // every g cell read before the LDS is rewritten
    flush_cells<HCH, STORE>(LU.u, gv, qa, ca, out, F, f0);
}

// Chunk `chunk` of the rows listed at rows[jlo:jhi]: a node of m rows uses
// gather_chunks(m) chunks of whole waves (other chunk numbers return at once).
template <bool HCH, bool SKIP>
__device__ __forceinline__ void hist_gather_packed(GatherLds& L, const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                   const float* __restrict__ grad, const float* __restrict__ hess,
                                                   int F, double scg, double sch, const int32_t* __restrict__ dflt,
                                                   const uint32_t* __restrict__ rows, int64_t jlo, int64_t jhi,
                                                   int64_t* out, int wlog, int tile, int chunk) {
    const int64_t m = jhi - jlo;
    if (tile * HFL >= F || m <= 0) return;
    const int nch = gather_chunks(m);
    if (chunk >= nch) return;
    const int64_t per = ((m + nch - 1) / nch + WAVE - 1) / WAVE * WAVE;
    const int64_t lo = jlo + (int64_t)chunk * per, hi = min(jhi, lo + per);
    hist_gather_rows<HCH, SKIP>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, rows, lo, hi, out, wlog, tile);
}

// job->active == 0 or *done != 0 (done may be NULL): nothing to do.  The
// packing window is q->wlog, or wlog_v when q is NULL (window_log2(n, wide)
// for the n rows and the contract the caller's shifts were chosen for).
static __global__ __attribute__((unused)) void __launch_bounds__(HBLOCK) k_hist_gather(const uint8_t* __restrict__ bins_rm, int64_t ld,
                                                        const float* __restrict__ grad,
                                                        const float* __restrict__ hess, int F, const Quant* q,
                                                        double scg_v, double sch_v,
                                                        const int32_t* __restrict__ dflt, const HistJob* job,
                                                        int count_mode, const int32_t* done, int wlog_v) {
    // independent loads first: the job record, the done flag, the shifts
    const HistJob jb = *job;
    const int32_t dn = done ? *done : 0;
    const double scg = q ? q->scg : scg_v, sch = q ? q->sch : sch_v;
    const int wlog = q ? q->wlog : wlog_v;
    const bool no_h = count_mode && q && q->const_h;
    if (dn || !jb.active) return;
    const int tile = blockIdx.x / GATHER_MAX_CHUNKS, chunk = blockIdx.x % GATHER_MAX_CHUNKS;
    __shared__ GatherLds L;
    if (no_h) {
        if (dflt)
            hist_gather_packed<false, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi,
                                            jb.out, wlog, tile, chunk);
        else
            hist_gather_packed<false, false>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi,
                                             jb.out, wlog, tile, chunk);
    } else {
        if (dflt)
            hist_gather_packed<true, true>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi,
                                           jb.out, wlog, tile, chunk);
        else
            hist_gather_packed<true, false>(L, bins_rm, ld, grad, hess, F, scg, sch, dflt, jb.rows, jb.lo, jb.hi,
                                            jb.out, wlog, tile, chunk);
    }
}

}  // namespace yabt
