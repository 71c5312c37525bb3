// dpep_internal.h -- host-side context and the kernel launchers shared by the
// translation units of libdpep.so.
#pragma once

#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include <type_traits>

#include "dpep_device.h"

// kern<<<grid, block, lds, s>>>(args...); with a profiling event pair (ev
// non-null: ev[0], ev[1]) the same launch through hipExtLaunchKernelGGL, which
// stamps the dispatch's own start and end into the two events, so a kernel's
// interval is its own and nothing is recorded between launches.  The kernel
// is passed in parentheses (a template's commas): DPEP_LAUNCH(ev, (k<T, L>), ...).
#define DPEP_UNPAREN(...) __VA_ARGS__
#define DPEP_LAUNCH(ev, kern, grid, block, lds, s, ...)                                   \
    do {                                                                                  \
        if (ev)                                                                           \
            hipExtLaunchKernelGGL(DPEP_UNPAREN kern, dim3(grid), dim3(block),              \
                                  (unsigned)(lds), s, (ev)[0], (ev)[1], 0u, __VA_ARGS__); \
        else                                                                              \
            DPEP_UNPAREN kern<<<dim3(grid), dim3(block), (lds), s>>>(__VA_ARGS__);         \
    } while (0)

namespace dpep {

// Rows per workgroup of the spectral passes are 2*F where F is the number of
// complex FFTs a workgroup holds in LDS.  The intermediate matrices are
// stored in tiles (T: TXT x TV, Ux / Uy: TX x TV elements) so that the passes
// move runs of whole tiles through HBM while writing "transposed".
int spectral_fpw(int L, int dtype);

struct Tiles {
    int TX;   // tile extent along x of Ux, Uy (= 2 * F of the length-N passes)
    int TV;   // tile extent along v of T, Ux, Uy (= 2 * F of the length-M pass)
    int TXT;  // tile extent along x of T: t_tile_rows()
};

// Rows of one T tile: at least the rows of a strip (the rows P1 writes at
// once) and TX, doubled until a tile fills a 128-byte cache line (P2 reads
// whole tiles: a half-line tile costs a second line fetch; at 4096 x 4096
// float32, 4-row tiles doubled P2's fetched bytes).  At most M.
__host__ __device__ constexpr int t_tile_rows(int R, int TX, int TV, size_t esz, int M)
{
    int t = R > TX ? R : TX;
    while ((size_t)t * TV * esz < 128 && t < M) t *= 2;
    return t;
}

struct SpectralArgs {
    int M, N;
    Tiles tiles;
    double wu_step;     // 2 pi / M
    double wv_step;     // 2 pi / N * bsx / bsy
    int potential;      // compute the potential map
    const void* twM;    // exp(-2 pi i m / M), m < M
    const void* postM;  // exp(-i pi k / 2M), k <= M/2
    const void* twN;
    const void* postN;
};

// Twiddle tables of a length-L transform on the device: tw[m] =
// exp(-2 pi i m / L) for m < L and post[k] = exp(-i pi k / 2L) for k <= L/2,
// interleaved (re, im) in T, evaluated in float64 (sincospi) and rounded once.
inline size_t twiddle_elems(int L) { return 2 * (size_t)L; }
inline size_t post_elems(int L) { return 2 * (size_t)(L / 2 + 1); }
template <typename T>
hipError_t launch_tables(int L, T* tw, T* post, hipStream_t s);

// Launchers (return hipError_t of the launch).  T = float or double.  ev:
// null, or the profiling event pair (start, end) of the pass's kernel.
template <typename T>
hipError_t launch_col_pass(const SpectralArgs& a, const T* Tt, T* Ux, T* Uy,
                           hipStream_t s, const hipEvent_t* ev = nullptr);
template <typename T>
hipError_t launch_row_inv(const SpectralArgs& a, const T* Ux, const T* Uy,
                          T* fx, T* fy, T* phi, hipStream_t s,
                          const hipEvent_t* ev = nullptr);
// ---------------------------------------------------------------------------
// Strip binning (kernels in dpep_bin.h)
// ---------------------------------------------------------------------------
constexpr int kBinThreads = 256;       // K1 / K3 workgroup size
constexpr int kCellsPerThread = 4;     // K1 / K3 cells per thread
constexpr int kCellsPerGroup = kBinThreads * kCellsPerThread;
constexpr int kOnceThreads = 512;      // one-pass K3 workgroup size
constexpr int kOnceCells = kOnceThreads * kCellsPerThread;   // its largest block
constexpr int kAccThreads = 1024;      // K4 workgroup size
constexpr int kCountSlots = 8;         // strip-total counters per strip
constexpr int kMaxSpanY = 4095;        // larger y spans take the tall path
constexpr int kSideBits = 128;         // column blocks tracked per strip in B
constexpr int kSideWords = kSideBits / 32;

// Cells of one problem at most: record numbers (regions, then the overflow
// pool: about 4.25 per cell) stay below the reserved pos values.
constexpr int kMaxCells = 1 << 28;

// Chunk sizes a step may choose for K4 / G1 work items: kChunkMin << k.
constexpr int kChunkMin = 1024;
constexpr int kChunkCands = 21;        // up to 2^30 records: never splits
constexpr int kAccChunkMin = 8192;     // smallest K4 chunk a step chooses

// Records of the (slot, strip) regions a step's plan may hold beyond the
// records themselves: each region gets its last demand plus an eighth plus
// kRegionSlack, so the regions of all slots and strips fit
// region_capacity() records.
constexpr unsigned kRegionSlack = 16;

// Shared between host (sizing) and device.
//
// Records live in kCountSlots regions per strip (workgroup g reserves its
// runs in region g % kCountSlots of each strip: the reservation atomics are
// spread over kCountSlots counters per strip).  K3's workgroup 0 publishes
// the step's plan: where the regions are (pbase, pcap) and the K4 / G1 work
// items.  Within a strip the records are numbered region after region,
// without the unfilled tail of each region ("strip-relative" numbers).  Two
// ways to fill:
//   fresh  K1 counts every (slot, strip) first; K3 places the regions
//          exactly (none overflows);
//   once   K3 alone: each region sized from the previous step's count of it
//          plus slack; K3 reserves in the regions as it sorts, and records
//          past a region's capacity go to the overflow pool: a block's part
//          of a strip that does not fit is one run of that strip's overflow
//          list (ovst, oruns), which K4 and G1 walk after the strip's
//          regions.
// The counts of a step stay for the next one: two sets, by step parity.
// K4's workgroup 0 re-zeroes the older set (and its pool count) once K3 has
// read it.
struct BinArgs {
    int S, R, lgR;          // strips, rows per strip, log2 R
    int G1;                 // K1/K3 workgroups of this step
    int Pacc, Pgat;         // K4 / G1 workgroups the device holds at once
    int Wacc, Wgat;         // K4 / G1 grids = capacities of their item lists
    int ch_force;           // > 0: every chunk this many records (tests only)
    int tight;              // 1: size each region at half its previous count,
                            // so the step overflows (tests only)
    int par;                // parity of this step: its set of counts
    int cus;                // CUs of the device
    int qcells;             // cells per one-pass block, the unit of the count
                            // slots (set per step: once_blocks)
    int sub, qsub;          // counting workgroups per one-pass block, and the
                            // cells of each but the block's last
                            // (set_count_blocks)
    unsigned reg_cap;       // records the regions of a plan may hold in total
    unsigned pool0;         // record number of the overflow pool's first entry
    unsigned pool_cap;      // capacity of the overflow pool (0: fresh-only)
    unsigned* cnt;          // [G1max][S] fresh: base of workgroup g in its slot
    unsigned* xtot;         // [2][kCountSlots][S] records counted / reserved per
                            // (slot, strip), the set of parity par this step
    unsigned* pbase;        // [kCountSlots][S] plan: first record of a region
    unsigned* pcap;         // [kCountSlots][S] plan: capacity of a region
    unsigned* chunk;        // [2] records per K4 / G1 item, chosen per plan
    uint4* items;           // [Wacc] K4 items: {strip | chunk << 16, first,
                            // end strip-relative record, chunks of the strip}
    unsigned* nitems;       // [2] K4, G1 item counts
    uint4* items_g;         // [Wgat] G1 items (same layout)
    unsigned* pool_n;       // [2] overflow records of the step of each parity
    unsigned long long* ovst;  // [2][S] per strip, the step of each parity:
                               // (overflow runs << 32) | overflow records
                               // (the older set zero again after K4)
    uint2* oruns;           // [S][rmax] a strip's overflow runs, in the order
                            // of its ovst atomics: {pool index of the run's
                            // first record, that record's number in the
                            // strip's overflow list}
    int rmax;               // runs a strip's list holds: one per one-pass
                            // block (run_capacity)
    unsigned* done;         // [S] K4 chunks done per strip (zero between steps)
    void* recg;             // [pool0 + pool_cap] record geometry, vec4 of T
    unsigned* recm;         // [pool0 + pool_cap] record span word (float64)
    unsigned long long* pos;   // [nc_max] records of cell i: first strip (or
                               // kPosTall / kPosNone) | second strip << 32
    void* gtmp;             // [pool0 + pool_cap] vec2 forces by record
    unsigned* bigflag;      // [kSideWords S] per strip: bitmap of the column
                            // blocks of its rows that hold tall-cell sums in B
                            // (zero between steps)
    void* B;                // [M*N] uint64, zero between steps: tall cells and
                            // the chunks of split strips add into it
    void* raw;              // [M*N] of T or null: the scattered cells' density
                            // alone (no initial density), written by K4's flush
};

// Geometry of one problem (bins, die, stretch, fixed-point scale) and the
// spectral passes' arguments (everything but the table pointers), shared by
// dpep_create and the no-alloc entry point so both compute identically.
inline void make_grid(Grid& g, int M, int N, double xl, double yl, double xh, double yh,
                      bool stretch, int nc_max, int esz)
{
    g = Grid{};
    g.M = M; g.N = N; g.xl = xl; g.yl = yl; g.xh = xh; g.yh = yh;
    g.bsx = (xh - xl) / M;
    g.bsy = (yh - yl) / N;
    g.inv_ba = 1.0 / (g.bsx * g.bsy);
    g.inv_bsx = 1.0 / g.bsx;
    g.inv_bsy = 1.0 / g.bsy;
    g.minw = M_SQRT2 * g.bsx;
    g.minh = M_SQRT2 * g.bsy;
    g.stretch = stretch ? 1 : 0;
    g.fix_scale = ldexp(1.0, fix_exponent_of(nc_max, esz));
}

// Host-side sizing of the binning buffers (shared with the CPU emulator).
constexpr size_t kTileBytes = 131072;  // LDS tile of K4 (uint64 words) and G1

// Rows per strip of an N-column grid: K4's LDS tile of R rows of N uint64
// words holds at most kTileBytes.
__host__ __device__ constexpr int strip_rows(int N)
{
    int R = 8;
    while (R > 1 && (size_t)R * N * 8 > kTileBytes) R >>= 1;
    return R;
}

struct BinPlan {
    int S, R, lgR, G1max;
    size_t cap;             // records (2 per cell)
    size_t reg_cap;         // region capacity of a planned step (>= cap)
    size_t geo_bytes;       // bytes of one record's geometry (4 elements)
    size_t span_bytes;      // bytes of its span word in recm (float64 only;
                            // float32 records carry it in the geometry)
};

// Records all (slot, strip) regions of a plan hold at most: every region's
// demand d plus d / 8 plus kRegionSlack, with sum d <= cap.
inline size_t region_capacity(size_t cap, int S)
{
    return cap + cap / 8 + (size_t)kRegionSlack * kCountSlots * (size_t)S;
}

// Rows of BinArgs::cnt: an upper bound of the counting workgroups
// (set_count_blocks) of any step of at most nc cells.  With q >= 1024 cells
// per one-pass block and at most kOnceThreads * kOnceMaxCpt, blocks * parts
// <= (nc / q + 1) * (q / 1024 + 1) <= 2 * nc / 1024 + 3.5.
inline int count_grid_max(long long nc)
{
    return (int)(2 * ((nc + kCellsPerGroup - 1) / kCellsPerGroup) + 4);
}

inline BinPlan make_bin_plan(int M, int N, int nc_max, size_t elem_bytes)
{
    BinPlan p{};
    p.geo_bytes = 4 * elem_bytes;
    p.span_bytes = elem_bytes == 4 ? 0 : sizeof(unsigned);
    int R = strip_rows(N);
    if (R > M) R = M;
    p.R = R;
    p.lgR = 0;
    while ((1 << p.lgR) < R) ++p.lgR;
    p.S = M / R;
    const long long nc = nc_max > 1 ? nc_max : 1;
    p.G1max = count_grid_max(nc);
    p.cap = (size_t)(2 * nc);
    p.reg_cap = region_capacity(p.cap, p.S);
    return p;
}

inline void make_spectral_args(SpectralArgs& a, const Grid& g, int dtype, bool potential)
{
    const size_t esz = dtype == 0 ? 4 : 8;
    a = SpectralArgs{};
    a.M = g.M; a.N = g.N;
    a.tiles.TX = 2 * spectral_fpw(g.N, dtype);
    a.tiles.TV = 2 * spectral_fpw(g.M, dtype);
    a.tiles.TXT = t_tile_rows(strip_rows(g.N), a.tiles.TX, a.tiles.TV, esz, g.M);
    a.wu_step = 2.0 * M_PI / g.M;
    a.wv_step = 2.0 * M_PI / g.N * (g.bsx / g.bsy);
    a.potential = potential ? 1 : 0;
}

// The work-item grids of K4 and G1 from the per-CU occupancy of each (both
// at least one workgroup per strip).
inline void set_item_grids(BinArgs& b, int acc_per_cu, int gat_per_cu, int cus)
{
    b.cus = cus > 0 ? cus : 1;
    b.Pacc = (acc_per_cu > 0 ? acc_per_cu : 1) * (cus > 0 ? cus : 1);
    b.Pgat = (gat_per_cu > 0 ? gat_per_cu : 1) * (cus > 0 ? cus : 1);
    b.Wacc = b.Pacc > b.S ? b.Pacc : b.S;
    b.Wgat = b.Pgat > b.S ? b.Pgat : b.S;
}

// The cell blocks of a step with nc cells, walked by the one-pass K3 and by
// G2 (one workgroup of kOnceThreads per block), and the unit of the count
// slots (block b counts in slot b % kCountSlots).  Equal blocks of q cells
// (a multiple of 64), as many per CU as are resident at once (three at
// float32, two at float64: registers), so every CU sorts the same number of
// cells in one round: 1.1 M float32 cells on 256 CUs make 748 blocks of
// 1472, where blocks of 2048 left 26 CUs a third block and K3 waited for
// them (two blocks of 2176 per CU measured 1.2 us slower than three).
// Blocks stay at kOnceMinCells or more (a block's records in a strip form
// one run: shorter runs write more partial lines); past that many blocks'
// worth of kOnceThreads * cpt cells they hold kOnceCells and run in rounds.
// cpt = ceil(q / kOnceThreads), the cells per thread the kernels are
// instantiated for, at most kOnceMaxCpt (five float64 cells per thread spill
// 48 of K3's registers, and still measured faster than a second round of
// 2048-cell blocks: 1.1 M float64 cells at 512^2 0.1062 -> 0.1002 ms).
constexpr int kOnceMaxCpt = 5;
constexpr int kOnceMinCells = kOnceThreads * 2;

// Overflow runs a strip's list can hold: each one-pass block adds at most
// one per strip, and a step of at most nc cells has at most
// ceil(nc / kOnceMinCells) blocks (once_blocks).
inline int run_capacity(long long nc_max)
{
    const long long nc = nc_max > 0 ? nc_max : 0;
    return (int)(nc / kOnceMinCells + 2);
}
struct OnceBlocks {
    int grid;   // blocks (at least one)
    int q;      // cells per block (the last one may hold fewer)
    int cpt;    // cells per thread: 2 .. kOnceMaxCpt
};
inline OnceBlocks once_blocks(int nc, int cus, size_t elem_bytes)
{
    const long long n = nc > 0 ? nc : 0;
    const long long per = (elem_bytes == 4 ? 3LL : 2LL) * (cus > 0 ? cus : 1);
    const long long qmax = (long long)kOnceThreads * kOnceMaxCpt;
    long long q = (n + per - 1) / per;
    q = (q + 63) / 64 * 64;
    if (q < kOnceMinCells) q = kOnceMinCells;
    if (q > qmax) q = kOnceCells;
    OnceBlocks o;
    o.q = (int)q;
    o.grid = (int)(n > q ? (n + q - 1) / q : 1);
    o.cpt = (int)((q + kOnceThreads - 1) / kOnceThreads);
    return o;
}

// The counting workgroups of a step (K1 and the fresh K3): one-pass block
// o is split into sub = ceil(q / kCellsPerGroup) parts of qsub cells (the
// block's last part takes the rest), workgroup w taking part w % sub of
// block w / sub.  No counting workgroup straddles two one-pass blocks, so
// the counts a fresh step leaves in each slot are exactly what the next
// one-pass step reserves there.
inline void set_count_blocks(BinArgs& b, const OnceBlocks& o)
{
    b.qcells = o.q;
    b.sub = (o.q + kCellsPerGroup - 1) / kCellsPerGroup;
    b.qsub = ((o.q + b.sub - 1) / b.sub + 63) / 64 * 64;
    b.G1 = o.grid * b.sub;
}

// fn(std::integral_constant<int, cpt>{}) for the cells per thread of a
// one-pass block (once_blocks().cpt); hipErrorInvalidValue for another.
template <typename Fn>
inline hipError_t with_cpt(int cpt, Fn&& fn)
{
    switch (cpt) {
    case 2: return fn(std::integral_constant<int, 2>{});
    case 3: return fn(std::integral_constant<int, 3>{});
    case 4: return fn(std::integral_constant<int, 4>{});
    case 5: return fn(std::integral_constant<int, 5>{});
    default: return hipErrorInvalidValue;
    }
}

// Strip-binned scatter (K1 unless `once`, K3, K4; K4 also runs the row DCT,
// writing T) and gather (G1, G2); the scatter's ev (nullable) receives 3
// ev (nullable): profiling event pairs (start, end), the scatter's for K1,
// K3 and K4 (six events; K1's unused when `once`), the gather's for G1 and G2
// (four).  `once` needs the counts of a previous step (parity b.par ^ 1) on
// the same buffers and an overflow pool of 2 * nc records (pool_cap).
template <typename T>
hipError_t launch_bin_scatter(const T* px, const T* py, const T* sx,
                              const T* sy, int nc, const Grid& g, BinArgs b,
                              const SpectralArgs& a, const T* d0n, T* dens, T* Tt,
                              bool once, hipStream_t s, const hipEvent_t* ev);
template <typename T>
hipError_t launch_bin_gather(const T* px, const T* py, const T* sx,
                             const T* sy, int nc, const Grid& g,
                             const BinArgs& b, const T* fx, const T* fy,
                             T* gx, T* gy, hipStream_t s, const hipEvent_t* ev);

// D0n = target_density * exact overlap of n fixed cells / bin area, through
// the side map B (left at zero).
template <typename T>
hipError_t launch_fixed_density(const T* px, const T* py, const T* sx, const T* sy,
                                int n, const Grid& g, double target_density,
                                void* B, T* d0n, hipStream_t s);

// Workgroups of K4 (row length N) and G1 that one CU holds at once.
template <typename T>
hipError_t bin_occupancy(int N, int R, int& acc_per_cu, int& gat_per_cu);

// Sets the dynamic-LDS limits of every spectral / binning kernel;
// prepare_kernels() does both once per process (later calls return the
// first one's status).
hipError_t spectral_prepare();
hipError_t bin_prepare();
hipError_t prepare_kernels();

// Records msg as the calling thread's dpep_last_error() text; returns code.
int report_error(int code, const char* msg);

}  // namespace dpep
