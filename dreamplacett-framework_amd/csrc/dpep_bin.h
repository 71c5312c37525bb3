// dpep_bin.h -- strip-binned density scatter and field gather.
//
// The bin map is cut into S strips of R consecutive rows (R * N uint64
// accumulators fit a 128 KB LDS tile).  A counting sort puts every cell into
// the strip(s) its x-span touches; each strip is accumulated in LDS by the
// workgroup that owns it and flushed with plain coalesced stores, the fixed
// density folded in on the way.  No global atomics on the common path.
//
//   k_bin_count   per-workgroup strip histograms; each nonzero count  K1
//                 is added to one of kCountSlots totals per strip and
//                 the returned old total is the workgroup's base
//   k_bin_fill    each workgroup scans the strip totals for its own   K3
//                 offsets (workgroup 0 publishes the strip table, the
//                 step's chunk sizes and the K4 / G1 item lists);
//                 cells -> strip-sorted records; tall cells -> B
//                 (K1 and this form: the first step, or every step
//                 with DPEP_FLAG_TWO_PASS; each one-pass block split
//                 into counting parts of at most 1024 cells)
//   k_bin_fill_once  the steady state: K3 without K1, on regions   K3
//                 sized from the previous step's counts; one equal
//                 block of cells per workgroup (once_blocks); records
//                 past a region's room -> overflow pool, with their
//                 strip (K4 and G1 pick their strip's pool records out
//                 of it); tall cells added to B by 16-thread teams at
//                 the block's end
//   k_strip_acc   one work item = (strip, chunk): LDS accumulate,     K4
//                 flush rho = D0 + tile (+B); the chunks of a split
//                 strip add into B and the last one to finish flushes
//   k_gather_bin  one work item = (strip, chunk): the strip's field   G1
//                 rows staged in LDS, each record's partial force over
//                 the rows of this strip, in record order
//   k_gather_out  forces back to cell order: sum of the (one or two)  G2
//                 partials, on the one-pass blocks; tall cells
//                 gathered by 16-thread teams (larger ones by the
//                 whole workgroup)
//
// Accumulation is fixed point everywhere: round(v * 2^f) added as uint64
// (LDS, the side map B), with f = fix_exponent_of(nc_max, dtype) so a bin's
// sum cannot overflow (each contribution is <= 1).  Integer sums are exact
// and independent of order, so the density -- and everything computed from
// it -- is bitwise reproducible run to run.  (On gfx950 ds_add_u64 also
// runs about seven times faster than ds_add_f32.)
//
// K3 evaluates each cell's stretch and span once, in float64, and stores a
// record: geometry in bin units relative to the edges of its first bin
// (offsets dx, dy of the stretched corner, in [0, 1), and the cell's
// original extents w, h, from which K4 and G1 re-derive the stretched
// extents and the area ratio) and its first row and column (16 bytes in
// one word at float32, rec_geo; a double4 plus a span word at float64).  Short
// arithmetic on small numbers, which float32 carries to ~1e-7 of a bin
// (absolute die coordinates would not).  K3 also writes pos[i] (both slots),
// the records of cell i (in cell order, coalesced), so G2 can write the
// forces in cell order instead of G1 scattering them.
//
// A cell whose span covers more than R rows or more than kMaxSpanY + 1
// columns ("tall") skips the sort: K3 adds it with global atomics into the
// side map B (zero between steps) and marks the column blocks it touches in
// each of its strips; K4 folds and re-zeroes those blocks of B, and G2
// gathers the cell with a team of threads.  Every other cell touches at most
// two strips, so the record arrays hold 2*nc_max.
#pragma once

#include <type_traits>

#include "dpep_internal.h"
#include "dpep_spectral.h"

namespace dpep {

template <typename T> struct vec4;
template <> struct vec4<float> { using type = float4; };
template <> struct vec4<double> { using type = double4; };
template <typename T> using vec4_t = typename vec4<T>::type;

// Span word of a record in strip s (first row k0 = s * R):
//   bits 0-3   bxl - k0, two's complement in [-7, 7] (negative for the copy
//              of a cell that starts in the strip before)
//   bits 4-6   nx = bxh - bxl (< R <= 8)
//   bits 7-18  ny = byh - byl (<= kMaxSpanY)
//   bits 19-31 byl (< 8192)
__device__ __forceinline__ unsigned span_word(int rel, int nx, int ny, int byl)
{
    return ((unsigned)rel & 0xFu) | ((unsigned)nx << 4) | ((unsigned)ny << 7) |
           ((unsigned)byl << 19);
}

struct SpanBox {
    int bxl, nx, byl, ny;
};

__device__ __forceinline__ SpanBox span_of(unsigned m, int k0)
{
    SpanBox b;
    b.bxl = k0 + (((int)(m << 28)) >> 28);
    b.nx = (int)((m >> 4) & 7u);
    b.ny = (int)((m >> 7) & 0xFFFu);
    b.byl = (int)(m >> 19);
    return b;
}

// Stretched extents and area ratio from a record's original extents.
template <typename T>
__device__ __forceinline__ void stretch_of(const vec4_t<T>& r, int stretch, T& xr,
                                           T& yr, T& ratio)
{
    T wc = r.z, hc = r.w;
    ratio = (T)1;
    if (stretch) {
        const T m = (T)1.41421356237309504880;
        wc = r.z > m ? r.z : m;
        hc = r.w > m ? r.w : m;
        ratio = (r.z * r.w) * fast_rcp(wc * hc);
    }
    xr = r.x + wc;
    yr = r.y + hc;
}

// ---------------------------------------------------------------------------
// Stored records.  float64: the geometry (dx, dy, w, h) as a double4 in recg
// and the span word in recm.  float32: one 16-byte word per record in recg
// (recm unused).  dx and dy, the offsets of the stretched corner from its
// first bin's edges, are kept as the 23-bit mantissas of the floats 1 + dx
// and 1 + dy, whose sign and exponent bits are always the same and so carry
// the rest: the row offset rel (4 bits) and byl (13 bits, 5 in the dx word
// and 8 in the dy word); w and h are plain float32.  An offset is in [0, 1)
// except where the stretch moves a cell's corner past the die's lower edge
// (its first bin clamped to 0), in [-1, 0) then: along x the record starts
// one row earlier (rel - 1, at row -1, which every row loop clamps away) with
// dx + 1; along y it keeps dy + 1 and sets bit 31 of the dy word, and the
// decode subtracts 2 instead of 1.  Decoding an offset is an AND-OR and a
// subtraction (precision 2^-23 of a bin); the row and column counts are
// derived from the geometry (rec_view).  One aligned 16-byte store per record
// in K3 and one load in K4 and G1, where the 20-byte form took two of each
// into two arrays.  A cell whose corner lies more than a bin below the lower
// edge (placed outside the die) takes the tall path instead (cell_strips).
// ---------------------------------------------------------------------------
constexpr unsigned kOffMant = 0x007FFFFFu;     // mantissa bits of 1 + offset
constexpr unsigned kOne = 0x3F800000u;         // the bits of 1.0f
constexpr unsigned kSign = 0x80000000u;

// rel: the first row's offset in the cell's first strip, in [0, R).  A cell
// whose stretched corner is below the lower x edge starts at row 0 (rel 0)
// and spans one strip only (a cell spanning more than R rows is tall).
template <typename T>
__device__ __forceinline__ vec4_t<T> rec_geo(double ex, double ey, double wb, double hb, int byl,
                                             int rel)
{
    if constexpr (sizeof(T) == 4) {
        auto mant = [](double e) -> unsigned {
            const double v = e * 8388608.0 + 0.5;
            return v <= 0.0 ? 0u : (v >= 8388607.0 ? kOffMant : (unsigned)v);
        };
        const unsigned ub = (unsigned)byl;
        const bool lx = ex < 0.0, ly = ey < 0.0;
        float4 r;
        r.x = __uint_as_float(mant(lx ? ex + 1.0 : ex) | (((unsigned)(rel - lx) & 0xFu) << 23) |
                              ((ub & 0x1Fu) << 27));
        r.y = __uint_as_float(mant(ly ? ey + 1.0 : ey) | (((ub >> 5) & 0xFFu) << 23) |
                              (ly ? kSign : 0u));
        r.z = (float)wb;
        r.w = (float)hb;
        return r;
    } else {
        return vec4_t<T>{(T)ex, (T)ey, (T)wb, (T)hb};
    }
}

// The per-record part of a record in strip s (rel = bxl - s * R): the span
// word (float64), or at float32 whether s is the cell's second strip (the
// geometry word carries the first strip's rel, in [0, R), and the second
// strip's is R less: the same 4-bit field plus 16 - R, no carry), a constant
// at every call, so K3 keeps nothing per record for it.
template <typename T>
__device__ __forceinline__ unsigned rec_span(int rel, int nx, int ny, int byl, bool second)
{
    if constexpr (sizeof(T) == 4) return second ? 1u : 0u;
    else return span_word(rel, nx, ny, byl);
}

template <typename T>
__device__ __forceinline__ void rec_put(const BinArgs& b, vec4_t<T>* recg, unsigned p,
                                        const vec4_t<T>& geo, unsigned m)
{
    if constexpr (sizeof(T) == 4) {
        float4 r = geo;
        if (m) r.x = __uint_as_float(__float_as_uint(r.x) + ((16u - (unsigned)b.R) << 23));
        recg[p] = r;
    } else {
        recg[p] = geo;
        b.recm[p] = m;
    }
}

// The span word of record r (float64; float32 records carry it in recg).
template <typename T>
__device__ __forceinline__ unsigned rec_m(const BinArgs& b, unsigned r)
{
    if constexpr (sizeof(T) == 4) return 0u;
    else return b.recm[r];
}

// A record in the frame of its strip (first row k0): offsets dx, dy, far
// edges xr = dx + stretched w and yr, area ratio, first row and column,
// rows and columns past them (nx not clamped to the strip: callers clamp
// to their rows; ny clamped to the grid's N columns).
template <typename T>
struct RecView {
    T dx, dy, xr, yr, rat;
    int bxl, nx, byl, ny;
};

template <typename T>
__device__ __forceinline__ RecView<T> rec_view(const vec4_t<T>& rg, unsigned rm, int k0,
                                               int stretch, int N)
{
    RecView<T> v;
    if constexpr (sizeof(T) == 4) {
        const unsigned ux = __float_as_uint(rg.x), uy = __float_as_uint(rg.y);
        // 1 + offset minus 1; dy minus 2 where bit 31 of its word is set
        v.dx = __uint_as_float((ux & kOffMant) | kOne) - 1.f;
        v.dy = __uint_as_float((uy & kOffMant) | kOne) - __uint_as_float(kOne + ((uy >> 31) << 23));
        v.bxl = k0 + (((int)(ux << 5)) >> 28);
        v.byl = (int)((ux >> 27) | (((uy >> 23) & 0xFFu) << 5));
        const float w = rg.z, h = rg.w;
        float wc = w, hc = h;
        v.rat = 1.f;
        if (stretch) {
            const float m = 1.41421356237309504880f;
            wc = w > m ? w : m;
            hc = h > m ? h : m;
            v.rat = (w * h) * fast_rcp(wc * hc);
        }
        v.xr = v.dx + wc;
        v.yr = v.dy + hc;
        // a row or column past the cell's far edge adds nothing (its overlap
        // is not positive), so counting from the rounded edge is safe
        v.nx = (int)v.xr;
        v.ny = min((int)v.yr, N - 1 - v.byl);
    } else {
        const SpanBox sb = span_of(rm, k0);
        stretch_of<T>(rg, stretch, v.xr, v.yr, v.rat);
        v.dx = rg.x;
        v.dy = rg.y;
        v.bxl = sb.bxl;
        v.nx = sb.nx;
        v.byl = sb.byl;
        v.ny = sb.ny;
    }
    return v;
}

constexpr unsigned kPosTall = 0xFFFFFFFFu;     // record slot: tall cell (side map)
constexpr unsigned kPosNone = 0xFFFFFFFEu;     // record slot: none

// Columns of the side map B that hold a strip's tall-cell sums: a bitmap of
// kSideBits column blocks of side_block(N) columns (kSideWords words per
// strip), so K4 folds and re-zeroes only the blocks its tall cells touch.
__host__ __device__ constexpr int side_block(int N)
{
    return N / kSideBits > 16 ? N / kSideBits : 16;
}

// Sets the bits of column blocks [c0 / CB, c1 / CB] in one strip's words:
// one atomicOr per word the range overlaps.
__device__ __forceinline__ void side_mark(unsigned* __restrict__ words, int c0, int c1, int CB)
{
    const int b0 = c0 / CB, b1 = c1 / CB;
    for (int w = b0 >> 5; w <= (b1 >> 5); ++w) {
        const int lo = max(b0 - (w << 5), 0), hi = min(b1 - (w << 5), 31);
        const unsigned m = (hi == 31 ? 0xFFFFFFFFu : ((1u << (hi + 1)) - 1u)) & ~((1u << lo) - 1u);
        atomicOr(&words[w], m);
    }
}

// pos[i]: the records of cell i in its first and second strip, one word
__device__ __forceinline__ unsigned long long pos_pair(unsigned p0, unsigned p1)
{
    return (unsigned long long)p0 | ((unsigned long long)p1 << 32);
}

// Strips [s0, s1] a cell occupies and whether it takes the tall path: more
// rows than a strip, more than kMaxSpanY + 1 columns, or (float32 records,
// which hold non-negative offsets only) a stretched corner below the die's
// lower x or y edge.
template <typename T>
__device__ __forceinline__ void cell_strips(const CellSpan& c, const Grid& g, int R, int lgR,
                                            int& s0, int& s1, bool& tall)
{
    tall = (c.bxh - c.bxl + 1) > R || (c.byh - c.byl) > kMaxSpanY;
    // a float32 record holds offsets down to -1 bin (rec_geo)
    if constexpr (sizeof(T) == 4) tall = tall || c.x < g.xl - g.bsx || c.y < g.yl - g.bsy;
    s0 = c.bxl >> lgR;
    s1 = c.bxh >> lgR;
}

template <typename T>
__device__ __forceinline__ bool load_span(const T* px, const T* py,
                                          const T* sx, const T* sy, int i,
                                          const Grid& g, CellSpan& c)
{
    return cell_span((double)px[i], (double)py[i], (double)sx[i],
                     (double)sy[i], g, c);
}

// The CPT cells of thread tid in the block of NT * CPT cells starting at c0
// (zero past nc).  A full block loads unconditionally: with a branch per
// cell the compiler moves each float32 -> float64 conversion into the branch
// and waits there for the load, so the cells' loads no longer overlap.
template <typename T, int NT = kBinThreads, int CPT = kCellsPerThread>
__device__ __forceinline__ void load_cells(const T* __restrict__ px, const T* __restrict__ py,
                                           const T* __restrict__ sx, const T* __restrict__ sy,
                                           int nc, int c0, int tid, T* cx, T* cy, T* cw, T* ch)
{
    if (c0 + NT * CPT <= nc) {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int i = c0 + tid + j * NT;
            cx[j] = px[i];
            cy[j] = py[i];
            cw[j] = sx[i];
            ch[j] = sy[i];
        }
    } else {
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int i = c0 + tid + j * NT;
            const bool ok = i < nc;
            cx[j] = ok ? px[i] : (T)0;
            cy[j] = ok ? py[i] : (T)0;
            cw[j] = ok ? sx[i] : (T)0;
            ch[j] = ok ? sy[i] : (T)0;
        }
    }
}

// The cells [c0, cend) of counting workgroup blockIdx.x (K1, the fresh K3:
// part blockIdx.x % b.sub of one-pass block blockIdx.x / b.sub, see
// set_count_blocks) and its count slot, the one-pass block's.
__device__ __forceinline__ int count_cells(const BinArgs& b, int nc, int& c0, int& cend)
{
    const int ob = (int)blockIdx.x / b.sub, part = (int)blockIdx.x - ob * b.sub;
    const int base = ob * b.qcells;
    c0 = base + part * b.qsub;
    cend = min(min(c0 + b.qsub, base + b.qcells), nc);
    if (cend < c0) cend = c0;
    return ob & (kCountSlots - 1);
}

// The CPT cells of thread tid in the one-pass block [c0, cend) (slots past
// cend hold copies of cell cend - 1, which the caller skips).  Every load is
// unconditional (clamped index), so no per-cell branch holds the loads back.
// An empty block (a step of no cells, whose cell pointers may be null) reads
// the word at `spare` (any valid device address) instead, for cells the
// caller skips all the same; choosing the pointers, not the loads, keeps the
// values in registers (a branch around the loads made the compiler keep some
// of them in scratch memory).
template <typename T, int NT, int CPT>
__device__ __forceinline__ void load_block_cells(const T* __restrict__ px,
                                                 const T* __restrict__ py,
                                                 const T* __restrict__ sx,
                                                 const T* __restrict__ sy, int c0, int cend,
                                                 int tid, const void* spare, T* cx, T* cy,
                                                 T* cw, T* ch)
{
    const bool any = cend > c0;
    const T* qx = any ? px : static_cast<const T*>(spare);
    const T* qy = any ? py : static_cast<const T*>(spare);
    const T* qw = any ? sx : static_cast<const T*>(spare);
    const T* qh = any ? sy : static_cast<const T*>(spare);
    const int last = any ? cend - 1 : 0;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int i = min(c0 + tid + j * NT, last);
        cx[j] = qx[i];
        cy[j] = qy[i];
        cw[j] = qw[i];
        ch[j] = qh[i];
    }
}

__device__ __forceinline__ unsigned long long to_fixed(double v, double scale)
{
    return (unsigned long long)__double2ull_rn(v * scale);
}

// float32 contributions: the scale is 2^31 (fix_exponent_of), v <= 1, so
// v * scale is exact and below 2^32: a 32-bit round-to-nearest conversion.
__device__ __forceinline__ unsigned long long to_fixed(float v, float scale)
{
    return (unsigned long long)__float2uint_rn(v * scale);
}

// The same conversions of a value already scaled.
__device__ __forceinline__ unsigned long long to_fixed(double v)
{
    return (unsigned long long)__double2ull_rn(v);
}

__device__ __forceinline__ unsigned long long to_fixed(float v)
{
    return (unsigned long long)__float2uint_rn(v);
}

// ---------------------------------------------------------------------------
// The plan: regions of the (slot, strip) pairs and the K4 / G1 work items.
// ---------------------------------------------------------------------------
// Exclusive prefix sum of one value per thread over the NT threads of a
// workgroup: a shuffle scan within each wave, then the waves' totals through
// LDS (two barriers; a Hillis-Steele scan in LDS took sixteen).
// tmp: NT / 64 words.
constexpr int kWave = 64;

template <int NT = kBinThreads>
__device__ __forceinline__ unsigned block_exclusive_scan(unsigned v,
                                                         unsigned* tmp,
                                                         unsigned& total)
{
    constexpr int kBinWaves = NT / kWave;
    const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
    unsigned x = v;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const unsigned y = __shfl_up(x, (unsigned)o, kWave);
        if (lane >= o) x += y;
    }
    if (lane == kWave - 1) tmp[wv] = x;
    __syncthreads();
    unsigned before = 0u, all = 0u;
#pragma unroll
    for (int k = 0; k < kBinWaves; ++k) {
        const unsigned t = tmp[k];
        before += k < wv ? t : 0u;
        all += t;
    }
    total = all;
    __syncthreads();
    return before + x - v;
}

// The (slot, strip) counts of the step of parity par: [kCountSlots][S].
__device__ __forceinline__ unsigned* counts_of(const BinArgs& b, int par)
{
    return b.xtot + (size_t)(par & 1) * kCountSlots * b.S;
}

// Chunk sizes and the K4 / G1 work items from the strip totals tot[S] (LDS,
// the totals the plan expects), by one workgroup of NT threads; thread tid
// owns strips [r0, r1).  The chunk size of a list is the smallest
// kChunkMin << k whose item count sum_s max(1, ceil(t_s / chunk)) fits the
// workgroups the device holds at once (Pacc for K4, Pgat for G1), so a
// skewed placement spreads its heavy strips over otherwise idle CUs; every
// strip in one item when even the largest does not fit.  An item is
// {strip | chunk << 16, first, end strip-relative record, chunks of the
// strip}; the last chunk of a strip runs to the strip's actual end.
// LDS: tmp[NT + kChunkCands].
template <int NT = kBinThreads>
__device__ __forceinline__ void publish_items(const BinArgs& b, const unsigned* tot,
                                              unsigned* tmp, int r0, int r1)
{
    constexpr int kBinWaves = NT / kWave;
    const int tid = threadIdx.x, lane = tid % kWave, wv = tid / kWave;
    int lg_min = 0;
    while ((1 << lg_min) < kChunkMin) ++lg_min;
    // item counts of every candidate: wave wv counts candidates wv,
    // wv + kBinWaves, ... over all strips (its lanes split them; tot[] is
    // complete: the caller's scan has passed a barrier since it was
    // written), the reductions of a wave's candidates interleaved so their
    // shuffle latencies overlap; one barrier
    unsigned* cand = tmp;                       // [kChunkCands]
    constexpr int KPW = (kChunkCands + kBinWaves - 1) / kBinWaves;
    unsigned c[KPW];
#pragma unroll
    for (int q = 0; q < KPW; ++q) c[q] = 0u;
    for (int s = lane; s < b.S; s += kWave) {
        const unsigned t = tot[s];
#pragma unroll
        for (int q = 0; q < KPW; ++q) {
            const unsigned sh = (unsigned)(lg_min + wv + q * kBinWaves);
            const unsigned n = sh < 32u ? (t + ((1u << sh) - 1u)) >> sh : 1u;
            c[q] += n > 1u ? n : 1u;
        }
    }
#pragma unroll
    for (int o = kWave / 2; o > 0; o >>= 1) {
#pragma unroll
        for (int q = 0; q < KPW; ++q) c[q] += __shfl_xor(c[q], o, kWave);
    }
    if (lane == 0) {
#pragma unroll
        for (int q = 0; q < KPW; ++q) {
            const int k = wv + q * kBinWaves;
            if (k < kChunkCands) cand[k] = c[q];
        }
    }
    __syncthreads();
    auto pick = [&](int P) -> unsigned {
        if (b.ch_force > 0) return (unsigned)b.ch_force;
        for (int k = 0; k < kChunkCands; ++k)
            if (cand[k] <= (unsigned)P) return (unsigned)kChunkMin << k;
        return (unsigned)kChunkMin << (kChunkCands - 1);
    };
    // K4 splits no strip into chunks below kAccChunkMin records: a split
    // chunk pays device-scope atomics for its whole tile and the strip's
    // flush waits for the last chunk, which only the accumulation of large
    // strips repays (uniform 512^2 grids measured slower split).  G1's
    // chunks are independent and split down to the candidate size.
    unsigned cha = pick(b.Pacc);
    if (b.ch_force <= 0 && cha < (unsigned)kAccChunkMin) cha = (unsigned)kAccChunkMin;
    const unsigned chg = pick(b.Pgat);
    __syncthreads();                            // cand (tmp) is read: free again
    if (tid == 0) {
        b.chunk[0] = cha;
        b.chunk[1] = chg;
    }
    for (int list = 0; list < 2; ++list) {
        const unsigned ch = list == 0 ? cha : chg;
        uint4* items = list == 0 ? b.items : b.items_g;
        const unsigned W = (unsigned)(list == 0 ? b.Wacc : b.Wgat);
        unsigned nrun = 0u;
        for (int s = r0; s < r1; ++s) {
            const unsigned n = (tot[s] + ch - 1u) / ch;
            nrun += n > 1u ? n : 1u;
        }
        unsigned ntotal;
        unsigned ibase = block_exclusive_scan<NT>(nrun, tmp, ntotal);
        for (int s = r0; s < r1; ++s) {
            const unsigned t = tot[s];
            unsigned n = (t + ch - 1u) / ch;
            n = n > 1u ? n : 1u;
            for (unsigned c = 0; c < n; ++c)
                if (ibase + c < W)
                    items[ibase + c] = uint4{(unsigned)s | (c << 16), c * ch,
                                             min((c + 1u) * ch, t), n};
            ibase += n;
        }
        if (tid == 0) b.nitems[list] = ntotal < W ? ntotal : W;
    }
}

// Fresh plan, in K3 after K1: offsets of this workgroup's strip entries
// from K1's slot totals.  Every workgroup scans the totals itself (S values,
// a few microseconds of L2 reads spread over the grid) instead of one
// workgroup building a table behind all of K1.  The regions of a strip are
// its slots' totals back to back, exactly: cur[s] = strip offset + totals
// of the slots before g's + g's base within its slot.  Workgroup 0 also
// publishes the plan for K4 / G1.  LDS: cur[S] | tot[S] | tmp[kBinThreads]
// | cand[kChunkCands].
__device__ __forceinline__ void fresh_offsets(const BinArgs& b, unsigned* cur,
                                              unsigned* tot, unsigned* tmp)
{
    const int tid = threadIdx.x;
    const int S = b.S;
    int c0, cend;
    const int x = count_cells(b, 0, c0, cend);
    const unsigned* row = b.cnt + (size_t)blockIdx.x * S;
    const unsigned* xt = counts_of(b, b.par);
    for (int s = tid; s < S; s += kBinThreads) {
        unsigned t = 0u, pre = 0u;
#pragma unroll
        for (int xx = 0; xx < kCountSlots; ++xx) {
            const unsigned v = xt[(size_t)xx * S + s];
            pre += xx < x ? v : 0u;
            t += v;
        }
        tot[s] = t;
        cur[s] = pre + row[s];
    }
    __syncthreads();
    // exclusive scan of the strip totals (each thread a run of strips)
    const int per = (S + kBinThreads - 1) / kBinThreads;
    const int r0 = min(tid * per, S), r1 = min(r0 + per, S);
    unsigned run = 0u;
    for (int s = r0; s < r1; ++s) run += tot[s];
    unsigned total;
    unsigned base = block_exclusive_scan(run, tmp, total);
    const bool pub = blockIdx.x == 0;         // uniform across the group
    for (int s = r0; s < r1; ++s) {
        cur[s] += base;
        if (pub) {
            unsigned o = base;
#pragma unroll
            for (int xx = 0; xx < kCountSlots; ++xx) {
                const unsigned v = xt[(size_t)xx * S + s];
                b.pbase[(size_t)xx * S + s] = o;
                b.pcap[(size_t)xx * S + s] = v;
                o += v;
            }
        }
        base += tot[s];
    }
    if (pub) publish_items(b, tot, tmp, r0, r1);
}

// Capacity a one-pass step gives a region that counted d records in the
// step before.
__device__ __forceinline__ unsigned region_cap(unsigned d, int tight)
{
    return tight ? d / 2u : d + d / 8u + kRegionSlack;
}

// One-pass plan, in K3 without K1: the regions of this step from the
// previous step's counts (the other parity's set), each its count plus
// slack, strip after strip and slot after slot (they fit b.reg_cap:
// region_capacity).  start[s], room[s]: the region of this workgroup's slot
// in strip s.  Workgroup 0 also publishes the plan for K4 / G1: the regions
// and the work items, chunked by the expected strip totals.  NT threads.
// LDS: start[S] | room[S] | tot[S] | tmp[NT + kChunkCands].
template <int NT>
__device__ __forceinline__ void once_offsets(const BinArgs& b, unsigned* start,
                                             unsigned* room, unsigned* tot, unsigned* tmp)
{
    const int tid = threadIdx.x;
    const int S = b.S;
    const int x = (int)blockIdx.x & (kCountSlots - 1);     // block b: slot b % 8
    const unsigned* prev = counts_of(b, b.par ^ 1);
    const int per = (S + NT - 1) / NT;
    const int r0 = min(tid * per, S), r1 = min(r0 + per, S);
    unsigned run = 0u;
    for (int s = r0; s < r1; ++s) {
        unsigned t = 0u;
#pragma unroll
        for (int xx = 0; xx < kCountSlots; ++xx) {
            const unsigned d = prev[(size_t)xx * S + s];
            t += d;
            run += region_cap(d, b.tight);
        }
        tot[s] = t;
    }
    unsigned total;
    unsigned base = block_exclusive_scan<NT>(run, tmp, total);
    const bool pub = blockIdx.x == 0;         // uniform across the group
    for (int s = r0; s < r1; ++s) {
#pragma unroll
        for (int xx = 0; xx < kCountSlots; ++xx) {
            const size_t q = (size_t)xx * S + s;
            const unsigned c = region_cap(prev[q], b.tight);
            if (xx == x) {
                start[s] = base;
                room[s] = c;
            }
            if (pub) {
                b.pbase[q] = base;
                b.pcap[q] = c;
            }
            base += c;
        }
    }
    if (pub) publish_items<NT>(b, tot, tmp, r0, r1);
}

// A strip's records by strip-relative number: region after region (slot
// order), min(counted, capacity) records each.  Number v of region j sits
// at record slot v + D[j], D[j] = E[0] + ... + E[j]; P[j] is the region's
// first number.  (Written out for the 8 regions, and as a sum of steps
// rather than a choice among the D[j]: either of the plainer forms leaves
// the map in scratch memory.)
static_assert(kCountSlots == 8, "strip_map / map_record are written for 8 regions");
struct StripMap {
    unsigned P[kCountSlots];
    unsigned E[kCountSlots];
    unsigned n;                 // records of the strip in its regions
};

__device__ __forceinline__ void strip_map(const BinArgs& b, int s, StripMap& m)
{
    const unsigned* xt = counts_of(b, b.par);
    unsigned p = 0u, dprev = 0u;
    auto region = [&](int xx, unsigned& P, unsigned& E) {
        const size_t q = (size_t)xx * b.S + s;
        const unsigned c = xt[q], cap = b.pcap[q];
        const unsigned d = b.pbase[q] - p;
        P = p;
        E = d - dprev;
        dprev = d;
        p += c < cap ? c : cap;
    };
    region(0, m.P[0], m.E[0]);
    region(1, m.P[1], m.E[1]);
    region(2, m.P[2], m.E[2]);
    region(3, m.P[3], m.E[3]);
    region(4, m.P[4], m.E[4]);
    region(5, m.P[5], m.E[5]);
    region(6, m.P[6], m.E[6]);
    region(7, m.P[7], m.E[7]);
    m.n = p;
}

__device__ __forceinline__ unsigned map_record(const StripMap& m, unsigned v)
{
    unsigned r = v + m.E[0];
    r += v >= m.P[1] ? m.E[1] : 0u;
    r += v >= m.P[2] ? m.E[2] : 0u;
    r += v >= m.P[3] ? m.E[3] : 0u;
    r += v >= m.P[4] ? m.E[4] : 0u;
    r += v >= m.P[5] ? m.E[5] : 0u;
    r += v >= m.P[6] ? m.E[6] : 0u;
    r += v >= m.P[7] ? m.E[7] : 0u;
    return r;
}

// The strip-relative records [e0, e1) of work item it, clamped to what the
// strip holds this step (the last chunk takes everything past its start).
__device__ __forceinline__ void item_range(const uint4& it, const StripMap& m,
                                           unsigned& e0, unsigned& e1)
{
    const unsigned c = it.x >> 16, n = it.w;
    e0 = it.y < m.n ? it.y : m.n;
    e1 = c + 1u == n ? m.n : (it.z < m.n ? it.z : m.n);
    if (e1 < e0) e1 = e0;
}

// The per-strip overflow state of the step of parity par: [S] of
// (runs << 32) | records.
__device__ __forceinline__ unsigned long long* overflow_state(const BinArgs& b, int par)
{
    return b.ovst + (size_t)(par & 1) * b.S;
}

// Runs of a strip's overflow list that K4 and G1 stage in LDS at once.
constexpr int kRunBatch = 1024;

// fn(r) for every overflow-pool record r of strip s, by the kAccThreads
// threads of the strip's first work item (chunk 0; the strip's other chunks
// call nothing; every thread of the workgroup must call it).  The strip's
// overflow list is the records a one-pass step found no room for in the
// strip's regions: one run per K3 block that overflowed there, numbered in
// the order of the runs' atomics, each run contiguous in the pool.  The run
// table goes to LDS (lrun[kRunBatch], kRunBatch runs at a time) and each
// thread takes records e = tid, tid + kAccThreads, ... of the list, finding
// its run by a binary search of the runs' first numbers: every thread busy,
// whatever the runs' lengths.  Empty on a counted step and on a placement
// like the previous step's.
// The step's pool count is read first, after the strip's own records: one
// word every workgroup reads (an L2 hit after the first), zero unless the
// step overflowed; only then the strip's overflow_state entry.  (Each
// workgroup reading its strip's entry on every step, an address K3's
// device-scope atomics leave outside the L2, cost G1 1.3 us at 2M cells on
// 4096 x 4096; loaded with the work item and held across the record loop,
// 9 us; a flag derived from the strip map instead, 8 us: it changed how the
// compiler schedules G1's first loads.)
template <typename Fn>
__device__ __forceinline__ void for_overflow_records(const BinArgs& b, int s, const uint4& item,
                                                     int tid, uint2* lrun, Fn&& fn)
{
    if (b.pool_n[b.par & 1] == 0u || (item.x >> 16) != 0u) return;   // uniform
    const unsigned long long st = overflow_state(b, b.par)[s];
    const unsigned nr = (unsigned)(st >> 32), tot = (unsigned)st;
    if (tot == 0u) return;                              // uniform across the group
    const unsigned nrun = nr < (unsigned)b.rmax ? nr : (unsigned)b.rmax;
    const uint2* runs = b.oruns + (size_t)s * b.rmax;
    for (unsigned k0 = 0; k0 < nrun; k0 += kRunBatch) {
        const unsigned nb = min(nrun - k0, (unsigned)kRunBatch);
        __syncthreads();                        // the previous batch is read
        for (unsigned k = (unsigned)tid; k < nb; k += kAccThreads) lrun[k] = runs[k0 + k];
        __syncthreads();
        const unsigned v0 = lrun[0].y;
        const unsigned v1 = k0 + nb < nrun ? runs[k0 + nb].y : tot;
        for (unsigned e = v0 + (unsigned)tid; e < v1; e += kAccThreads) {
            unsigned lo = 0u, hi = nb - 1u;     // the last run starting at or before e
            while (lo < hi) {
                const unsigned mid = (lo + hi + 1u) >> 1;
                if (lrun[mid].y <= e) lo = mid;
                else hi = mid - 1u;
            }
            fn(b.pool0 + lrun[lo].x + (e - lrun[lo].y));
        }
    }
}

// ---------------------------------------------------------------------------
// K1: per-workgroup strip histogram, added into the slot totals.
// LDS: hist[S].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBinThreads) void k_bin_count(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b)
{
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned* hist = reinterpret_cast<unsigned*>(smem);
    const int tid = threadIdx.x;
    for (int s = tid; s < b.S; s += kBinThreads) hist[s] = 0u;
    __syncthreads();
    int c0, cend;
    const int x = count_cells(b, nc, c0, cend);
    // all loads of this thread's cells first (independent, in flight together)
    T cx[kCellsPerThread], cy[kCellsPerThread], cw[kCellsPerThread], ch[kCellsPerThread];
    load_cells(px, py, sx, sy, cend, c0, tid, cx, cy, cw, ch);
#pragma unroll
    for (int j = 0; j < kCellsPerThread; ++j) {
        CellSpan c;
        if (!cell_span((double)cx[j], (double)cy[j], (double)cw[j], (double)ch[j], g, c))
            continue;
        int s0, s1;
        bool tall;
        cell_strips<T>(c, g, b.R, b.lgR, s0, s1, tall);
        if (tall) continue;
        atomicAdd(&hist[s0], 1u);
        if (s1 != s0) atomicAdd(&hist[s1], 1u);
    }
    __syncthreads();
    // the block adds into its count slot: a label only, it spreads the
    // atomics over kCountSlots addresses per strip; the returned old total is
    // the block's base within its slot
    unsigned* row = b.cnt + (size_t)blockIdx.x * b.S;
    unsigned* slot = counts_of(b, b.par) + (size_t)x * b.S;
    for (int s = tid; s < b.S; s += kBinThreads) {
        const unsigned h = hist[s];
        row[s] = h ? atomicAdd(&slot[s], h) : 0u;
    }
}

// ---------------------------------------------------------------------------
// K3: fill the strip-sorted records; tall cells go to B; pos[i] for G2.
// Two forms.  This one stores each record straight to its slot (one 16- and
// one 4-byte store per record): at a few hundred strips a workgroup's run in
// a strip holds several records and the L2 merges the runs' partial lines;
// it needs no staging LDS, so every workgroup is resident at once.
// LDS: cur[S] | tot[S] | tmp[kBinThreads] | cand[kChunkCands].
// ---------------------------------------------------------------------------
template <typename T>
__global__ __launch_bounds__(kBinThreads) void k_bin_fill_direct(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b)
{
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned* cur = reinterpret_cast<unsigned*>(smem);
    const int tid = threadIdx.x;
    // the cells' loads are issued first: their latency overlaps the offsets
    int c0, cend;
    count_cells(b, nc, c0, cend);
    T cx[kCellsPerThread], cy[kCellsPerThread], cw[kCellsPerThread], chh[kCellsPerThread];
    load_cells(px, py, sx, sy, cend, c0, tid, cx, cy, cw, chh);
    fresh_offsets(b, cur, cur + b.S, cur + 2 * b.S);
    __syncthreads();
    vec4_t<T>* recg = reinterpret_cast<vec4_t<T>*>(b.recg);
    unsigned long long* Bm = reinterpret_cast<unsigned long long*>(b.B);
    for (int j = 0; j < kCellsPerThread; ++j) {
        const int i = c0 + tid + j * kBinThreads;
        if (i >= cend) break;
        CellSpan c;
        if (!cell_span((double)cx[j], (double)cy[j], (double)cw[j], (double)chh[j], g, c)) {
            b.pos[i] = pos_pair(kPosNone, kPosNone);
            continue;
        }
        int s0, s1;
        bool tall;
        cell_strips<T>(c, g, b.R, b.lgR, s0, s1, tall);
        if (tall) {
            const double sc = c.ratio() * g.inv_ba;
            for (int k = c.bxl; k <= c.bxh; ++k) {
                const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
                if (tx <= 0.0) continue;
                const double stx = sc * tx;
                const size_t rowi = (size_t)k * g.N;
                for (int q = c.byl; q <= c.byh; ++q) {
                    const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
                    if (ty <= 0.0) continue;
                    atomicAdd(&Bm[rowi + q], to_fixed(stx * ty, g.fix_scale));
                }
            }
            // the column blocks of B this cell touches, in each of its strips
            const int CB = side_block(g.N);
            for (int s = s0; s <= s1; ++s)
                side_mark(b.bigflag + (size_t)s * kSideWords, c.byl, c.byh, CB);
            b.pos[i] = pos_pair(kPosTall, kPosNone);
            continue;
        }
        // strip-relative record, evaluated in float64 and rounded once
        const double ex = (c.x - (g.xl + c.bxl * g.bsx)) * g.inv_bsx;
        const double ey = (c.y - (g.yl + c.byl * g.bsy)) * g.inv_bsy;
        const vec4_t<T> geo = rec_geo<T>(ex, ey, (double)cw[j] * g.inv_bsx,
                                         (double)chh[j] * g.inv_bsy, c.byl, c.bxl - (s0 << b.lgR));
        const int nx = c.bxh - c.bxl, ny = c.byh - c.byl;
        const unsigned p0 = atomicAdd(&cur[s0], 1u);
        rec_put<T>(b, recg, p0, geo, rec_span<T>(c.bxl - (s0 << b.lgR), nx, ny, c.byl, false));
        unsigned p1 = kPosNone;
        if (s1 != s0) {
            p1 = atomicAdd(&cur[s1], 1u);
            rec_put<T>(b, recg, p1, geo, rec_span<T>(c.bxl - (s1 << b.lgR), nx, ny, c.byl, true));
        }
        b.pos[i] = pos_pair(p0, p1);
    }
}

// ---------------------------------------------------------------------------
// K3, staged form, for grids of many strips (a workgroup's run in a strip
// is then one or two records, and straight stores become one partial line
// each: 2.8x the record bytes written at 4096 x 4096).
// A workgroup's records of one strip occupy one run of the strip's range
// (its base from fresh_offsets).  They are ranked per strip (LDS atomics),
// staged in LDS in strip order (the block's counting sort) and copied out
// with consecutive threads on consecutive slots, so a wave's stores cover
// whole runs instead of one scattered store per record: the
// lines of a run are written whole, by one workgroup, at once.  A staged
// slot's strip is found again by a binary search of the strip offsets, so
// the stage holds only the records (geometry and per-record word, 20 bytes
// each at float32) and five
// workgroups fit a CU: one round at 1.1 M cells.  Records past kStage
// slots go straight to their place.
// LDS: cur[S] | cnt[S] | tmp[kBinThreads + kChunkCands] | off[S + 1] |
// staged geometry[kStage] | staged span words[kStage].
// ---------------------------------------------------------------------------
constexpr int kStage = 1344;   // about the records of a 1024-cell block (1.3 to
                               // 1.4 per cell), so five workgroups fit a CU

// The staged form from this many strips on: fewer strips give longer runs,
// whose straight stores the L2 already merges, and the stage's scans and
// LDS then cost more than they save (measured on MI355X: 64 strips
// +4.5 us, 256 strips even, 1024 strips -25 us).
constexpr int kStageMinStrips = 512;

template <typename T>
__host__ __device__ constexpr size_t fill_lds_staged(int S)
{
    return ((size_t)(3 * S + 1 + kBinThreads + kChunkCands) * sizeof(unsigned) + 15) / 16 * 16 +
           (size_t)kStage * (sizeof(vec4_t<T>) + sizeof(unsigned));
}

template <typename T>
__global__ __launch_bounds__(kBinThreads, 5) void k_bin_fill_staged(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int S = b.S;
    unsigned* cur = reinterpret_cast<unsigned*>(smem);
    unsigned* cnt = cur + S;              // strip totals, then this block's counts
    unsigned* tmp = cnt + S;
    unsigned* off = tmp + kBinThreads + kChunkCands;   // S + 1 entries
    vec4_t<T>* sg = reinterpret_cast<vec4_t<T>*>(
        smem + ((size_t)(3 * S + 1 + kBinThreads + kChunkCands) * sizeof(unsigned) + 15) / 16 *
                   16);
    unsigned* sm = reinterpret_cast<unsigned*>(sg + kStage);
    const int tid = threadIdx.x;
    // the cells' loads are issued first: their latency overlaps the offsets
    int c0, cend;
    count_cells(b, nc, c0, cend);
    T cx[kCellsPerThread], cy[kCellsPerThread], cw[kCellsPerThread], chh[kCellsPerThread];
    load_cells(px, py, sx, sy, cend, c0, tid, cx, cy, cw, chh);
    fresh_offsets(b, cur, cnt, tmp);
    __syncthreads();
    for (int s = tid; s < S; s += kBinThreads) cnt[s] = 0u;
    __syncthreads();
    vec4_t<T>* recg = reinterpret_cast<vec4_t<T>*>(b.recg);
    unsigned long long* Bm = reinterpret_cast<unsigned long long*>(b.B);
    // per cell: its record geometry, the per-record parts (rec_span), strips
    // and ranks in them
    vec4_t<T> geo[kCellsPerThread];
    unsigned m0[kCellsPerThread], m1[kCellsPerThread], r0[kCellsPerThread],
        r1[kCellsPerThread];
    int s0v[kCellsPerThread], s1v[kCellsPerThread];
#pragma unroll
    for (int j = 0; j < kCellsPerThread; ++j) {
        s0v[j] = s1v[j] = -1;
        const int i = c0 + tid + j * kBinThreads;
        if (i >= cend) continue;
        CellSpan c;
        if (!cell_span((double)cx[j], (double)cy[j], (double)cw[j], (double)chh[j], g, c)) {
            b.pos[i] = pos_pair(kPosNone, kPosNone);
            continue;
        }
        int s0, s1;
        bool tall;
        cell_strips<T>(c, g, b.R, b.lgR, s0, s1, tall);
        if (tall) {
            const double sc = c.ratio() * g.inv_ba;
            for (int k = c.bxl; k <= c.bxh; ++k) {
                const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
                if (tx <= 0.0) continue;
                const double stx = sc * tx;
                const size_t rowi = (size_t)k * g.N;
                for (int q = c.byl; q <= c.byh; ++q) {
                    const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
                    if (ty <= 0.0) continue;
                    atomicAdd(&Bm[rowi + q], to_fixed(stx * ty, g.fix_scale));
                }
            }
            // the column blocks of B this cell touches, in each of its strips
            const int CB = side_block(g.N);
            for (int s = s0; s <= s1; ++s)
                side_mark(b.bigflag + (size_t)s * kSideWords, c.byl, c.byh, CB);
            b.pos[i] = pos_pair(kPosTall, kPosNone);
            continue;
        }
        // strip-relative record, evaluated in float64 and rounded once
        const double ex = (c.x - (g.xl + c.bxl * g.bsx)) * g.inv_bsx;
        const double ey = (c.y - (g.yl + c.byl * g.bsy)) * g.inv_bsy;
        geo[j] = rec_geo<T>(ex, ey, (double)cw[j] * g.inv_bsx, (double)chh[j] * g.inv_bsy,
                            c.byl, c.bxl - (s0 << b.lgR));
        const int nx = c.bxh - c.bxl, ny = c.byh - c.byl;
        s0v[j] = s0;
        m0[j] = rec_span<T>(c.bxl - (s0 << b.lgR), nx, ny, c.byl, false);
        r0[j] = atomicAdd(&cnt[s0], 1u);
        if (s1 != s0) {
            s1v[j] = s1;
            m1[j] = rec_span<T>(c.bxl - (s1 << b.lgR), nx, ny, c.byl, true);
            r1[j] = atomicAdd(&cnt[s1], 1u);
        }
    }
    __syncthreads();
    // offsets of the strips' runs within the block: exclusive scan of cnt
    unsigned nrec;
    {
        const int per = (S + kBinThreads - 1) / kBinThreads;
        const int a0 = min(tid * per, S), a1 = min(a0 + per, S);
        unsigned run = 0u;
        for (int s = a0; s < a1; ++s) run += cnt[s];
        unsigned base = block_exclusive_scan(run, tmp, nrec);
        for (int s = a0; s < a1; ++s) {
            off[s] = base;
            base += cnt[s];
        }
        if (tid == 0) off[S] = nrec;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < kCellsPerThread; ++j) {
        if (s0v[j] < 0) continue;
        const int i = c0 + tid + j * kBinThreads;
        const unsigned k0 = off[s0v[j]] + r0[j], d0 = cur[s0v[j]] + r0[j];
        if (k0 < (unsigned)kStage) {
            sg[k0] = geo[j];
            sm[k0] = m0[j];
        } else {
            rec_put<T>(b, recg, d0, geo[j], m0[j]);
        }
        unsigned d1 = kPosNone;
        if (s1v[j] >= 0) {
            const unsigned k1 = off[s1v[j]] + r1[j];
            d1 = cur[s1v[j]] + r1[j];
            if (k1 < (unsigned)kStage) {
                sg[k1] = geo[j];
                sm[k1] = m1[j];
            } else {
                rec_put<T>(b, recg, d1, geo[j], m1[j]);
            }
        }
        b.pos[i] = pos_pair(d0, d1);
    }
    __syncthreads();
    // staged records out, consecutive threads on consecutive slots: slot k
    // belongs to the last strip s with off[s] <= k (empty strips share
    // their successor's offset and are passed over), at cur[s] + k - off[s]
    const unsigned ns = nrec < (unsigned)kStage ? nrec : (unsigned)kStage;
    int lg = 0;
    while ((1 << lg) < S + 1) ++lg;
    for (unsigned k = tid; k < ns; k += kBinThreads) {
        int lo = 0, hi = S;                   // off[lo] <= k < off[hi]
        for (int q = 0; q < lg; ++q) {
            const int mid = (lo + hi) >> 1;
            if (mid > lo && off[mid] <= k) lo = mid;
            else if (mid > lo) hi = mid;
        }
        const unsigned d = cur[lo] + (k - off[lo]);
        rec_put<T>(b, recg, d, sg[k], sm[k]);
    }
}

// One record's fixed-point contributions to the bins of rows [k0, k1] (its
// strip), added into K4's LDS tile (row - k0, column) at tile[(row - k0) * N
// + column] (for the strip's records and its overflow records alike).  The
// scale fs is a power of two, so folding it into the row's weight (rat * tx
// * fs, exact) rounds each value as (rat * tx * ty) * fs would; a row's
// address steps by N, its columns are immediate offsets from it, and its x
// overlap is formed as in record_partial (bitwise the same value).  The
// first Q columns' adds are unrolled (each under its own lane mask), Q = 4
// where a lane of the wave has a record spanning four or more columns and 3
// otherwise (float64: 4), as in G1.
template <typename T, int Q>
__device__ __forceinline__ void density_rows(const RecView<T>& rv, const T* tyv, int ka, int kb,
                                             int k0, int N, T fs, unsigned long long* tile)
{
    const T xr = rv.xr, yr = rv.yr, rat = rv.rat, dx = rv.dx, dy = rv.dy;
    unsigned long long* row = tile + (__umul24((unsigned)(ka - k0), (unsigned)N) + (unsigned)rv.byl);
    T jx = (T)(ka - rv.bxl);
    for (int k = ka; k <= kb; ++k, row += N, jx += (T)1) {
        const T tx = min(xr - jx, (T)1) - max(dx - jx, (T)0);
        if (!(tx > (T)0)) continue;
        const T rtxs = (rat * tx) * fs;
#pragma unroll
        for (int q = 0; q < Q; ++q)
            if (tyv[q] > (T)0) atomicAdd(row + q, to_fixed(rtxs * tyv[q]));
        for (int q = Q; q <= rv.ny; ++q) {
            const T ty = min(yr, (T)(q + 1)) - max(dy, (T)q);
            if (!(ty > (T)0)) continue;
            atomicAdd(row + q, to_fixed(rtxs * ty));
        }
    }
}

template <typename T>
__device__ __forceinline__ void record_density(const vec4_t<T>& rg, unsigned rm, int k0,
                                               int k1, int N, int stretch, T fs,
                                               unsigned long long* tile)
{
    const RecView<T> rv = rec_view<T>(rg, rm, k0, stretch, N);
    const int ka = max(rv.bxl, k0), kb = min(rv.bxl + rv.nx, k1);
    // y overlaps of the (usual) first 4 columns, shared by the rows; yr
    // clamped to the grid's last column edge gives the columns past it no
    // positive overlap and the others their own
    const T yrc = min(rv.yr, (T)(N - rv.byl));
    T tyv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) tyv[q] = min(yrc, (T)(q + 1)) - max(rv.dy, (T)q);
    if (sizeof(T) == 8 || __any(rv.ny >= 3))    // uniform (float64: Q = 4, as G1)
        density_rows<T, 4>(rv, tyv, ka, kb, k0, N, fs, tile);
    else
        density_rows<T, 3>(rv, tyv, ka, kb, k0, N, fs, tile);
}

// Threads per team that handles one tall cell (K3's side-map adds, G2's
// gather).
constexpr int kTallTeam = 16;

// A tall cell's density added into the side map B by a team of kTallTeam
// threads (lane: index in the team; every lane calls it for the same cell,
// its px, py, sx, sy): its bins strided over the team, each the value
// a single thread's row-by-row loop adds, (ratio / bin area * tx) * ty in
// fixed point, so the sums are bitwise the same in any order; the lanes
// also mark the cell's column blocks in each of its strips.  One thread per
// tall cell held its workgroup ~10 us for a cell of ~50 bins (float64).
template <typename T>
__device__ __forceinline__ void scatter_tall_team(const vec4_t<T>& cell, int lane,
                                                  const Grid& g, const BinArgs& b,
                                                  unsigned long long* __restrict__ Bm)
{
    CellSpan c;
    if (!cell_span((double)cell.x, (double)cell.y, (double)cell.z, (double)cell.w, g, c))
        return;
    int s0, s1;
    bool tall;
    cell_strips<T>(c, g, b.R, b.lgR, s0, s1, tall);
    const double sc = c.ratio() * g.inv_ba;
    const int ny1 = c.byh - c.byl + 1;
    const int nb = (c.bxh - c.bxl + 1) * ny1;
    for (int e = lane; e < nb; e += kTallTeam) {
        const int k = c.bxl + e / ny1, q = c.byl + e % ny1;
        const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
        const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
        if (tx <= 0.0 || ty <= 0.0) continue;
        const double stx = sc * tx;
        atomicAdd(&Bm[(size_t)k * g.N + q], to_fixed(stx * ty, g.fix_scale));
    }
    const int CB = side_block(g.N);
    for (int s = s0 + lane; s <= s1; s += kTallTeam)
        side_mark(b.bigflag + (size_t)s * kSideWords, c.byl, c.byh, CB);
}

// ---------------------------------------------------------------------------
// K3, single pass (no K1): the regions are sized from the previous step's
// counts (once_offsets).  Workgroup g ranks its records per strip in LDS,
// reserves one run per strip in region g % kCountSlots of the strip (one
// atomic per strip it touches: the total is the next step's count), and
// stores each record straight to its slot.  Records past the region's
// capacity -- a strip that gained more than the slack -- go to the overflow
// pool with their strip number; K4 adds them into the strip's LDS tile and
// G1 gathers them from the strip's rows in LDS like the strip's other
// records (for_overflow_records).  Every record is computed as in the fresh
// fill, and each one's partial force is summed in the same order of row
// groups, so the results do not depend on which records overflow.  (Adding
// an overflow record's bins into the side map B with device-scope atomics,
// as an earlier form did, cost 60 us at 1.1M cells when 3.5 % of the
// records overflowed: those atomics execute beyond the XCD's L2, and the
// overflow of a changed placement gathers on the strips that grew.)
// Tall cells are listed as they are found (their index; the coordinates of
// the first kTallList too) and added into B by teams of threads at the end
// (scatter_tall_team), where no per-cell registers are live.
// LDS: start[S] | room[S] | cnt[S] (the expected strip totals while the plan
// is made) | tmp[kOnceThreads + kChunkCands] | pool count, pool base | tall
// count | tall cells[kOnceThreads * kOnceMaxCpt] | (16-byte aligned) the
// first kTallList tall cells' px, py, sx, sy.
// ---------------------------------------------------------------------------
constexpr int kTallList = 256;

__host__ __device__ constexpr size_t fill_once_words(int S)
{
    return ((size_t)(3 * S + kOnceThreads + kChunkCands + 3 + kOnceThreads * kOnceMaxCpt) +
            3) / 4 * 4;
}

template <typename T>
__host__ __device__ constexpr size_t fill_once_lds(int S)
{
    return fill_once_words(S) * sizeof(unsigned) + (size_t)kTallList * sizeof(vec4_t<T>);
}

// NT = kOnceThreads threads, up to CPT cells each: one block of b.qcells
// cells (once_blocks: equal blocks, as many per CU as are resident, at
// least 1024 cells so a block's runs in a strip stay long and few
// reservation atomics land on each counter).  Six waves per SIMD where the
// registers allow it (float32 up to 4 cells per thread: three workgroups
// per CU), else four (two workgroups per CU).
template <typename T, int CPT>
__host__ __device__ constexpr int once_waves()
{
    return sizeof(T) == 4 && CPT <= 4 ? 6 : 4;
}

template <typename T, int CPT>
__global__ __launch_bounds__(kOnceThreads, (once_waves<T, CPT>())) void k_bin_fill_once(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int S = b.S;
    unsigned* start = reinterpret_cast<unsigned*>(smem);   // first slot of the run
    unsigned* room = start + S;                 // slots of the run in the region
    unsigned* cnt = room + S;                   // this block's records per strip
    unsigned* tmp = cnt + S;
    unsigned* npool = tmp + kOnceThreads + kChunkCands;  // [0] overflow, [1] pool base
    unsigned* ntall = npool + 2;
    unsigned* tall_idx = ntall + 1;             // [kOnceThreads * kOnceMaxCpt]
    vec4_t<T>* tall_cell =                      // [kTallList]
        reinterpret_cast<vec4_t<T>*>(smem + fill_once_words(S) * sizeof(unsigned));
    static_assert(CPT <= kOnceMaxCpt, "tall_idx holds kOnceMaxCpt cells per thread");
    const int tid = threadIdx.x;
    constexpr int NT = kOnceThreads;
    const int c0 = (int)blockIdx.x * b.qcells;
    const int cend = min(c0 + b.qcells, nc);
    unsigned* xrow = counts_of(b, b.par) + (size_t)(blockIdx.x & (kCountSlots - 1)) * S;
    // the cells' loads are issued first: their latency overlaps the plan
    T cx[CPT], cy[CPT], cw[CPT], chh[CPT];
    load_block_cells<T, NT, CPT>(px, py, sx, sy, c0, cend, tid, b.recg, cx, cy, cw, chh);
    once_offsets<NT>(b, start, room, cnt, tmp);
    __syncthreads();
    for (int s = tid; s < S; s += NT) cnt[s] = 0u;
    if (tid == 0) {
        npool[0] = 0u;
        *ntall = 0u;
    }
    __syncthreads();
    vec4_t<T>* recg = reinterpret_cast<vec4_t<T>*>(b.recg);
    unsigned long long* Bm = reinterpret_cast<unsigned long long*>(b.B);
    vec4_t<T> geo[CPT];
    unsigned m0[CPT], m1[CPT], r0[CPT],
        r1[CPT], p0[CPT], p1[CPT];
    int s0v[CPT], s1v[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        s0v[j] = s1v[j] = -1;
        p0[j] = p1[j] = kPosNone;
        const int i = c0 + tid + j * NT;
        if (i >= cend) continue;
        CellSpan c;
        if (!cell_span((double)cx[j], (double)cy[j], (double)cw[j], (double)chh[j], g, c))
            continue;
        int s0, s1;
        bool tall;
        cell_strips<T>(c, g, b.R, b.lgR, s0, s1, tall);
        if (tall) {
            const unsigned t = atomicAdd(ntall, 1u);
            tall_idx[t] = (unsigned)i;
            if (t < (unsigned)kTallList) tall_cell[t] = vec4_t<T>{cx[j], cy[j], cw[j], chh[j]};
            p0[j] = kPosTall;
            continue;
        }
        // strip-relative record, evaluated in float64 and rounded once
        const double ex = (c.x - (g.xl + c.bxl * g.bsx)) * g.inv_bsx;
        const double ey = (c.y - (g.yl + c.byl * g.bsy)) * g.inv_bsy;
        geo[j] = rec_geo<T>(ex, ey, (double)cw[j] * g.inv_bsx, (double)chh[j] * g.inv_bsy,
                            c.byl, c.bxl - (s0 << b.lgR));
        const int nx = c.bxh - c.bxl, ny = c.byh - c.byl;
        s0v[j] = s0;
        m0[j] = rec_span<T>(c.bxl - (s0 << b.lgR), nx, ny, c.byl, false);
        r0[j] = atomicAdd(&cnt[s0], 1u);
        if (s1 != s0) {
            s1v[j] = s1;
            m1[j] = rec_span<T>(c.bxl - (s1 << b.lgR), nx, ny, c.byl, true);
            r1[j] = atomicAdd(&cnt[s1], 1u);
        }
    }
    __syncthreads();
    // one run per strip: its place in the region, and how much of it fits;
    // the part that does not (ov records) takes a block-local place in the
    // block's overflow (an LDS atomic): cnt[s] <- that place << 16 | ov
    // (both below 2 * kOnceThreads * kOnceMaxCpt < 2^16)
    for (int s = tid; s < S; s += NT) {
        const unsigned h = cnt[s];
        unsigned ov = 0u;
        if (h) {
            const unsigned o = atomicAdd(&xrow[s], h);
            start[s] += o;
            const unsigned rm = room[s] > o ? room[s] - o : 0u;
            room[s] = rm;
            ov = h > rm ? h - rm : 0u;
        }
        cnt[s] = ov ? (atomicAdd(&npool[0], ov) << 16) | ov : 0u;
    }
    __syncthreads();
    // records that fit: straight to their slot; the others (bit 2j / 2j + 1
    // of ovm) are placed below, once the block's overflow has its range
    unsigned ovm = 0u;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        if (s0v[j] < 0) continue;
        if (r0[j] < room[s0v[j]]) {
            p0[j] = start[s0v[j]] + r0[j];
            rec_put<T>(b, recg, p0[j], geo[j], m0[j]);
        } else {
            p0[j] = r0[j] - room[s0v[j]];       // its place in the strip's run
            ovm |= 1u << (2 * j);
        }
        if (s1v[j] >= 0) {
            if (r1[j] < room[s1v[j]]) {
                p1[j] = start[s1v[j]] + r1[j];
                rec_put<T>(b, recg, p1[j], geo[j], m1[j]);
            } else {
                p1[j] = r1[j] - room[s1v[j]];
                ovm |= 1u << (2 * j + 1);
            }
        }
    }
    __syncthreads();
    const unsigned nover = npool[0];            // uniform across the group
    if (nover) {
        // the block's overflow takes one range of the pool (one atomic);
        // each strip's part is one run of that strip's overflow list (one
        // 64-bit atomic gives the run its place in the list and its first
        // record's number).  cnt[s] <- the pool index of the run's first
        // record; a record's place in its run (in p0 / p1) is its rank past
        // the room.
        if (tid == 0) npool[1] = atomicAdd(&b.pool_n[b.par & 1], nover);
        __syncthreads();
        const unsigned pb = npool[1];
        unsigned long long* ost = overflow_state(b, b.par);
        for (int s = tid; s < S; s += NT) {
            const unsigned c = cnt[s];
            const unsigned ov = c & 0xFFFFu;
            if (!ov) continue;
            const unsigned q = pb + (c >> 16);
            const unsigned long long old = atomicAdd(&ost[s], (1ull << 32) | ov);
            const unsigned k = (unsigned)(old >> 32);
            if (k < (unsigned)b.rmax)   // always: one run per block and strip
                b.oruns[(size_t)s * b.rmax + k] = uint2{q, (unsigned)old};
            cnt[s] = q;
        }
        __syncthreads();
        auto place = [&](unsigned& p, int s, unsigned m, const vec4_t<T>& gm) {
            const unsigned q = cnt[s] + p;
            if (q >= b.pool_cap) {      // cannot happen: the pool holds 2 nc
                p = kPosNone;
                return;
            }
            p = b.pool0 + q;
            rec_put<T>(b, recg, p, gm, m);
        };
        if (ovm) {
#pragma unroll
            for (int j = 0; j < CPT; ++j) {
                if ((ovm >> (2 * j)) & 1u) place(p0[j], s0v[j], m0[j], geo[j]);
                if ((ovm >> (2 * j + 1)) & 1u) place(p1[j], s1v[j], m1[j], geo[j]);
            }
        }
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int i = c0 + tid + j * NT;
        if (i < cend) b.pos[i] = pos_pair(p0[j], p1[j]);
    }
    // the tall cells, by teams of threads, last: the per-cell arrays above
    // are dead here (earlier, their registers spilled); coordinates past the
    // first kTallList come from the cell arrays
    const unsigned nt = *ntall;                 // uniform across the group
    const int team = tid / kTallTeam, lane = tid % kTallTeam;
    for (unsigned t = (unsigned)team; t < nt; t += NT / kTallTeam) {
        const unsigned i = tall_idx[t];
        const vec4_t<T> cell = t < (unsigned)kTallList
                                   ? tall_cell[t]
                                   : vec4_t<T>{px[i], py[i], sx[i], sy[i]};
        scatter_tall_team<T>(cell, lane, g, b, Bm);
    }
}

// One record's partial force over rows [ka', kb'] = its rows within
// [kg0, kg1] (a row group of its strip with first row k0) from rows, row kg0
// of the group's (fx, fy) pairs in LDS with rows N pairs apart.  G1 takes
// the strip's records and its overflow records alike through it: the same
// values in the same order, so the same partial.
// The first Q columns of a row are read unconditionally (float32: Q = 4 where
// a lane of the wave has a record spanning four or more columns, the wave's
// choice by __any, else 3; float64: 4), with weight zero where the record has no positive overlap
// (a column past its last, or a row or column it only touches): those terms
// add a signed zero, which leaves every sum bitwise as if they were skipped,
// so either Q gives the same partial.  Branching around each read instead
// made every read wait for its own LDS round trip; Q = 4 for every wave
// measured slower where records span two or three columns (C3, C5), Q = 3
// for every wave slower where many span four (C2).  So up to 3 pairs past
// any column of a row must be readable and finite: the next row's pairs, or
// (after the last row) padding (kGatherPadBins).
// A row's x overlap is min(xr - jx, 1) - max(dx - jx, 0) for the row jx
// rows past the record's first: xr - jx is exact for every row the record
// spans (jx is an integer no larger than xr) and dx - jx is negative past the
// first row, so the overlap equals min(xr, jx + 1) - max(dx, jx) bit for bit
// with a float counter and no conversion per row.
template <typename T, int Q>
__device__ __forceinline__ vec2_t<T> partial_rows(const RecView<T>& rv, const T* tyv, int ka,
                                                  int kb, int kg0, int N, const vec2_t<T>* rows)
{
    const T xr = rv.xr, yr = rv.yr, dx = rv.dx, dy = rv.dy;
    T ax = (T)0, ay = (T)0;
    // row offsets below 2^24 (rows < 8, N <= 8192): a 24-bit multiply
    const vec2_t<T>* rf = rows + (__umul24((unsigned)(ka - kg0), (unsigned)N) + (unsigned)rv.byl);
    T jx = (T)(ka - rv.bxl);
    for (int k = ka; k <= kb; ++k, rf += N, jx += (T)1) {
        const T t = min(xr - jx, (T)1) - max(dx - jx, (T)0);
        const T tx = t > (T)0 ? t : (T)0;
        vec2_t<T> fq[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) fq[q] = rf[q];
        T sx_ = (T)0, sy_ = (T)0;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            sx_ += tyv[q] * fq[q].x;
            sy_ += tyv[q] * fq[q].y;
        }
        for (int q = Q; q <= rv.ny; ++q) {
            const T ty = min(yr, (T)(q + 1)) - max(dy, (T)q);
            if (!(ty > (T)0)) continue;
            const vec2_t<T> f = rf[q];
            sx_ += ty * f.x;
            sy_ += ty * f.y;
        }
        ax += tx * sx_;
        ay += tx * sy_;
    }
    return vec2_t<T>{ax, ay};
}

template <typename T>
__device__ __forceinline__ vec2_t<T> record_partial(const vec4_t<T>& rg, unsigned rm, int k0,
                                                    int kg0, int kg1, int N, int stretch, T ba,
                                                    const vec2_t<T>* rows)
{
    const RecView<T> rv = rec_view<T>(rg, rm, k0, stretch, N);
    const int ka = max(rv.bxl, kg0), kb = min(rv.bxl + rv.nx, kg1);
    // y overlaps of the (usual) first 4 columns, shared by the rows (zero
    // where not positive); yr clamped to the grid's last column edge gives
    // the columns past it no positive overlap and the others their own
    const T yrc = min(rv.yr, (T)(N - rv.byl));
    T tyv[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) tyv[q] = max(min(yrc, (T)(q + 1)) - max(rv.dy, (T)q), (T)0);
    // float64 keeps Q = 4 (the choice measured +1.2 us at 1.1M cells, 2048^2)
    const vec2_t<T> a = (sizeof(T) == 8 || __any(rv.ny >= 3))   // uniform
                            ? partial_rows<T, 4>(rv, tyv, ka, kb, kg0, N, rows)
                            : partial_rows<T, 3>(rv, tyv, ka, kb, kg0, N, rows);
    const T sc = rv.rat * ba;
    return vec2_t<T>{sc * a.x, sc * a.y};
}

// rho = D0 + fixed-point sum, rounded once to T.
template <typename T>
__device__ __forceinline__ void flush_value(unsigned long long v, size_t gi,
                                            const T* __restrict__ d0n,
                                            T* __restrict__ dens, double inv)
{
    dens[gi] = (T)((double)d0n[gi] + (double)v * inv);
}

// ---------------------------------------------------------------------------
// K4: accumulate one (strip, chunk) work item in an LDS tile of R x N
// uint64 fixed-point words; the workgroup that completes a strip flushes it
// (rho = D0 + tile (+B)) and runs the strip's row DCT-II (the first spectral
// pass) on the rows it already holds, writing T in the tile layout: the
// density is never read back.  A strip split into n > 1 chunks: each chunk
// adds its tile into the strip's rows of the side map B; the last chunk to
// finish reads them back and completes the strip.
// ---------------------------------------------------------------------------

// Elements per thread of K4's row DCT: the fewest (8 or more) that keep the
// strip's R / 2 FFTs within the workgroup, so every thread takes part.
__host__ __device__ constexpr int acc_e(int L, int R)
{
    int e = 8;
    while (e < fft_e(L) && (R / 2) * (L / e) > kAccThreads) e <<= 1;
    return e < L ? e : L;
}

template <typename T, int L>
__host__ __device__ constexpr size_t acc_lds_main()
{
    constexpr int R = strip_rows(L);
    // the tile, the split-strip flag (16 bytes), the overflow run table
    const size_t tile = (size_t)R * L * sizeof(unsigned long long) + 16 +
                        (size_t)kRunBatch * sizeof(uint2);
    const size_t fft = (size_t)(R / 2) * lds_len(L) * sizeof(vec2_t<T>);
    return ((tile > fft ? tile : fft) + 15) / 16 * 16;
}

// Whether K4 copies the table of W^m (m < L) into LDS at its start, beside
// the tile (float32, where a CU still holds as many K4 workgroups): the row
// DCT then reads its twiddles from LDS, with no global-load latency between
// the flush and the FFT.
template <typename T, int L>
__host__ __device__ constexpr bool acc_twiddles_in_lds()
{
    constexpr size_t kLds = 163840, main = acc_lds_main<T, L>();
    constexpr size_t with = main + (size_t)L * sizeof(vec2_t<T>);
    return sizeof(T) == 4 && with <= kLds && kLds / with == kLds / main;
}

template <typename T, int L>
__host__ __device__ constexpr size_t acc_lds_bytes()
{
    return acc_lds_main<T, L>() +
           (acc_twiddles_in_lds<T, L>() ? (size_t)L * sizeof(vec2_t<T>) : 0);
}

template <typename T, int L>
__global__ __launch_bounds__(kAccThreads) void k_strip_acc(
    Grid g, BinArgs b, SpectralArgs a, const T* __restrict__ d0n,
    T* __restrict__ dens, T* __restrict__ Tt)
{
    using A = unsigned long long;
    using C = vec2_t<T>;
    constexpr int R = strip_rows(L);
    constexpr int RN = R * L;
    constexpr int N = L;
    extern __shared__ __align__(16) unsigned char smem[];
    A* tile = reinterpret_cast<A*>(smem);
    const int w = blockIdx.x;
    const int tid = threadIdx.x;
    if (w == 0) {   // K3 has read the previous step's counts: zero them
        unsigned* old = counts_of(b, b.par ^ 1);
        for (int e = tid; e < kCountSlots * b.S; e += kAccThreads) old[e] = 0u;
        unsigned long long* ost = overflow_state(b, b.par ^ 1);
        for (int e = tid; e < b.S; e += kAccThreads) ost[e] = 0ull;
        if (tid == 0) b.pool_n[(b.par ^ 1) & 1] = 0u;
    }
    if (w >= (int)b.nitems[0]) return;          // uniform across the group
    const uint4 item = b.items[w];
    const int s = (int)(item.x & 0xFFFFu);
    const int k0 = s * R, k1 = k0 + R - 1;
    const unsigned n = item.w;                  // chunks of this strip
    unsigned* last_flag = reinterpret_cast<unsigned*>(tile + RN);   // LDS word
    // the strip's map (its loads in flight while the tile is zeroed), then
    // one record per thread per pass, the next one's loads in flight while
    // it is added (measured faster here than 2, 4 or 8 records per pass, or
    // than two ahead)
    StripMap sm;
    strip_map(b, s, sm);
    constexpr bool kTwL = acc_twiddles_in_lds<T, L>();
    C* twl = reinterpret_cast<C*>(smem + acc_lds_main<T, L>());   // kTwL: W^m, m < L
    if constexpr (kTwL) {   // read at the row DCT, many barriers on
        const C* tw = reinterpret_cast<const C*>(a.twN);
        for (int e = tid; e < L; e += kAccThreads) twl[e] = tw[e];
    }
    for (int e = tid; e < RN; e += kAccThreads) tile[e] = 0ull;
    unsigned e0, e1;                            // this chunk's records
    item_range(item, sm, e0, e1);
    const vec4_t<T>* recg = reinterpret_cast<const vec4_t<T>*>(b.recg);
    const T fs = (T)g.fix_scale;
    vec4_t<T> rgn{};
    unsigned rmn = 0u;
    if (e0 + tid < e1) {
        const unsigned r = map_record(sm, e0 + tid);
        rgn = recg[r];
        rmn = rec_m<T>(b, r);
    }
    __syncthreads();
    for (unsigned eb = e0 + tid; eb < e1; eb += kAccThreads) {
        const vec4_t<T> rg = rgn;
        const unsigned rm = rmn;
        if (eb + kAccThreads < e1) {     // the next record, in flight meanwhile
            const unsigned r = map_record(sm, eb + kAccThreads);
            rgn = recg[r];
            rmn = rec_m<T>(b, r);
        }
        record_density<T>(rg, rm, k0, k1, N, g.stretch, fs, tile);
    }
    // the strip's overflow list (records past their region's room), by the
    // strip's first chunk, added into the tile like the others
    for_overflow_records(b, s, item, tid, reinterpret_cast<uint2*>(tile + RN + 2),
                         [&](unsigned r) {
                             record_density<T>(recg[r], rec_m<T>(b, r), k0, k1, N, g.stretch, fs,
                                               tile);
                         });
    __syncthreads();

    const size_t gbase = (size_t)k0 * N;
    const double inv = 1.0 / g.fix_scale;
    A* Bm = reinterpret_cast<A*>(b.B);
    if (n > 1u) {
        // A strip split into n chunks: every chunk but the last to finish
        // adds its tile into the strip's rows of B with device-scope atomics;
        // the last one folds B in its flush.  Ordering: each wave awaits the
        // results of its own atomics (so they are performed before the
        // barrier), the barrier orders the waves before thread 0, and thread
        // 0 takes the strip's ticket with an acquire-release RMW at agent
        // scope: every chunk's sums happen-before the ticket that follows
        // them, and the chunk that draws the last ticket reads B after it.
        unsigned long long got = 0ull;
        for (int e = tid; e < RN; e += kAccThreads) {
            const A v = tile[e];
            if (v) got |= atomicAdd(&Bm[gbase + e], v);
        }
        // never true (sums stay below 2^63); it makes the results live
        if (got >> 63) *last_flag = 0u;
        __syncthreads();
        if (tid == 0)
            *last_flag = __hip_atomic_fetch_add(&b.done[s], 1u, __ATOMIC_ACQ_REL,
                                                __HIP_MEMORY_SCOPE_AGENT) == n - 1u
                             ? 1u : 0u;
        __syncthreads();
        if (*last_flag == 0u) return;           // uniform across the group
        if (tid == 0) b.done[s] = 0u;
    }

    // ---- flush: rho = D0 + tile (+B), kept in registers ------------------
    constexpr int PER = (RN + kAccThreads - 1) / kAccThreads;
    // the column blocks of the strip's rows that hold sums in B: those its
    // tall cells marked, or all of them for a split strip (read at device
    // scope: the other chunks added them in this launch)
    const bool split = n > 1u;
    constexpr int CB = side_block(N);
    unsigned side[kSideWords];
    bool bf = split;
#pragma unroll
    for (int q = 0; q < kSideWords; ++q) {
        side[q] = split ? 0xFFFFFFFFu : b.bigflag[(size_t)s * kSideWords + q];
        bf = bf || side[q] != 0u;
    }
    T rv[PER];
    {
        A v[PER];
        T d[PER];
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = tid + j * kAccThreads;
            if (e < RN) {
                v[j] = split ? 0ull : tile[e];  // a split strip's tiles are all in B
                d[j] = d0n[gbase + e];
            }
        }
        if (bf) {
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int e = tid + j * kAccThreads;
                const int cb = (e & (N - 1)) / CB;
                if (e < RN && ((side[cb >> 5] >> (cb & 31)) & 1u)) {
                    v[j] += split ? __hip_atomic_load(&Bm[gbase + e], __ATOMIC_RELAXED,
                                                      __HIP_MEMORY_SCOPE_AGENT)
                                  : Bm[gbase + e];
                    Bm[gbase + e] = 0ull;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < PER; ++j) {
            const int e = tid + j * kAccThreads;
            if (e < RN) {
                rv[j] = (T)((double)d[j] + (double)v[j] * inv);
                dens[gbase + e] = rv[j];
            }
        }
        // the cells' own density, before the initial density is added (the
        // reference server's density read-back, kept for its dump and its
        // CPU-solve mode); a uniform branch, off unless the context asks
        if (b.raw) {
            T* raw = reinterpret_cast<T*>(b.raw);
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int e = tid + j * kAccThreads;
                if (e < RN) raw[gbase + e] = (T)((double)v[j] * inv);
            }
        }
    }
    __syncthreads();   // the tile is dead (the FFT buffers alias it); bitmap read
    if (tid < kSideWords && (split || side[tid] != 0u))
        b.bigflag[(size_t)s * kSideWords + tid] = 0u;

    // ---- row DCT-II of the strip's R rows: rows (2p, 2p+1) -> FFT slot p --
    constexpr int LP = lds_len(L), E = acc_e(L, R), TPF = L / E;
    const bool act = tid < (R / 2) * TPF;
    const int f = act ? tid / TPF : 0, t = tid % TPF;
    // the transform's twiddles, loaded before the rows go to LDS (float32;
    // at float64 the registers they would hold while the rows are live
    // spill, so they are read where used)
    const C* post = reinterpret_cast<const C*>(a.postN);
    FftTw<T, L, E> twp;
    C pst[E / 2];
    if constexpr (sizeof(T) == 4) {
        fft_tw_fetch<T, L, E>(twp, t, kTwL ? twl : reinterpret_cast<const C*>(a.twN));
#pragma unroll
        for (int i = 0; i < E / 2; ++i) pst[i] = post_of<T, L>(post, t + TPF * i);
    }
    C* sbuf = reinterpret_cast<C*>(smem);
#pragma unroll
    for (int j = 0; j < PER; ++j) {
        const int e = tid + j * kAccThreads;
        if (e < RN) {
            const int r = e / L, m = e % L;
            comp<T>(sbuf[(r >> 1) * LP + lds_pad(makhoul_pos<L>(m))], r & 1) = rv[j];
        }
    }
    __syncthreads();
    C* buf = sbuf + f * LP;
    if constexpr (sizeof(T) == 4)
        fft_lds<T, L, false>(buf, t, twp, act);
    else
        fft_lds<T, L, false, E>(buf, t, reinterpret_cast<const C*>(a.twN), act);
    {
        const T scale = (T)2 / (T)L;
        C Xk[E / 2], Xm[E / 2];
        if (act) {
#pragma unroll
            for (int i = 0; i < E / 2; ++i)
                dct_post<T, L>(buf, t + TPF * i,
                               sizeof(T) == 4 ? pst[i] : post_of<T, L>(post, t + TPF * i),
                               scale, Xk[i], Xm[i]);
        }
        __syncthreads();
        if (act) {
#pragma unroll
            for (int i = 0; i < E / 2; ++i) {
                const int sl = t + TPF * i;
                buf[lds_pad(sl)] = Xk[i];
                buf[lds_pad(sl == 0 ? L / 2 : L - sl)] = Xm[i];
            }
        }
    }
    __syncthreads();

    // ---- T in the tile layout: bands of min(R, TX) rows ------------------
    {
        constexpr int V = kVec<T>;
        const int TX = a.tiles.TXT, TV = a.tiles.TV;
        const int lgTV = __builtin_ctz(TV);
        const int lgTX = __builtin_ctz(TX), lgNBV = __builtin_ctz(L) - lgTV;
        const int TXe = R < TX ? R : TX;
        const int lgTXe = __builtin_ctz(TXe);
        constexpr int lgL = __builtin_ctz(L);
        for (int n0 = tid * V; n0 < RN; n0 += kAccThreads * V) {
            const int band = n0 >> (lgTXe + lgL);
            const int nb = n0 & ((TXe << lgL) - 1);
            const int bv = nb >> (lgTXe + lgTV);
            const int wv = nb & ((TXe << lgTV) - 1);
            const int r = band * TXe + (wv >> lgTV);        // row within the strip
            const int x = k0 + r;
            const int v = (bv << lgTV) + (wv & (TV - 1));
            const C* rowp = sbuf + (r >> 1) * LP;
            pack<T> o;
#pragma unroll
            for (int q = 0; q < V; ++q) o.v[q] = comp_of<T>(rowp[lds_pad(v + q)], r & 1);
            // tile (x / TX, bv), row x % TX within it (powers of two: shifts)
            const unsigned gi =
                (((((unsigned)x >> lgTX) << lgNBV) + (unsigned)bv) << (lgTX + lgTV)) +
                (((unsigned)x & (TX - 1)) << lgTV) + (unsigned)(wv & (TV - 1));
            *reinterpret_cast<pack<T>*>(Tt + gi) = o;
        }
    }
}

// ---------------------------------------------------------------------------
// G1: one (strip, chunk) work item.  The strip's field rows are staged in
// LDS, RG rows at a time (RG = R for float32; fewer for float64), and each
// record's partial force over the rows of this strip is written (first row
// group) or added (later groups) to gtmp in record order.
// ---------------------------------------------------------------------------
template <typename T>
__host__ __device__ constexpr int gather_rows(int R, int N)
{
    int rg = R;
    while (rg > 1 && (size_t)rg * N * 2 * sizeof(T) > kTileBytes) rg >>= 1;
    return rg;
}

// G1's LDS: the staged rows of both field maps, kGatherPadBins zero (fx, fy)
// pairs (record_partial reads up to 3 bins past a record's first column,
// also in the last staged row), then the overflow run table.
constexpr int kGatherPadBins = 4;

template <typename T>
__host__ __device__ constexpr size_t gather_lds_fields(int R, int N)
{
    return (size_t)gather_rows<T>(R, N) * N * 2 * sizeof(T);
}
template <typename T>
__host__ __device__ constexpr size_t gather_lds_runs(int R, int N)
{
    return gather_lds_fields<T>(R, N) + (size_t)kGatherPadBins * 2 * sizeof(T);
}
template <typename T>
__host__ __device__ constexpr size_t gather_lds(int R, int N)
{
    return gather_lds_runs<T>(R, N) + (size_t)kRunBatch * sizeof(uint2);
}

template <typename T, bool kGuess>
__global__ __launch_bounds__(kAccThreads) void k_gather_bin(
    Grid g, BinArgs b, const T* __restrict__ fx, const T* __restrict__ fy)
{
    extern __shared__ __align__(16) unsigned char smem[];
    const int w = blockIdx.x;
    const int tid = threadIdx.x;
    const int R = b.R, N = g.N;
    const int RG = gather_rows<T>(R, N);
    const vec4_t<T>* recg = reinterpret_cast<const vec4_t<T>*>(b.recg);
    vec2_t<T>* out = reinterpret_cast<vec2_t<T>*>(b.gtmp);
    const T ba = (T)(g.bsx * g.bsy);
    // kGuess (a grid of one workgroup per strip, b.Wgat == b.S): item w is
    // strip w unless a strip is split, so the map of strip w is requested
    // with the item and their loads are in flight together (G1 22.8 -> 21.8
    // us at 1.1M cells on 2048^2; a run-time choice between the two forms
    // measured slower than either; in K4 the same measured slower, its map's
    // latency already overlapping the tile's zeroing).  With more items than
    // strips (small grids) the guess is mostly wrong: wait for the item.
    StripMap sm;
    if constexpr (kGuess) strip_map(b, w, sm);
    if (w < (int)b.nitems[1]) {                 // uniform across the group
        const uint4 item = b.items_g[w];
        const int s = (int)(item.x & 0xFFFFu);
        const int k0 = s * R;
        if (!kGuess || s != w) strip_map(b, s, sm);  // uniform across the group
        unsigned e0, e1;                        // this item's records
        item_range(item, sm, e0, e1);
        // both fields of a bin side by side: one 2-element LDS read per bin;
        // then the overflow run table
        vec2_t<T>* lf = reinterpret_cast<vec2_t<T>*>(smem);
        uint2* lrun = reinterpret_cast<uint2*>(smem + gather_lds_runs<T>(R, N));
        if (tid < kGatherPadBins)               // written before the loop's first barrier
            lf[(size_t)RG * N + tid] = vec2_t<T>{(T)0, (T)0};
        vec4_t<T> rg0{};
        unsigned rm0 = 0u, rn0 = 0u;
        if (e0 + tid < e1) {                    // the first record, before the rows
            rn0 = map_record(sm, e0 + tid);
            rg0 = recg[rn0];
            rm0 = rec_m<T>(b, rn0);
        }
        for (int kg0 = k0; kg0 < k0 + R; kg0 += RG) {
            const int kg1 = kg0 + RG - 1;
            __syncthreads();                    // previous group's readers done
            const size_t gb = (size_t)kg0 * N;
            {
                // 16-byte vectors, all of a thread's loads in flight at once
                using V16 = typename std::conditional<sizeof(T) == 4, float4, double2>::type;
                constexpr int V = 16 / (int)sizeof(T);
                // RG rows of both maps fill at most kTileBytes
                constexpr int PV = (int)(kTileBytes / (2 * 16) / kAccThreads);
                const int nv = RG * N / V;
                const V16* gx4 = reinterpret_cast<const V16*>(fx + gb);
                const V16* gy4 = reinterpret_cast<const V16*>(fy + gb);
                V16* l4 = reinterpret_cast<V16*>(lf);
                // V bins of fx and of fy -> V interleaved (fx, fy) pairs
                auto put = [&](int e, const V16& x, const V16& y) {
                    if constexpr (sizeof(T) == 4) {
                        l4[2 * e] = V16{x.x, y.x, x.y, y.y};
                        l4[2 * e + 1] = V16{x.z, y.z, x.w, y.w};
                    } else {
                        l4[2 * e] = V16{x.x, y.x};
                        l4[2 * e + 1] = V16{x.y, y.y};
                    }
                };
                if (nv == PV * kAccThreads) {
                    V16 vx[PV], vy[PV];
#pragma unroll
                    for (int j = 0; j < PV; ++j) {
                        vx[j] = gx4[tid + j * kAccThreads];
                        vy[j] = gy4[tid + j * kAccThreads];
                    }
#pragma unroll
                    for (int j = 0; j < PV; ++j) put(tid + j * kAccThreads, vx[j], vy[j]);
                } else {
                    for (int e = tid; e < nv; e += kAccThreads) put(e, gx4[e], gy4[e]);
                }
            }
            __syncthreads();
            const bool first = kg0 == k0;
            // one record per pass, the next one in flight
            vec4_t<T> rgn = rg0;
            unsigned rmn = rm0, rn = rn0;
            if (kg0 != k0 && e0 + tid < e1) {
                rn = map_record(sm, e0 + tid);
                rgn = recg[rn];
                rmn = rec_m<T>(b, rn);
            }
            for (unsigned eb = e0 + tid; eb < e1; eb += kAccThreads) {
                const vec4_t<T> rg = rgn;
                const unsigned rm = rmn, r = rn;
                if (eb + kAccThreads < e1) {
                    rn = map_record(sm, eb + kAccThreads);
                    rgn = recg[rn];
                    rmn = rec_m<T>(b, rn);
                }
                vec2_t<T> v = record_partial<T>(rg, rm, k0, kg0, kg1, N, g.stretch, ba, lf);
                if (!first) {
                    const vec2_t<T> o = out[r];
                    v.x += o.x;
                    v.y += o.y;
                }
                out[r] = v;
            }
            // the strip's overflow list, by the strip's first chunk, from
            // the same rows in LDS and in the same order of row groups
            for_overflow_records(b, s, item, tid, lrun, [&](unsigned r) {
                vec2_t<T> v = record_partial<T>(recg[r], rec_m<T>(b, r), k0, kg0, kg1, N,
                                                g.stretch, ba, lf);
                if (!first) {
                    const vec2_t<T> o = out[r];
                    v.x += o.x;
                    v.y += o.y;
                }
                out[r] = v;
            });
        }
    }
}

// ---------------------------------------------------------------------------
// Fixed-cell density D0n = target_density * sum of exact overlaps / bin area
// (no stretch: DREAMPlace's fixed density map, the initial_density_map the
// reference's client uploads at integration/scatter_ttnn_client.py:786-795).
// One workgroup per fixed cell walks its bin rectangle and adds uint64 fixed
// point into the side map B (exact, order-free); a second kernel converts
// and re-zeroes B.  A set-up computation, run once per placement.
// ---------------------------------------------------------------------------
constexpr int kFixedThreads = 256;

template <typename T>
__global__ __launch_bounds__(kFixedThreads) void k_fixed_overlap(
    const T* __restrict__ px, const T* __restrict__ py, const T* __restrict__ sx,
    const T* __restrict__ sy, int n, Grid g, double scale,
    unsigned long long* __restrict__ B)
{
    const int i = blockIdx.x;
    if (i >= n) return;
    CellSpan c;
    if (!cell_span((double)px[i], (double)py[i], (double)sx[i], (double)sy[i], g, c))
        return;
    const int nrow = c.bxh - c.bxl + 1, ncol = c.byh - c.byl + 1;
    const long long total = (long long)nrow * ncol;
    for (long long e = threadIdx.x; e < total; e += kFixedThreads) {
        const int k = c.bxl + (int)(e / ncol), q = c.byl + (int)(e % ncol);
        const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
        const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
        const double v = tx * ty * g.inv_ba;
        if (v > 0.0) atomicAdd(&B[(size_t)k * g.N + q], to_fixed(v, scale));
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_fixed_flush(unsigned long long* __restrict__ B,
                                                     T* __restrict__ d0n, size_t mn,
                                                     double factor)
{
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= mn) return;
    d0n[i] = (T)((double)B[i] * factor);
    B[i] = 0ull;
}

// ---------------------------------------------------------------------------
// G2: forces in cell order: gx[i], gy[i] from the record pos[i]; cells that
// contribute nothing get zero.  Tall cells are gathered in float64 by the
// whole workgroup, one cell at a time: the threads split the cell's bins and
// a fixed-shape tree in LDS sums their parts (deterministic), so a wide cell
// costs one round of loads instead of a serial walk over its bins.
// LDS: ntall | list[kCellsPerGroup] | red[2][kBinThreads] (doubles).
// ---------------------------------------------------------------------------
// LDS of G2: the tall-cell count and list, one bit per list entry marking
// the cells too large for a team, and the workgroup-wide reduction buffer
template <int NT, int CPT>
__host__ __device__ constexpr size_t gather_out_lds()
{
    return ((1 + NT * CPT + NT * CPT / 32) * sizeof(unsigned) + 15) / 16 * 16 +
           2 * NT * sizeof(double);
}

template <typename T, int NT>
__device__ __forceinline__ void gather_tall(int i, const T* __restrict__ px,
                                            const T* __restrict__ py,
                                            const T* __restrict__ sx,
                                            const T* __restrict__ sy, const Grid& g,
                                            const T* __restrict__ fx,
                                            const T* __restrict__ fy, double* red,
                                            T* __restrict__ gx, T* __restrict__ gy)
{
    const int tid = threadIdx.x;
    CellSpan c;
    double ax = 0.0, ay = 0.0;
    const bool ok = load_span(px, py, sx, sy, i, g, c);     // uniform: same cell
    if (ok) {
        const int ny1 = c.byh - c.byl + 1;
        const long long nb = (long long)(c.bxh - c.bxl + 1) * ny1;
        for (long long e = tid; e < nb; e += NT) {
            const int k = c.bxl + (int)(e / ny1), q = c.byl + (int)(e % ny1);
            const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
            const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
            const double a = tx * ty;
            if (a > 0.0) {
                const size_t gi = (size_t)k * g.N + q;
                ax += a * (double)fx[gi];
                ay += a * (double)fy[gi];
            }
        }
    }
    red[tid] = ax;
    red[NT + tid] = ay;
    __syncthreads();
    for (int h = NT / 2; h > 0; h >>= 1) {
        if (tid < h) {
            red[tid] += red[tid + h];
            red[NT + tid] += red[NT + tid + h];
        }
        __syncthreads();
    }
    if (tid == 0) {
        const double rat = ok ? c.ratio() : 0.0;
        gx[i] = ok ? (T)(red[0] * rat) : (T)0;
        gy[i] = ok ? (T)(red[NT] * rat) : (T)0;
    }
    __syncthreads();                      // red is reused by the next cell
}

// A tall cell of at most kTallTeamBins bins, gathered by the kTallTeam
// threads of one team (lane: index in the team; every lane calls it for the
// same cell): the bins strided over the team, float64 partial sums reduced
// by shuffles within the team in a fixed order.  Returns false (nothing
// written) for a larger cell, which the whole workgroup then gathers.
constexpr long long kTallTeamBins = 256;

template <typename T>
__device__ __forceinline__ bool gather_tall_team(int i, int lane, const T* __restrict__ px,
                                                 const T* __restrict__ py,
                                                 const T* __restrict__ sx,
                                                 const T* __restrict__ sy, const Grid& g,
                                                 const T* __restrict__ fx,
                                                 const T* __restrict__ fy,
                                                 T* __restrict__ gx, T* __restrict__ gy)
{
    CellSpan c;
    const bool ok = load_span(px, py, sx, sy, i, g, c);     // same for the team
    if (ok && (long long)(c.bxh - c.bxl + 1) * (c.byh - c.byl + 1) > kTallTeamBins)
        return false;
    double ax = 0.0, ay = 0.0;
    if (ok) {
        const int ny1 = c.byh - c.byl + 1;
        const int nb = (c.bxh - c.bxl + 1) * ny1;
        for (int e = lane; e < nb; e += kTallTeam) {
            const int k = c.bxl + e / ny1, q = c.byl + e % ny1;
            const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
            const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
            const double a = tx * ty;
            if (a > 0.0) {
                const size_t gi = (size_t)k * g.N + q;
                ax += a * (double)fx[gi];
                ay += a * (double)fy[gi];
            }
        }
    }
#pragma unroll
    for (int m = kTallTeam / 2; m > 0; m >>= 1) {
        ax += __shfl_xor(ax, m, kTallTeam);
        ay += __shfl_xor(ay, m, kTallTeam);
    }
    if (lane == 0) {
        const double rat = ok ? c.ratio() : 0.0;
        gx[i] = ok ? (T)(ax * rat) : (T)0;
        gy[i] = ok ? (T)(ay * rat) : (T)0;
    }
    return true;
}

// One workgroup of NT threads per one-pass K3 block of b.qcells <= NT * CPT
// cells (the same cell-to-thread map): the records of a block sit in one
// short run per strip, so each run's partials are read whole, by one CU.
// Tall cells: a team of kTallTeam threads per cell of at most kTallTeamBins
// bins, larger ones one at a time by the whole workgroup.
template <typename T, int NT, int CPT>
__global__ __launch_bounds__(NT) void k_gather_out(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b, const T* __restrict__ fx, const T* __restrict__ fy,
    T* __restrict__ gx, T* __restrict__ gy)
{
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned* ntall = reinterpret_cast<unsigned*>(smem);
    unsigned* list = ntall + 1;
    constexpr int QC = NT * CPT;                // cells of the block
    unsigned* large = list + QC;
    double* red = reinterpret_cast<double*>(
        smem + ((1 + QC + QC / 32) * sizeof(unsigned) + 15) / 16 * 16);
    if (threadIdx.x == 0) *ntall = 0u;
    if (threadIdx.x < QC / 32) large[threadIdx.x] = 0u;
    __syncthreads();
    const int cb = (int)blockIdx.x * b.qcells;
    const int cend = min(cb + b.qcells, nc);
    const int c0 = cb + threadIdx.x;
    const vec2_t<T>* res = reinterpret_cast<const vec2_t<T>*>(b.gtmp);
    unsigned p[CPT], p2[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int i = c0 + j * NT;
        const unsigned long long pp = i < cend ? b.pos[i] : pos_pair(kPosNone, kPosNone);
        p[j] = (unsigned)pp;
        p2[j] = (unsigned)(pp >> 32);
    }
    vec2_t<T> v[CPT], v2[CPT];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        v[j] = p[j] < kPosNone ? res[p[j]] : vec2_t<T>{(T)0, (T)0};
        v2[j] = p2[j] < kPosNone ? res[p2[j]] : vec2_t<T>{(T)0, (T)0};
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int i = c0 + j * NT;
        if (i >= cend) break;
        if (p[j] == kPosTall) {
            list[atomicAdd(ntall, 1u)] = (unsigned)i;
            continue;
        }
        gx[i] = v[j].x + v2[j].x;
        gy[i] = v[j].y + v2[j].y;
    }
    __syncthreads();
    const unsigned n = *ntall;                // uniform across the group
    if (n == 0u) return;
    // one team per tall cell; a team's lane 0 marks the cells too large for
    // it, which the whole workgroup gathers afterwards
    constexpr int kTeams = NT / kTallTeam;
    const int team = threadIdx.x / kTallTeam, lane = threadIdx.x % kTallTeam;
    for (unsigned t = team; t < n; t += kTeams)
        if (!gather_tall_team<T>((int)list[t], lane, px, py, sx, sy, g, fx, fy, gx, gy) &&
            lane == 0)
            atomicOr(&large[t >> 5], 1u << (t & 31u));
    __syncthreads();
    for (unsigned t = 0; t < n; ++t)          // uniform across the group
        if ((large[t >> 5] >> (t & 31u)) & 1u)
            gather_tall<T, NT>((int)list[t], px, py, sx, sy, g, fx, fy, red, gx, gy);
}

}  // namespace dpep
