// dpep_bin.h -- strip-binned density scatter and field gather.
//
// The bin map is cut into S strips of R consecutive rows (R * N accumulator
// words fit a 64 KB LDS tile).  A counting sort puts every cell into the
// strip(s) its x-span touches; each strip is then accumulated in LDS by the
// workgroup that owns it and flushed with plain coalesced stores, the fixed
// density folded in on the way.  No global atomics on the common path.
//
//   k_bin_count   per-workgroup strip histograms (cnt[g][s])          K1
//   k_bin_scan    strip offsets, per-workgroup bases, chunk list      K2
//   k_bin_fill    cells -> strip-sorted entries; tall cells -> B      K3
//   k_strip_acc   one work item = (strip, chunk): LDS accumulate,     K4
//                 flush rho = D0 + tile (+B) or a partial slot
//   k_strip_red   strips split into several chunks: sum partials      K4r
//   k_gather_bin  forces from the fields, walking the sorted entries  G
//
// A cell whose span covers more than R rows ("tall") skips the sort: K3 adds
// it with global atomics into the side map B (zero between steps), marks the
// strips it touches, and K4/K4r fold and re-zero those rows of B.  Every
// other cell touches at most two strips, so the entry arrays hold 2*nc_max.
// Deterministic mode accumulates round(v * 2^f) in uint64 everywhere (LDS,
// B, partials); the sums are then independent of order.
#pragma once

#include <type_traits>

#include "dpep_internal.h"

namespace dpep {

template <typename T> struct vec4;
template <> struct vec4<float> { using type = float4; };
template <> struct vec4<double> { using type = double4; };
template <typename T> using vec4_t = typename vec4<T>::type;

// Strips [s0, s1] a cell occupies and whether it is tall.
__device__ __forceinline__ void cell_strips(const CellSpan& c, int R, int lgR,
                                            int& s0, int& s1, bool& tall)
{
    tall = (c.bxh - c.bxl + 1) > R;
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

// ---------------------------------------------------------------------------
// K1: per-workgroup strip histogram.
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
    const int c0 = blockIdx.x * kCellsPerGroup;
    const int c1 = min(c0 + kCellsPerGroup, nc);
    for (int i = c0 + tid; i < c1; i += kBinThreads) {
        CellSpan c;
        if (!load_span(px, py, sx, sy, i, g, c)) continue;
        int s0, s1;
        bool tall;
        cell_strips(c, b.R, b.lgR, s0, s1, tall);
        if (tall) continue;
        atomicAdd(&hist[s0], 1u);
        if (s1 != s0) atomicAdd(&hist[s1], 1u);
    }
    __syncthreads();
    unsigned* row = b.cnt + (size_t)blockIdx.x * b.S;
    for (int s = tid; s < b.S; s += kBinThreads) row[s] = hist[s];
}

// ---------------------------------------------------------------------------
// K2: one workgroup.  strip_off = exclusive scan of strip totals; cnt[g][s]
// becomes the first entry slot of workgroup g in strip s; work items.
// ---------------------------------------------------------------------------
__device__ __forceinline__ unsigned block_exclusive_scan(unsigned v,
                                                         unsigned* tmp,
                                                         unsigned& total)
{
    // Hillis-Steele over kScanThreads values in LDS.
    const int tid = threadIdx.x;
    tmp[tid] = v;
    __syncthreads();
    for (int off = 1; off < kScanThreads; off <<= 1) {
        const unsigned a = tid >= off ? tmp[tid - off] : 0u;
        __syncthreads();
        tmp[tid] += a;
        __syncthreads();
    }
    const unsigned incl = tmp[tid];
    total = tmp[kScanThreads - 1];
    __syncthreads();
    return incl - v;
}

__global__ __launch_bounds__(kScanThreads) void k_bin_scan(BinArgs b)
{
    // LDS: tot[S] | part[4][256] | tmp[1024]
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned* tot = reinterpret_cast<unsigned*>(smem);
    unsigned* part = tot + b.S;
    unsigned* tmp = part + 4 * 256;
    const int tid = threadIdx.x;
    const int S = b.S, G1 = b.G1;
    const int q = tid >> 8, lane = tid & 255;
    const int gq0 = (G1 * q) / 4, gq1 = (G1 * (q + 1)) / 4;

    // pass 1: totals per strip, in blocks of 256 strips
    for (int sb = 0; sb < S; sb += 256) {
        const int s = sb + lane;
        unsigned acc = 0u;
        if (s < S)
            for (int gg = gq0; gg < gq1; ++gg) acc += b.cnt[(size_t)gg * S + s];
        part[q * 256 + lane] = acc;
        __syncthreads();
        if (q == 0 && s < S)
            tot[s] = part[lane] + part[256 + lane] + part[512 + lane] + part[768 + lane];
        __syncthreads();
    }
    // pass 2: exclusive scan of tot -> strip_off (each thread a run of strips)
    const int per = (S + kScanThreads - 1) / kScanThreads;
    const int r0 = min(tid * per, S), r1 = min(r0 + per, S);
    unsigned run = 0u;
    for (int s = r0; s < r1; ++s) run += tot[s];
    unsigned total;
    unsigned base = block_exclusive_scan(run, tmp, total);
    for (int s = r0; s < r1; ++s) {
        const unsigned t = tot[s];
        b.strip_off[s] = base;
        tot[s] = base;          // tot now holds the strip offsets
        base += t;
        // chunks of this strip
        const unsigned n = (t + (unsigned)b.CH - 1u) / (unsigned)b.CH;
        b.nch[s] = n > 1u ? n : 1u;
    }
    if (tid == 0) {
        b.strip_off[S] = total;
        *b.big_count = 0u;
    }
    __syncthreads();
    // pass 3: per-workgroup bases, 4 contiguous g-blocks per strip
    for (int sb = 0; sb < S; sb += 256) {
        const int s = sb + lane;
        unsigned acc = 0u;
        if (s < S)
            for (int gg = gq0; gg < gq1; ++gg) acc += b.cnt[(size_t)gg * S + s];
        part[q * 256 + lane] = acc;
        __syncthreads();
        if (s < S) {
            unsigned off = tot[s];
            for (int qq = 0; qq < q; ++qq) off += part[qq * 256 + lane];
            for (int gg = gq0; gg < gq1; ++gg) {
                const unsigned v = b.cnt[(size_t)gg * S + s];
                b.cnt[(size_t)gg * S + s] = off;
                off += v;
            }
        }
        __syncthreads();
    }
    // pass 4: work items (strip, chunk)
    unsigned nrun = 0u;
    for (int s = r0; s < r1; ++s) nrun += b.nch[s];
    unsigned ntotal;
    unsigned ibase = block_exclusive_scan(nrun, tmp, ntotal);
    for (int s = r0; s < r1; ++s) {
        const unsigned n = b.nch[s];
        b.item_start[s] = ibase;
        for (unsigned c = 0; c < n; ++c)
            if (ibase + c < (unsigned)b.Wmax) b.items[ibase + c] = (unsigned)s | (c << 16);
        ibase += n;
    }
    if (tid == 0) *b.nitems = ntotal < (unsigned)b.Wmax ? ntotal : (unsigned)b.Wmax;
}

// ---------------------------------------------------------------------------
// K3: fill the strip-sorted entries; tall cells go to B; invalid cells get
// zero force.
// ---------------------------------------------------------------------------
template <typename T, bool FIXED>
__global__ __launch_bounds__(kBinThreads) void k_bin_fill(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    BinArgs b, T* __restrict__ gx, T* __restrict__ gy)
{
    using A = typename std::conditional<FIXED, unsigned long long, T>::type;
    extern __shared__ __align__(16) unsigned char smem[];
    unsigned* cur = reinterpret_cast<unsigned*>(smem);
    const int tid = threadIdx.x;
    const unsigned* row = b.cnt + (size_t)blockIdx.x * b.S;
    for (int s = tid; s < b.S; s += kBinThreads) cur[s] = row[s];
    __syncthreads();
    vec4_t<T>* ent = reinterpret_cast<vec4_t<T>*>(b.entries);
    A* Bm = reinterpret_cast<A*>(b.B);
    const int c0 = blockIdx.x * kCellsPerGroup;
    const int c1 = min(c0 + kCellsPerGroup, nc);
    for (int i = c0 + tid; i < c1; i += kBinThreads) {
        CellSpan c;
        const T x = px[i], y = py[i], w = sx[i], h = sy[i];
        if (!cell_span((double)x, (double)y, (double)w, (double)h, g, c)) {
            if (gx) { gx[i] = (T)0; gy[i] = (T)0; }
            continue;
        }
        int s0, s1;
        bool tall;
        cell_strips(c, b.R, b.lgR, s0, s1, tall);
        if (tall) {
            const double sc = c.ratio * g.inv_ba;
            for (int k = c.bxl; k <= c.bxh; ++k) {
                const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
                if (tx <= 0.0) continue;
                const double stx = sc * tx;
                const size_t rowi = (size_t)k * g.N;
                for (int q = c.byl; q <= c.byh; ++q) {
                    const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
                    if (ty <= 0.0) continue;
                    const double v = stx * ty;
                    if constexpr (FIXED)
                        atomicAdd(&Bm[rowi + q], (unsigned long long)__double2ull_rn(v * g.fix_scale));
                    else
                        unsafeAtomicAdd(&Bm[rowi + q], (T)v);
                }
            }
            for (int s = s0; s <= s1; ++s) b.bigflag[s] = 1u;
            b.big_list[atomicAdd(b.big_count, 1u)] = (unsigned)i;
            continue;
        }
        const vec4_t<T> rec = {x, y, w, h};
        const unsigned p0 = atomicAdd(&cur[s0], 1u);
        ent[p0] = rec;
        b.eidx[p0] = (unsigned)i;
        if (s1 != s0) {
            const unsigned p1 = atomicAdd(&cur[s1], 1u);
            ent[p1] = rec;
            b.eidx[p1] = (unsigned)i | kSecondStrip;
        }
    }
}

// Writes one accumulated strip value: rho = D0 + v (float modes) or the
// fixed-point accumulator (deterministic mode, folded by the row DCT).
template <typename T, bool FIXED>
__device__ __forceinline__ void flush_value(
    typename std::conditional<FIXED, unsigned long long, T>::type v,
    size_t gi, const T* __restrict__ d0n, T* __restrict__ dens,
    uint64_t* __restrict__ acc)
{
    if constexpr (FIXED) acc[gi] = (uint64_t)v;
    else dens[gi] = d0n[gi] + v;
}

// ---------------------------------------------------------------------------
// K4: accumulate one (strip, chunk) work item in LDS.
// ---------------------------------------------------------------------------
template <typename T, bool FIXED>
__global__ __launch_bounds__(kAccThreads) void k_strip_acc(
    Grid g, BinArgs b, const T* __restrict__ d0n, T* __restrict__ dens,
    uint64_t* __restrict__ acc)
{
    using A = typename std::conditional<FIXED, unsigned long long, T>::type;
    extern __shared__ __align__(16) unsigned char smem[];
    A* tile = reinterpret_cast<A*>(smem);
    const int w = blockIdx.x;
    if (w >= (int)*b.nitems) return;            // uniform across the group
    const unsigned item = b.items[w];
    const int s = (int)(item & 0xFFFFu);
    const int chunk = (int)(item >> 16);
    const int tid = threadIdx.x;
    const int R = b.R, N = g.N;
    const int RN = R * N;
    const int k0 = s * R, k1 = k0 + R - 1;
    // read before the barriers below: thread 0 clears it after the flush
    const bool single = b.nch[s] == 1u;
    const bool bf = b.bigflag[s] != 0u;
    for (int e = tid; e < RN; e += kAccThreads) tile[e] = (A)0;
    __syncthreads();

    const unsigned e0 = b.strip_off[s] + (unsigned)chunk * (unsigned)b.CH;
    const unsigned eend = b.strip_off[s + 1];
    const unsigned e1 = min(e0 + (unsigned)b.CH, eend);
    const vec4_t<T>* ent = reinterpret_cast<const vec4_t<T>*>(b.entries);
    for (unsigned e = e0 + tid; e < e1; e += kAccThreads) {
        const vec4_t<T> r = ent[e];
        CellSpan c;
        if (!cell_span((double)r.x, (double)r.y, (double)r.z, (double)r.w, g, c))
            continue;
        const double sc = c.ratio * g.inv_ba;
        const int ka = max(c.bxl, k0), kb = min(c.bxh, k1);
        for (int k = ka; k <= kb; ++k) {
            const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
            if (tx <= 0.0) continue;
            const double stx = sc * tx;
            A* trow = tile + (k - k0) * N;
            for (int q = c.byl; q <= c.byh; ++q) {
                const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
                if (ty <= 0.0) continue;
                const double v = stx * ty;
                if constexpr (FIXED)
                    atomicAdd(&trow[q], (unsigned long long)__double2ull_rn(v * g.fix_scale));
                else
                    atomicAdd(&trow[q], (T)v);
            }
        }
    }
    __syncthreads();

    const size_t gbase = (size_t)k0 * N;
    if (single) {
        A* Bm = reinterpret_cast<A*>(b.B);
        for (int e = tid; e < RN; e += kAccThreads) {
            A v = tile[e];
            if (bf) {
                v += Bm[gbase + e];
                Bm[gbase + e] = (A)0;
            }
            flush_value<T, FIXED>(v, gbase + e, d0n, dens, acc);
        }
        if (bf && tid == 0) b.bigflag[s] = 0u;
    } else {
        A* slot = reinterpret_cast<A*>(b.partial) + (size_t)w * RN;
        for (int e = tid; e < RN; e += kAccThreads) slot[e] = tile[e];
    }
}

// ---------------------------------------------------------------------------
// K4r: strips split into several chunks: rho = D0 + sum of partials (+B).
// ---------------------------------------------------------------------------
template <typename T, bool FIXED>
__global__ __launch_bounds__(kAccThreads) void k_strip_red(
    Grid g, BinArgs b, const T* __restrict__ d0n, T* __restrict__ dens,
    uint64_t* __restrict__ acc)
{
    using A = typename std::conditional<FIXED, unsigned long long, T>::type;
    const int s = blockIdx.x;
    const unsigned n = b.nch[s];
    if (n == 1u) return;
    const int tid = threadIdx.x;
    const int RN = b.R * g.N;
    const size_t gbase = (size_t)s * b.R * g.N;
    const unsigned w0 = b.item_start[s];
    const A* part = reinterpret_cast<const A*>(b.partial);
    A* Bm = reinterpret_cast<A*>(b.B);
    const bool bf = b.bigflag[s] != 0u;
    for (int e = tid; e < RN; e += kAccThreads) {
        A v = (A)0;
        for (unsigned c = 0; c < n; ++c) v += part[(size_t)(w0 + c) * RN + e];
        if (bf) {
            v += Bm[gbase + e];
            Bm[gbase + e] = (A)0;
        }
        flush_value<T, FIXED>(v, gbase + e, d0n, dens, acc);
    }
    __syncthreads();   // every thread has read bigflag[s]
    if (bf && tid == 0) b.bigflag[s] = 0u;
}

// ---------------------------------------------------------------------------
// G: per-cell field gather over the strip-sorted entries (each non-tall cell
// once, through its first strip) and the tall-cell list.
// ---------------------------------------------------------------------------
template <typename T>
__device__ __forceinline__ void gather_one(const CellSpan& c, const Grid& g,
                                           const T* __restrict__ fx,
                                           const T* __restrict__ fy,
                                           double& ax, double& ay)
{
    ax = 0.0;
    ay = 0.0;
    for (int k = c.bxl; k <= c.bxh; ++k) {
        const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
        if (tx <= 0.0) continue;
        const size_t row = (size_t)k * g.N;
        for (int q = c.byl; q <= c.byh; ++q) {
            const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, q);
            if (ty <= 0.0) continue;
            const double a = tx * ty;
            ax += a * (double)fx[row + q];
            ay += a * (double)fy[row + q];
        }
    }
    ax *= c.ratio;
    ay *= c.ratio;
}

template <typename T>
__global__ __launch_bounds__(256) void k_gather_bin(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, Grid g, BinArgs b,
    const T* __restrict__ fx, const T* __restrict__ fy, T* __restrict__ gx,
    T* __restrict__ gy)
{
    const unsigned total = b.strip_off[b.S];
    const unsigned nbig = *b.big_count;
    const unsigned stride = gridDim.x * blockDim.x;
    const vec4_t<T>* ent = reinterpret_cast<const vec4_t<T>*>(b.entries);
    for (unsigned e = blockIdx.x * blockDim.x + threadIdx.x; e < total; e += stride) {
        const unsigned id = b.eidx[e];
        if (id & kSecondStrip) continue;
        const vec4_t<T> r = ent[e];
        CellSpan c;
        double ax = 0.0, ay = 0.0;
        if (cell_span((double)r.x, (double)r.y, (double)r.z, (double)r.w, g, c))
            gather_one(c, g, fx, fy, ax, ay);
        gx[id] = (T)ax;
        gy[id] = (T)ay;
    }
    for (unsigned t = blockIdx.x * blockDim.x + threadIdx.x; t < nbig; t += stride) {
        const unsigned i = b.big_list[t];
        CellSpan c;
        double ax = 0.0, ay = 0.0;
        if (load_span(px, py, sx, sy, (int)i, g, c)) gather_one(c, g, fx, fy, ax, ay);
        gx[i] = (T)ax;
        gy[i] = (T)ay;
    }
}

}  // namespace dpep
