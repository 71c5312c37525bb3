// dpep_device.h -- device-side building blocks shared by the dpep kernels:
// vector types, the per-cell stretch/span/overlap geometry, and the
// LDS-resident mixed-radix Stockham FFT used by the spectral passes.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dpep {

// ---------------------------------------------------------------------------
// Grid description passed by value to every kernel.
// ---------------------------------------------------------------------------
struct Grid {
    int M, N;                 // bins along x (rows) and y (contiguous)
    double xl, yl, xh, yh;    // die
    double bsx, bsy;          // bin sizes
    double inv_ba;            // 1 / (bsx * bsy)
    double inv_bsx, inv_bsy;  // 1 / bsx, 1 / bsy
    double minw, minh;        // sqrt2 * bsx, sqrt2 * bsy (stretch floor)
    double fix_scale;         // 2^fix_exponent_of(nc_max, dtype): fixed-point scale
    int stretch;              // 1: DREAMPlace small-cell stretch
};

// Fixed-point scale of the density accumulators: each contribution
// ratio * tx * ty / bin_area is at most 1 (tx <= bsx, ty <= bsy, ratio <= 1),
// so a bin's sum is below nc_max and round(v * 2^f) with
// f = 62 - ceil(log2(nc_max)) (capped to [20, 52]) never overflows the
// unsigned 64-bit word.  fix_exponent() is shared by host and device.
__host__ __device__ inline int fix_exponent(int nc_max)
{
    int lg = 0;
    while (lg < 31 && (1ll << lg) < (long long)(nc_max > 1 ? nc_max : 1)) ++lg;
    int f = 62 - lg;
    return f > 52 ? 52 : (f < 20 ? 20 : f);
}

// The scale of a context: float32 contributions use 2^31 (never above
// fix_exponent for nc_max < 2^31), so round(v * 2^31) of a contribution
// v <= 1 fits 32 bits and converts in two instructions; the quantum 2^-31
// is far below float32's own rounding of v.  float64 keeps fix_exponent.
__host__ __device__ inline int fix_exponent_of(int nc_max, int elem_bytes)
{
    const int f = fix_exponent(nc_max);
    return elem_bytes == 4 && f > 31 ? 31 : f;
}

template <typename T> struct vec2;
template <> struct vec2<float> { using type = float2; };
template <> struct vec2<double> { using type = double2; };
template <typename T> using vec2_t = typename vec2<T>::type;

template <typename C>
__device__ __forceinline__ C cadd(C a, C b) { return C{a.x + b.x, a.y + b.y}; }
template <typename C>
__device__ __forceinline__ C csub(C a, C b) { return C{a.x - b.x, a.y - b.y}; }
template <typename C>
__device__ __forceinline__ C cmul(C a, C b)
{
    return C{a.x * b.x - a.y * b.y, a.x * b.y + a.y * b.x};
}
template <typename C>
__device__ __forceinline__ C cconj(C a) { return C{a.x, -a.y}; }

// Reciprocal: the hardware's (about 1 ulp) for float, exact for double.
__device__ __forceinline__ float fast_rcp(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ double fast_rcp(double x) { return 1.0 / x; }
// multiply by -i (forward) or +i (inverse)
template <bool INV, typename C>
__device__ __forceinline__ C cmul_mi(C a)
{
    return INV ? C{-a.y, a.x} : C{a.y, -a.x};
}

// ---------------------------------------------------------------------------
// XCD-aware block numbering.  MI355X dispatches workgroup b to XCD b % 8;
// this returns a logical index such that logical blocks
// [x * n/8, (x+1) * n/8) all run on XCD x, so consecutive logical blocks
// share that XCD's L2.  Blocks beyond the largest multiple of 8 keep their
// index.  A bijection on [0, n) whatever the hardware mapping is.
// ---------------------------------------------------------------------------
constexpr int kNumXcd = 8;

__device__ __forceinline__ unsigned xcd_logical_block(unsigned b, unsigned n)
{
    const unsigned per = n / kNumXcd;
    if (b >= per * kNumXcd) return b;
    return (b % kNumXcd) * per + b / kNumXcd;
}

// ---------------------------------------------------------------------------
// Cell geometry: stretch, bin span, 1-D overlap.  Evaluated in float64 with
// contraction disabled so the GPU reproduces the float64 oracle's spans.
// ---------------------------------------------------------------------------
struct CellSpan {
    double x, y, w, h;      // stretched corner and extents
    double sx, sy;          // original extents
    int bxl, bxh, byl, byh;
    // area ratio sx*sy / (w*h) (1 without stretch); a float64 division, so
    // only the paths that need it (tall cells) evaluate it
    __device__ __forceinline__ double ratio() const
    {
        return (sx == w && sy == h) ? 1.0 : (sx * sy) / (w * h);
    }
};

// Index of the bin containing v (origin + k*bs <= v < origin + (k+1)*bs for
// the edges as computed in float64): reciprocal-multiply estimate corrected
// against the exact edges (the reference's correct_bin_idx idea,
// kernels/v4_compute.cpp:91-102); no float64 division.
__device__ __forceinline__ double floor_bin(double v, double origin,
                                            double bs, double inv)
{
#pragma clang fp contract(off)
    double k = floor((v - origin) * inv);
    if (origin + k * bs > v) k -= 1.0;
    else if (origin + (k + 1.0) * bs <= v) k += 1.0;
    return k;
}

__device__ __forceinline__ bool cell_span(double px, double py, double sx,
                                          double sy, const Grid& g,
                                          CellSpan& c)
{
#pragma clang fp contract(off)
    if (!(isfinite(px) && isfinite(py) && isfinite(sx) && isfinite(sy)))
        return false;
    if (!(sx > 0.0 && sy > 0.0)) return false;
    double w = sx, h = sy, x = px, y = py;
    if (g.stretch) {
        w = sx > g.minw ? sx : g.minw;
        h = sy > g.minh ? sy : g.minh;
        x = px + 0.5 * (sx - w);
        y = py + 0.5 * (sy - h);
    }
    double fxl = floor_bin(x, g.xl, g.bsx, g.inv_bsx);
    double fxh = floor_bin(x + w, g.xl, g.bsx, g.inv_bsx);
    double fyl = floor_bin(y, g.yl, g.bsy, g.inv_bsy);
    double fyh = floor_bin(y + h, g.yl, g.bsy, g.inv_bsy);
    fxl = fxl < 0.0 ? 0.0 : fxl;
    fyl = fyl < 0.0 ? 0.0 : fyl;
    fxh = fxh > (double)(g.M - 1) ? (double)(g.M - 1) : fxh;
    fyh = fyh > (double)(g.N - 1) ? (double)(g.N - 1) : fyh;
    if (fxl > fxh || fyl > fyh) return false;
    c.x = x; c.y = y; c.w = w; c.h = h; c.sx = sx; c.sy = sy;
    c.bxl = (int)fxl; c.bxh = (int)fxh;
    c.byl = (int)fyl; c.byh = (int)fyh;
    return true;
}

__device__ __forceinline__ double overlap_1d(double lo, double ext,
                                             double origin, double bs, int k)
{
#pragma clang fp contract(off)
    const double bl = origin + k * bs;
    const double br = origin + (k + 1) * bs;
    const double hi = lo + ext;
    const double a = lo > bl ? lo : bl;
    const double b = hi < br ? hi : br;
    const double o = b - a;
    return o > 0.0 ? o : 0.0;
}

// ---------------------------------------------------------------------------
// LDS FFT.  One complex FFT of length L is computed by TPF = L / E threads,
// each holding E elements per stage (E = min(16, L) unless a pass picks a
// smaller power of two).  Stages are radix E while the remaining factor
// allows, then one smaller radix (Stockham autosort: natural order in and
// out, in place through registers between barriers).
// ---------------------------------------------------------------------------
__host__ __device__ constexpr int fft_e(int L) { return L < 16 ? L : 16; }
__host__ __device__ constexpr int lds_pad(int e) { return e + (e >> 5); }
// Row stride of one FFT's buffer: the padded length plus a skew of 8
// elements, so rows of consecutive FFTs start 8 banks-pairs apart and the
// tile loads/stores that touch one element of several rows do not collide.
__host__ __device__ constexpr int lds_len(int L) { return L + (L >> 5) + 8; }

// 16-byte vector of T (global loads and stores of the spectral passes).
template <typename T, int V = 16 / (int)sizeof(T)>
struct alignas(16) pack {
    T v[V];
};

// Makhoul's even/odd-reversed ordering: x[m] sits at position perm(m).
template <int L>
__device__ __forceinline__ int makhoul_pos(int m)
{
    return (m & 1) ? (L - 1 - (m >> 1)) : (m >> 1);
}

// In-register DFTs of size 2, 4, 8, 16 (natural order in and out).
// Forward uses W = exp(-2 pi i / R); INV conjugates.
template <bool INV, typename C>
__device__ __forceinline__ void dft2(C& a, C& b)
{
    C t = csub(a, b);
    a = cadd(a, b);
    b = t;
}

template <bool INV, typename C>
__device__ __forceinline__ void dft4(C& x0, C& x1, C& x2, C& x3)
{
    C a = cadd(x0, x2), b = csub(x0, x2);
    C c = cadd(x1, x3), d = cmul_mi<INV>(csub(x1, x3));
    x0 = cadd(a, c);
    x2 = csub(a, c);
    x1 = cadd(b, d);
    x3 = csub(b, d);
}

// twiddle W_R^k for R in {8, 16}; k <= 9
template <typename T, bool INV>
__device__ __forceinline__ vec2_t<T> w16(int k)
{
    using C = vec2_t<T>;
    const T c1 = (T)0.92387953251128675613, s1 = (T)0.38268343236508977173;
    const T c2 = (T)0.70710678118654752440;
    C w;
    switch (k) {
    case 0: w = C{(T)1, (T)0}; break;
    case 1: w = C{c1, -s1}; break;
    case 2: w = C{c2, -c2}; break;
    case 3: w = C{s1, -c1}; break;
    case 4: w = C{(T)0, (T)-1}; break;
    case 5: w = C{-s1, -c1}; break;
    case 6: w = C{-c2, -c2}; break;
    case 7: w = C{-c1, -s1}; break;
    case 8: w = C{(T)-1, (T)0}; break;
    default: w = C{-c1, s1}; break;
    }
    if (INV) w.y = -w.y;
    return w;
}

template <typename T, bool INV>
__device__ __forceinline__ void dft8(vec2_t<T>* v)
{
    using C = vec2_t<T>;
    // n = 2 n1 + n2, k = k1 + 4 k2
    C e0 = v[0], e1 = v[2], e2 = v[4], e3 = v[6];
    C o0 = v[1], o1 = v[3], o2 = v[5], o3 = v[7];
    dft4<INV>(e0, e1, e2, e3);
    dft4<INV>(o0, o1, o2, o3);
    o1 = cmul(o1, w16<T, INV>(2));   // W8^1 = W16^2
    o2 = cmul_mi<INV>(o2);           // W8^2
    o3 = cmul(o3, w16<T, INV>(6));   // W8^3 = W16^6
    v[0] = cadd(e0, o0); v[4] = csub(e0, o0);
    v[1] = cadd(e1, o1); v[5] = csub(e1, o1);
    v[2] = cadd(e2, o2); v[6] = csub(e2, o2);
    v[3] = cadd(e3, o3); v[7] = csub(e3, o3);
}

template <typename T, bool INV>
__device__ __forceinline__ void dft16(vec2_t<T>* v)
{
    using C = vec2_t<T>;
    // n = 4 n1 + n2, k = k1 + 4 k2
    C y[4][4];
#pragma unroll
    for (int n2 = 0; n2 < 4; ++n2) {
        C a = v[n2], b = v[n2 + 4], c = v[n2 + 8], d = v[n2 + 12];
        dft4<INV>(a, b, c, d);
        y[n2][0] = a; y[n2][1] = b; y[n2][2] = c; y[n2][3] = d;
    }
#pragma unroll
    for (int n2 = 1; n2 < 4; ++n2)
#pragma unroll
        for (int k1 = 1; k1 < 4; ++k1)
            y[n2][k1] = cmul(y[n2][k1], w16<T, INV>(n2 * k1));
#pragma unroll
    for (int k1 = 0; k1 < 4; ++k1) {
        C a = y[0][k1], b = y[1][k1], c = y[2][k1], d = y[3][k1];
        dft4<INV>(a, b, c, d);
        v[k1] = a; v[k1 + 4] = b; v[k1 + 8] = c; v[k1 + 12] = d;
    }
}

template <typename T, int R, bool INV>
__device__ __forceinline__ void dft_r(vec2_t<T>* v)
{
    if constexpr (R == 2) dft2<INV>(v[0], v[1]);
    else if constexpr (R == 4) dft4<INV>(v[0], v[1], v[2], v[3]);
    else if constexpr (R == 8) dft8<T, INV>(v);
    else dft16<T, INV>(v);
}

// Radix of the stage that starts at sub-length NS when each thread holds E
// elements: E while the remaining factor allows, then the remainder.
template <int L, int NS, int E>
__host__ __device__ constexpr int fft_radix()
{
    return L / NS >= E ? E : L / NS;
}

__host__ __device__ constexpr int ilog2c(int x) { return x <= 1 ? 0 : 1 + ilog2c(x / 2); }

// Twiddle-table reads of one thread in the stages from sub-length NS on:
// E/R butterflies per stage, log2(R) reads each (the power-of-two exponents;
// the others are products of them), none in the first stage.
template <int L, int NS, int E>
__host__ __device__ constexpr int fft_tw_count()
{
    if constexpr (NS >= L) {
        return 0;
    } else {
        constexpr int R = fft_radix<L, NS, E>();
        return (NS > 1 ? (E / R) * ilog2c(R) : 0) + fft_tw_count<L, NS * R, E>();
    }
}

template <int L, int NS, int E>
__host__ __device__ constexpr int fft_tw_next(int off)
{
    return off + (NS > 1 ? (E / fft_radix<L, NS, E>()) * ilog2c(fft_radix<L, NS, E>()) : 0);
}

// Every twiddle a thread's stages read, loaded into registers up front: the
// loads then overlap the pass's data loads instead of each stage waiting on
// its own between the LDS reads and the butterflies.  Entries are the
// forward twiddles exp(-2 pi i m / L); inverse stages conjugate them.
template <typename T, int L, int E = fft_e(L)>
struct FftTw {
    static constexpr int N = fft_tw_count<L, 1, E>();
    vec2_t<T> w[N > 0 ? N : 1];
};

// The twiddles of the stage at sub-length NS, entries [OFF, OFF + count).
template <typename T, int L, int E, int NS, int OFF>
__device__ __forceinline__ void fft_tw_stage(FftTw<T, L, E>& p, int t,
                                             const vec2_t<T>* __restrict__ tw)
{
    constexpr int R = fft_radix<L, NS, E>();
    constexpr int TPF = L / E, NB = E / R, LG = ilog2c(R);
    if constexpr (NS > 1) {
        constexpr int S = L / (NS * R);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int k = (t + TPF * b) % NS;
#pragma unroll
            for (int q = 0; q < LG; ++q) p.w[OFF + b * LG + q] = tw[(1 << q) * k * S];
        }
    }
}

template <typename T, int L, int E, int NS = 1, int OFF = 0>
__device__ __forceinline__ void fft_tw_fetch(FftTw<T, L, E>& p, int t,
                                             const vec2_t<T>* __restrict__ tw)
{
    if constexpr (NS < L) {
        fft_tw_stage<T, L, E, NS, OFF>(p, t, tw);
        fft_tw_fetch<T, L, E, NS * fft_radix<L, NS, E>(), fft_tw_next<L, NS, E>(OFF)>(p, t, tw);
    }
}

// One Stockham stage over the FFT held in `buf` (LDS, padded indexing).
// t: this thread's index within the FFT's TPF = L / E threads.  pw: this
// stage's twiddles in the thread's FftTw.  act = false: a thread of the
// workgroup that holds no FFT; it only takes part in the barriers.
template <typename T, int L, int E, int R, int NS, bool INV>
__device__ __forceinline__ void fft_stage(vec2_t<T>* buf, int t,
                                          const vec2_t<T>* pw, bool act)
{
    using C = vec2_t<T>;
    constexpr int TPF = L / E;
    constexpr int NB = E / R;
    constexpr int LG = ilog2c(R);
    C v[NB][R];
    if (act) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int j = t + TPF * b;
#pragma unroll
        for (int r = 0; r < R; ++r) v[b][r] = buf[lds_pad(j + r * (L / R))];
    }
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        if constexpr (NS > 1) {
            // W^(r k S) for r < R (k = j mod NS, S = L / (NS R)): the
            // power-of-two exponents come from the table, the others are
            // products of at most three of them
            C w[R];
#pragma unroll
            for (int r = 1; r < R; ++r) {
                const int hi = 1 << (31 - __builtin_clz(r));
                if (hi == r) {
                    w[r] = pw[b * LG + ilog2c(r)];
                    if (INV) w[r].y = -w[r].y;
                } else {
                    w[r] = cmul(w[hi], w[r - hi]);
                }
            }
#pragma unroll
            for (int r = 1; r < R; ++r) v[b][r] = cmul(v[b][r], w[r]);
        }
        dft_r<T, R, INV>(v[b]);
    }
    }
    __syncthreads();
    if (act) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int j = t + TPF * b;
        const int k = j % NS;
        const int base = (j / NS) * NS * R + k;
#pragma unroll
        for (int r = 0; r < R; ++r) buf[lds_pad(base + r * NS)] = v[b][r];
    }
    }
    __syncthreads();
}

template <typename T, int L, int E, int NS, int OFF, bool INV>
__device__ __forceinline__ void fft_stages(vec2_t<T>* buf, int t,
                                           const FftTw<T, L, E>& p, bool act)
{
    if constexpr (NS < L) {
        constexpr int R = fft_radix<L, NS, E>();
        fft_stage<T, L, E, R, NS, INV>(buf, t, p.w + OFF, act);
        fft_stages<T, L, E, NS * R, fft_tw_next<L, NS, E>(OFF), INV>(buf, t, p, act);
    }
}

// Stages that read their own twiddles from the table as they start (fewer
// registers held than a full FftTw; each stage waits on its reads).
template <typename T, int L, int E, int NS, int OFF, bool INV>
__device__ __forceinline__ void fft_stages_tw(vec2_t<T>* buf, int t,
                                              const vec2_t<T>* __restrict__ tw, bool act)
{
    if constexpr (NS < L) {
        constexpr int R = fft_radix<L, NS, E>();
        FftTw<T, L, E> p;
        fft_tw_stage<T, L, E, NS, OFF>(p, t, tw);
        fft_stage<T, L, E, R, NS, INV>(buf, t, p.w + OFF, act);
        fft_stages_tw<T, L, E, NS * R, fft_tw_next<L, NS, E>(OFF), INV>(buf, t, tw, act);
    }
}

// Full in-place FFT with the thread's twiddles already in registers; caller
// must __syncthreads() before (data in LDS).  Every thread of the workgroup
// calls it (the stages hold barriers); threads with act = false hold no FFT.
template <typename T, int L, bool INV, int E>
__device__ __forceinline__ void fft_lds(vec2_t<T>* buf, int t, const FftTw<T, L, E>& p,
                                        bool act = true)
{
    fft_stages<T, L, E, 1, 0, INV>(buf, t, p, act);
}

// The same, each stage reading its twiddles from tw (exp(-2 pi i m / L)).
template <typename T, int L, bool INV, int E = fft_e(L)>
__device__ __forceinline__ void fft_lds(vec2_t<T>* buf, int t,
                                        const vec2_t<T>* __restrict__ tw,
                                        bool act = true)
{
    fft_stages_tw<T, L, E, 1, 0, INV>(buf, t, tw, act);
}

}  // namespace dpep
