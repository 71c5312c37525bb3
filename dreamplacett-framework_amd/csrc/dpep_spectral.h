// dpep_spectral.h -- kernels of the DCT-based Poisson solve (three row passes).
//
// Maths (reference host/density_scatter_ttnn_server_host.cpp:124-181,
// :251-263, :281-295):
//   A  = C_M rho C_N^T,          C_K[k,n] = (2/K) cos(pi k (n+1/2) / K)
//   fx = (2 S_M)(A . Wx) I_N^T,  fy = (2 I_M)(A . Wy) S_N^T
//   phi = I_M (A / D) I_N^T      (potential; not in the reference)
// with I_K[k,0] = 1, I_K[k,n>0] = 2 cos(pi n (k+1/2)/K),
// S_K[k,n] = sin(pi n (k+1/2)/K), w_u = 2 pi u / M,
// w_v = 2 pi v / N * bsx / bsy, D = w_u^2 + w_v^2, Wx = w_u / 2D,
// Wy = w_v / 2D, and all weights zero at (0,0).
//
// Each 1-D transform is one complex FFT of length L on two packed real
// lines (Makhoul's even/odd reordering):
//   DCT-II:  z = v1 + i v2, Z = FFT(z), X[k] = Re(e^{-i pi k/2L} V[k]) with
//            V1 = (Z[k] + conj Z[L-k]) / 2, V2 = -i (Z[k] - conj Z[L-k]) / 2,
//            and X[L-k] = -Im(e^{-i pi k/2L} V[k]).
//   I_K:     V[k] = e^{i pi k/2L} (X[k] - i X[L-k]), z = IFFT(V) (unscaled),
//            y[2n] = z[n], y[2n+1] = z[L-1-n].
//   S_K:     S(X)[n] = (-1)^n / 2 * I(X')[n], X'[k] = X[L-k], X'[0] = 0.
// A thread owns the index pair {s, L-s} (s = 0 owns {0, L/2}) so the pre- and
// post-processing never crosses threads.
//
// The potential needs no transform of its own along x: w_v depends only on
// the column v, so for v >= 1
//   Up[:, v] = I_M (A[:, v] / D[:, v]) = Uy[:, v] / w_v(v)
// with Uy = 2 I_M (A . Wy) as stored.  Column 0 of Uy would be zero
// (w_v(0) = 0) and the S-type transform that turns Uy into fy never reads
// it, so P2 stores w_v(1) Up[:, 0] there instead: the weight of column 1,
// so the two columns that share one complex FFT keep similar magnitudes
// (the FFT's rounding is relative to the pair, not to each column).
//
// Passes and HBM traffic (MN = M*N elements):
//   P1  (in k_strip_acc, dpep_bin.h): each strip's rows, already in LDS after
//       the density flush -> T tiled                             write MN
//   P2  k_col_pass: T rows (along x)    -> Ux, Uy   tiled      read MN, write 2MN
//                   (DCT-II, weights, two inverse transforms)
//   P3  k_row_inv : Ux, Uy rows (y)     -> fx, fy, phi         read 2MN, write 3MN
// T is stored in tiles of TXT x TV elements and Ux, Uy in tiles of TX x TV
// (TV = 2 fpw(M), the columns of a P2 workgroup; TX = 2 fpw(N), the rows of
// a P3 type-B workgroup; TXT >= the rows of a strip, the rows P1 writes at
// once): every global access is a run of whole tiles while P1 and P2 write
// "transposed" relative to the rows they process.
#pragma once

#include "dpep_internal.h"

namespace dpep {

// FFTs held by one workgroup of the length-L passes.  Two at L = 2048 (not
// four): twice the workgroups, two of them per CU, measured 2-3 us faster
// per pass at 2048 x 2048.  Two at L <= 512 as well (with 8 elements per
// thread, below): a 512-point pass has only N / 2F workgroups to spread
// over the CUs.
template <typename T>
__host__ __device__ constexpr int fpw(int L)
{
    return sizeof(T) == 4 ? ((L <= 1024 && L > 512) ? 4 : 2) : 2;
}

// Elements per thread of the passes at L <= 512: 8, so each FFT has twice
// the threads (the passes are latency-bound at these sizes).
template <typename T>
__host__ __device__ constexpr int small_e(int L)
{
    return (L <= 512 && L >= 8) ? 8 : fft_e(L);
}

// Elements per thread of the FFTs of the column pass (P2) and of the row
// pass (P3).  A column-pass workgroup holds only F = fpw FFTs and there are
// N / 2F of them, so fewer elements per thread (more threads per FFT) is
// how the pass gets more waves in flight.
template <typename T>
__host__ __device__ constexpr int col_e(int L)
{
    return small_e<T>(L);
}

template <typename T>
__host__ __device__ constexpr int row_e(int L)
{
    return small_e<T>(L);
}

template <typename T>
__host__ __device__ constexpr int col_threads(int L)
{
    return fpw<T>(L) * (L / col_e<T>(L));
}

template <typename T>
__host__ __device__ constexpr int row_threads(int L)
{
    return fpw<T>(L) * (L / row_e<T>(L));
}

// Tile extents of a square L x L grid, as make_spectral_args sets them.
// The passes compiled for square grids (kSq) take them as constants, so their
// tile offsets become constant shifts and immediate offsets instead of
// shifts by amounts loaded at run time.
template <typename T, int L>
__host__ __device__ constexpr Tiles square_tiles()
{
    Tiles t{};
    t.TX = 2 * fpw<T>(L);
    t.TV = 2 * fpw<T>(L);
    t.TXT = t_tile_rows(strip_rows(L), t.TX, t.TV, sizeof(T), L);
    return t;
}

// Square grids of at least kSquareMin bins a side run the passes compiled
// with their tile extents as constants; other grids, and smaller squares (one
// form fewer to compile per length), read them from the args.
constexpr int kSquareMin = 512;

template <typename T, int L>
inline bool square_form(const SpectralArgs& a)
{
    constexpr Tiles kT = square_tiles<T, L>();
    return L >= kSquareMin && a.M == L && a.N == L && a.tiles.TX == kT.TX &&
           a.tiles.TV == kT.TV && a.tiles.TXT == kT.TXT;
}

template <typename T>
__device__ __forceinline__ T& comp(vec2_t<T>& c, int which)
{
    return which ? c.y : c.x;
}

template <typename T>
__device__ __forceinline__ T comp_of(const vec2_t<T>& c, int which)
{
    return which ? c.y : c.x;
}

// Global accesses of the passes move 16-byte vectors: V elements each, NV
// vectors per thread for a block of `elems` elements.
template <typename T>
constexpr int kVec = 16 / (int)sizeof(T);

// 1 / D(u, v) = 1 / (w_u^2 + w_v^2), zero at (0, 0).
template <typename T>
__device__ __forceinline__ T inv_d(int u, int v, const SpectralArgs& a)
{
    if (u == 0 && v == 0) return (T)0;
    const T wu = (T)u * (T)a.wu_step;
    const T wv = (T)v * (T)a.wv_step;
    return fast_rcp(wu * wu + wv * wv);
}

// The post-processing twiddle of slot s: post[s], or post[L/2] for s = 0
// (the slot that owns {0, L/2}).  post[k] = exp(-i pi k / 2L).
template <typename T, int L>
__device__ __forceinline__ vec2_t<T> post_of(const vec2_t<T>* __restrict__ post, int s)
{
    return post[s == 0 ? L / 2 : s];
}

// Forward post-processing of slot s for two packed rows: returns X at k and m
// (x component = first row, y = second row).
template <typename T, int L>
__device__ __forceinline__ void dct_post(const vec2_t<T>* buf, int s,
                                         vec2_t<T> pc, T scale, vec2_t<T>& Xk,
                                         vec2_t<T>& Xm)
{
    using C = vec2_t<T>;
    if (s == 0) {
        const C z0 = buf[0];
        const C zh = buf[lds_pad(L / 2)];
        const T c45 = pc.x;
        Xk = C{z0.x * scale, z0.y * scale};
        Xm = C{zh.x * c45 * scale, zh.y * c45 * scale};
    } else {
        const C za = buf[lds_pad(s)];
        const C zb = buf[lds_pad(L - s)];
        const C v1 = C{(T)0.5 * (za.x + zb.x), (T)0.5 * (za.y - zb.y)};
        const C v2 = C{(T)0.5 * (za.y + zb.y), (T)-0.5 * (za.x - zb.x)};
        const C w1 = cmul(pc, v1);
        const C w2 = cmul(pc, v2);
        Xk = C{w1.x * scale, w2.x * scale};
        Xm = C{-w1.y * scale, -w2.y * scale};
    }
}

// Inverse pre-processing of slot s for one real spectrum given X[k], X[m]
// (k = s, m = L - s; for s = 0: k = 0, m = L/2).  rev selects X'[k] = X[L-k].
template <typename T, int L>
__device__ __forceinline__ void inv_pre(int s, T xk, T xm, bool rev, vec2_t<T> c,
                                        vec2_t<T>& Vk, vec2_t<T>& Vm)
{
    using C = vec2_t<T>;
    if (s == 0) {
        Vk = C{rev ? (T)0 : xk, (T)0};
        // conj(c) * (xm - i xm)
        Vm = C{c.x * xm - c.y * xm, -c.x * xm - c.y * xm};
    } else {
        const T a = rev ? xm : xk;
        const T b = rev ? xk : xm;
        // conj(c) * (a - i b)
        Vk = C{c.x * a - c.y * b, -c.x * b - c.y * a};
        // i * c * (b - i a) = i*(c.x b + c.y a) + ... expand:
        // c*(b - i a) = (c.x b + c.y a) + i (c.y b - c.x a); times i:
        Vm = C{-(c.y * b - c.x * a), c.x * b + c.y * a};
    }
}

template <typename T>
__device__ __forceinline__ vec2_t<T> pack2(vec2_t<T> v1, vec2_t<T> v2)
{
    // v1 + i v2
    return vec2_t<T>{v1.x - v2.y, v1.y + v2.x};
}

// ---------------------------------------------------------------------------
// P2: per pair of v-rows of T: DCT-II along x, spectral weights, then the
// three inverse transforms along x; writes Ux, Uy and Up (Up over T) tiled.
// ---------------------------------------------------------------------------
template <typename T, int L, int F, bool kSq>
__global__ __launch_bounds__(col_threads<T>(L)) void k_col_pass(
    SpectralArgs a, const T* __restrict__ Tt, T* __restrict__ Ux,
    T* __restrict__ Uy)
{
    constexpr Tiles kT = square_tiles<T, L>();
    using C = vec2_t<T>;
    constexpr int E = col_e<T>(L), TPF = L / E, NT = F * TPF, LP = lds_len(L);
    constexpr int TV = 2 * F;
    extern __shared__ __align__(16) unsigned char smem[];
    C* sb = reinterpret_cast<C*>(smem);
    const int tid = threadIdx.x, f = tid / TPF, t = tid % TPF;
    C* buf = sb + f * LP;
    const int TX = kSq ? kT.TX : a.tiles.TX;      // Ux, Uy tiles (stores)
    const int lgTX = __builtin_ctz(TX);
    const int TXT = kSq ? kT.TXT : a.tiles.TXT;   // T tiles (loads)
    const int lgTXT = __builtin_ctz(TXT);
    // tile offsets by shifts: every tile extent and N are powers of two
    const int lgNBV = __builtin_ctz(kSq ? L : a.N) - __builtin_ctz(TV);
    const int b2 = blockIdx.x;
    const int v0 = b2 * TV;
    constexpr int lgTV = __builtin_ctz(TV);
    const int tile_elems = TX * TV;
    const int lgTE = lgTX + lgTV;

    // load the tiles (bx, b2) of T for every bx: each vector holds V
    // consecutive columns v (pairs of them form the complex input of one
    // FFT) of one x
    constexpr int V = kVec<T>, NV = L * TV / (NT * V);
    static_assert(NV * NT * V == L * TV && V % 2 == 0 && TV % V == 0, "P2 vector split");
    const C* post = reinterpret_cast<const C*>(a.postM);
    C pst[E / 2];           // post-processing twiddles of the thread's slots
    FftTw<T, L, E> twp;     // and its FFT twiddles (forward; inverse conjugates)
    {
        const int tile_t = TXT * TV;
        const int lgTET = lgTXT + lgTV;
        pack<T> r[NV];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e0 = (tid + i * NT) * V;
            const int bx = e0 >> lgTET;
            const int w = e0 & (tile_t - 1);
            r[i] = *reinterpret_cast<const pack<T>*>(
                Tt + (((((unsigned)bx << lgNBV) + (unsigned)b2) << lgTET) + (unsigned)w));
        }
#pragma unroll
        for (int i = 0; i < E / 2; ++i) pst[i] = post_of<T, L>(post, t + TPF * i);
        fft_tw_fetch<T, L, E>(twp, t, reinterpret_cast<const C*>(a.twM));
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e0 = (tid + i * NT) * V;
            const int bx = e0 >> lgTET;
            const int w = e0 & (tile_t - 1);
            const int x = (bx << lgTXT) + (w >> lgTV);
            const int v_in = w & (TV - 1);
            const int px = lds_pad(makhoul_pos<L>(x));
#pragma unroll
            for (int q = 0; q < V; q += 2)
                sb[((v_in + q) >> 1) * LP + px] = C{r[i].v[q], r[i].v[q + 1]};
        }
    }
    __syncthreads();
    fft_lds<T, L, false>(buf, t, twp);

    const T scale = (T)2 / (T)L;
    C Ak[E / 2], Am[E / 2];
#pragma unroll
    for (int i = 0; i < E / 2; ++i)
        dct_post<T, L>(buf, t + TPF * i, pst[i], scale, Ak[i], Am[i]);

    // A / D once (zero at (0,0)); the rounds then only scale by w_u / 2
    // (a function of the row k), w_v / 2 (of the column) or 1, so nothing
    // per-element has to stay live across the rounds.
    const int v1 = v0 + 2 * f, v2 = v1 + 1;
#pragma unroll
    for (int i = 0; i < E / 2; ++i) {
        const int s = t + TPF * i;
        const int k = s, m = (s == 0) ? L / 2 : L - s;
        Ak[i].x *= inv_d<T>(k, v1, a);
        Ak[i].y *= inv_d<T>(k, v2, a);
        Am[i].x *= inv_d<T>(m, v1, a);
        Am[i].y *= inv_d<T>(m, v2, a);
    }
    const T hu = (T)0.5 * (T)a.wu_step;
    const T hv1 = (T)0.5 * (T)v1 * (T)a.wv_step, hv2 = (T)0.5 * (T)v2 * (T)a.wv_step;
    // column 0: w_v(1) I_M (A / D) in the otherwise-zero column of Uy
    const T hv1z = v1 == 0 ? (T)0.5 * (T)a.wv_step : hv1;
    for (int round = 0; round < 2; ++round) {
        const bool rev = (round == 0);
        C Vk[E / 2], Vm[E / 2];
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            const int k = s, m = (s == 0) ? L / 2 : L - s;
            T w1k, w1m, w2k, w2m;
            if (round == 0) {
                w1k = w2k = (T)k * hu;
                w1m = w2m = (T)m * hu;
            } else {
                w1k = w1m = hv1z;
                w2k = w2m = hv2;
            }
            const T b1k = Ak[i].x * w1k;
            const T b1m = Am[i].x * w1m;
            const T b2k = Ak[i].y * w2k;
            const T b2m = Am[i].y * w2m;
            C p1k, p1m, p2k, p2m;
            inv_pre<T, L>(s, b1k, b1m, rev, pst[i], p1k, p1m);
            inv_pre<T, L>(s, b2k, b2m, rev, pst[i], p2k, p2m);
            Vk[i] = pack2<T>(p1k, p2k);
            Vm[i] = pack2<T>(p1m, p2m);
        }
        __syncthreads();   // previous round's readers of buf are done
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            buf[lds_pad(s)] = Vk[i];
            buf[lds_pad(s == 0 ? L / 2 : L - s)] = Vm[i];
        }
        __syncthreads();
        fft_lds<T, L, true>(buf, t, twp);

        T* dst = round == 0 ? Ux : Uy;
        const T rscale = round == 1 ? (T)2 : (T)1;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int e0 = (tid + i * NT) * V;
            const int bx = e0 >> lgTE;
            const int w = e0 & (tile_elems - 1);
            const int x = (bx << lgTX) + (w >> lgTV);
            const int v_in = w & (TV - 1);
            const int px = lds_pad(makhoul_pos<L>(x));
            const T sc = (round == 0 && (x & 1)) ? -rscale : rscale;
            pack<T> o;
#pragma unroll
            for (int q = 0; q < V; q += 2) {
                const C z = sb[((v_in + q) >> 1) * LP + px];
                o.v[q] = z.x * sc;
                o.v[q + 1] = z.y * sc;
            }
            *reinterpret_cast<pack<T>*>(
                dst + (((((unsigned)bx << lgNBV) + (unsigned)b2) << lgTE) + (unsigned)w)) = o;
        }
    }
}

// ---------------------------------------------------------------------------
// P3: inverse transforms along y.  Rows come in groups of TX = 2F; a group
// has two type-A blocks (F rows each, one row per FFT packing (Ux row,
// reversed Uy row) -> fx and fy) and, with the potential, one type-B block
// (two rows per FFT of Up = Uy / w_v, column 0 = Uy / w_v(1) -> phi).  The blocks
// of a group are consecutive in XCD-logical order, so the Uy rows the
// type-B block re-reads are still in that XCD's L2.
// ---------------------------------------------------------------------------
// Waves per SIMD P3 is compiled for: four at float32 (128 VGPRs, which the
// pass fits), so a CU holds the four workgroups of 2048-point FFTs its LDS
// allows; float64 takes what it needs.
template <typename T>
__host__ __device__ constexpr int row_waves()
{
    return sizeof(T) == 4 ? 4 : 1;
}

template <typename T, int L, int F, bool kSq>
__global__ __launch_bounds__(row_threads<T>(L), row_waves<T>()) void k_row_inv(
    SpectralArgs a, const T* __restrict__ Ux, const T* __restrict__ Uy,
    T* __restrict__ fx, T* __restrict__ fy, T* __restrict__ phi)
{
    constexpr Tiles kT = square_tiles<T, L>();
    using C = vec2_t<T>;
    constexpr int E = row_e<T>(L), TPF = L / E, NT = F * TPF, LP = lds_len(L);
    constexpr int TX = 2 * F;
    extern __shared__ __align__(16) unsigned char smem[];
    C* sb = reinterpret_cast<C*>(smem);
    const int tid = threadIdx.x, f = tid / TPF, t = tid % TPF;
    C* buf = sb + f * LP;
    const int TV = kSq ? kT.TV : a.tiles.TV;
    const int lgTV = __builtin_ctz(TV);
    const int lgNBV = __builtin_ctz(L) - lgTV;
    const C* post = reinterpret_cast<const C*>(a.postN);
    const C* tw = reinterpret_cast<const C*>(a.twN);
    const int per_group = a.potential ? 3 : 2;
    const int lb = (int)xcd_logical_block(blockIdx.x, gridDim.x);
    const int grp = lb / per_group, role = lb % per_group;
    // every twiddle the thread needs, loaded before the rows so the latency
    // of these small (cache-resident) tables overlaps theirs
    C pst[E / 2];
#pragma unroll
    for (int i = 0; i < E / 2; ++i) pst[i] = post_of<T, L>(post, t + TPF * i);
    FftTw<T, L, E> twp;
    fft_tw_fetch<T, L, E>(twp, t, tw);

    if (role < 2) {
        const int ab = 2 * grp + role;
        const int x0 = ab * F;
        const int bx = ab >> 1, half = ab & 1;
        const int chunk = F * TV;
        const int lgCH = __builtin_ctz(F) + lgTV;
        constexpr int V = kVec<T>, NVA = F * L / (NT * V);
        static_assert(NVA * NT * V == F * L, "P3 vector split");
        {
            pack<T> rx[NVA], ry[NVA];
#pragma unroll
            for (int i = 0; i < NVA; ++i) {
                const int e0 = (tid + i * NT) * V;
                const int bv = e0 >> lgCH;
                const int w = e0 & (chunk - 1);
                const unsigned g =
                    ((((unsigned)bx << lgNBV) + (unsigned)bv) << (__builtin_ctz(TX) + lgTV)) +
                    (unsigned)(half * chunk + w);
                rx[i] = *reinterpret_cast<const pack<T>*>(Ux + g);
                ry[i] = *reinterpret_cast<const pack<T>*>(Uy + g);
            }
#pragma unroll
            for (int i = 0; i < NVA; ++i) {
                const int e0 = (tid + i * NT) * V;
                const int bv = e0 >> lgCH;
                const int w = e0 & (chunk - 1);
                const int xr = w >> lgTV;
                const int v = (bv << lgTV) + (w & (TV - 1));
#pragma unroll
                for (int q = 0; q < V; ++q)
                    sb[xr * LP + lds_pad(v + q)] = C{rx[i].v[q], ry[i].v[q]};
            }
        }
        __syncthreads();
        C Vk[E / 2], Vm[E / 2];
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            const C zk = buf[lds_pad(s)];
            const C zm = buf[lds_pad(s == 0 ? L / 2 : L - s)];
            C pxk, pxm, pyk, pym;
            inv_pre<T, L>(s, zk.x, zm.x, false, pst[i], pxk, pxm);
            inv_pre<T, L>(s, zk.y, zm.y, true, pst[i], pyk, pym);
            Vk[i] = pack2<T>(pxk, pyk);
            Vm[i] = pack2<T>(pxm, pym);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            buf[lds_pad(s)] = Vk[i];
            buf[lds_pad(s == 0 ? L / 2 : L - s)] = Vm[i];
        }
        __syncthreads();
        fft_lds<T, L, true>(buf, t, twp);
        const size_t base = (size_t)x0 * L;
#pragma unroll
        for (int i = 0; i < NVA; ++i) {
            const int e0 = (tid + i * NT) * V;
            const int xr = e0 / L, y0 = e0 % L;
            pack<T> ox, oy;
#pragma unroll
            for (int q = 0; q < V; ++q) {
                const C z = sb[xr * LP + lds_pad(makhoul_pos<L>(y0 + q))];
                ox.v[q] = z.x;
                oy.v[q] = (q & 1) ? (T)-0.5 * z.y : (T)0.5 * z.y;   // y0 is even
            }
            *reinterpret_cast<pack<T>*>(fx + base + e0) = ox;
            *reinterpret_cast<pack<T>*>(fy + base + e0) = oy;
        }
    } else {
        const int bb = grp;
        const int x0 = bb * TX;
        const size_t base = (size_t)x0 * L;
        const int lgTE = __builtin_ctz(TX) + lgTV;
        constexpr int V = kVec<T>, NVB = TX * L / (NT * V);
        static_assert(NVB * NT * V == TX * L, "P3 vector split");
        const T wv = (T)a.wv_step;
        {
            const pack<T>* src = reinterpret_cast<const pack<T>*>(Uy + base);
            pack<T> r[NVB];
#pragma unroll
            for (int i = 0; i < NVB; ++i) r[i] = src[tid + i * NT];
#pragma unroll
            for (int i = 0; i < NVB; ++i) {
                const int e0 = (tid + i * NT) * V;
                const int bv = e0 >> lgTE;
                const int w = e0 & ((1 << lgTE) - 1);
                const int x_in = w >> lgTV;
                const int v = (bv << lgTV) + (w & (TV - 1));
                C* rowp = sb + (x_in >> 1) * LP;
#pragma unroll
                for (int q = 0; q < V; ++q) comp<T>(rowp[lds_pad(v + q)], x_in & 1) = r[i].v[q];
            }
        }
        __syncthreads();
        C Vk[E / 2], Vm[E / 2];
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            const int m = s == 0 ? L / 2 : L - s;
            const C zk = buf[lds_pad(s)];
            const C zm = buf[lds_pad(m)];
            // Up = Uy / w_v at the slot's two columns (column 0: / w_v(1))
            const T rk = fast_rcp((T)(s > 0 ? s : 1) * wv), rm = fast_rcp((T)m * wv);
            C pak, pam, pbk, pbm;
            inv_pre<T, L>(s, zk.x * rk, zm.x * rm, false, pst[i], pak, pam);
            inv_pre<T, L>(s, zk.y * rk, zm.y * rm, false, pst[i], pbk, pbm);
            Vk[i] = pack2<T>(pak, pbk);
            Vm[i] = pack2<T>(pam, pbm);
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < E / 2; ++i) {
            const int s = t + TPF * i;
            buf[lds_pad(s)] = Vk[i];
            buf[lds_pad(s == 0 ? L / 2 : L - s)] = Vm[i];
        }
        __syncthreads();
        fft_lds<T, L, true>(buf, t, twp);
        pack<T>* dst = reinterpret_cast<pack<T>*>(phi + base);
#pragma unroll
        for (int i = 0; i < NVB; ++i) {
            const int e0 = (tid + i * NT) * V;
            const int r = e0 / L, y0 = e0 % L;
            const C* rowp = sb + (r >> 1) * LP;
            pack<T> o;
#pragma unroll
            for (int q = 0; q < V; ++q)
                o.v[q] = comp_of<T>(rowp[lds_pad(makhoul_pos<L>(y0 + q))], r & 1);
            dst[tid + i * NT] = o;
        }
    }
}

}  // namespace dpep
