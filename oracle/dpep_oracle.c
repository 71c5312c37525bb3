/*
 * dpep_oracle.c -- CPU restatement of DREAMPlace's electric-potential step.
 *
 * TEST INFRASTRUCTURE ONLY.  This file is the checker the GPU path is compared
 * against; it is never linked into, loaded by or called from the product
 * library (libdpep.so), the shm server or the Python client.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Everything here accumulates in float64 from the caller's inputs (which the
 * tests convert exactly from the float32/float64 values the GPU receives).
 *
 * Reference algorithm followed, per function (paths relative to the
 * DREAMPlaceTT-Framework tree):
 *   oracle_cell_geom     tools/v13_offset_ratio_stats.py:54-67 (sqrt2*bin
 *                        stretch, offset=(s-s_c)/2, ratio=area/area_c) and
 *                        integration/scatter_ttnn_client.py:619-633
 *   oracle_density       kernels/v4_compute.cpp:128-176 (overlap formula),
 *                        tools/cpu_vs_tt_density.py:45-76 (float64 loops over
 *                        the bin span), tools/v11_phase2_smoke.py:21-94
 *                        (float64 accumulate, *inv_ba), host/
 *                        density_scatter_ttnn_server_host.cpp:1770-1777 (D0 fold),
 *                        layout rho[bx*N+by] (kernels/v11_accum_dm.cpp:386-398)
 *   oracle_solve_direct  host/density_scatter_ttnn_server_host.cpp:124-181
 *                        (C_K, I_K, S_K matrices), :251-263 (wu, wv, (0,0)->0),
 *                        :281-295 (A = C_M rho C_N^T; fx = 2S_M(A.Wx)I_N^T;
 *                        fy = 2I_M(A.Wy)S_N^T) -- literal matrix products
 *   oracle_solve_fft     same maths through zero-padded 2K-point complex FFTs
 *                        (an algorithm independent of the GPU's)
 *   oracle_gather        per-cell sum_k sum_h ratio*tx(k)*ty(h)*field[k*N+h],
 *                        the consumer of ctx.field_map_x/y stashed at
 *                        integration/scatter_ttnn_client.py:831-855
 *
 * The potential phi = I_M (A / D) I_N^T has no counterpart in the reference
 * (the TT server never computes it); it is the unique phi whose spectral
 * gradient reproduces fx and fy above: (fx, fy) = -bsx * grad(phi).
 *
 * Pinned by tests/test_oracle.py: brute-force O(cells x bins) density on tiny
 * inputs, mass conservation, whole-bin translation, direct-vs-FFT solve,
 * scipy.fft DCT/DST golden vectors (tests/golden/), single-mode closed forms,
 * and the scatter/gather adjoint identity.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

#define ORACLE_OK 0
#define ORACLE_ERR_ARG 1
#define ORACLE_ERR_NOMEM 4

/* ------------------------------------------------------------------------- */
/* Cell geometry                                                              */
/* ------------------------------------------------------------------------- */

typedef struct {
    double x, y;       /* lower-left corner after the stretch shift      */
    double w, h;       /* stretched extent                               */
    double ratio;      /* original area / stretched area                 */
    int bxl, bxh;      /* inclusive bin span along x (clipped to [0,M))  */
    int byl, byh;      /* inclusive bin span along y (clipped to [0,N))  */
} cell_geom;

/* Index of the bin containing v: the k with origin + k*bs <= v <
 * origin + (k+1)*bs for the bin edges as computed in floating point.  The
 * reciprocal-multiply estimate is corrected against those exact edges, the
 * approach of the reference's correct_bin_idx (kernels/v4_compute.cpp:91-102). */
double oracle_floor_bin(double v, double origin, double bs, double inv)
{
    double k = floor((v - origin) * inv);
    if (origin + k * bs > v) k -= 1.0;
    else if (origin + (k + 1.0) * bs <= v) k += 1.0;
    return k;
}

/* Returns 1 when the cell contributes, 0 for padding / degenerate cells.   */
int oracle_cell_geom(double px, double py, double sx, double sy,
                     int M, int N, double xl, double yl, double xh, double yh,
                     int stretch, cell_geom* g)
{
    if (!(isfinite(px) && isfinite(py) && isfinite(sx) && isfinite(sy)))
        return 0;
    if (!(sx > 0.0 && sy > 0.0))
        return 0;
    const double bsx = (xh - xl) / M;
    const double bsy = (yh - yl) / N;
    double w = sx, h = sy, ratio = 1.0, x = px, y = py;
    if (stretch) {
        const double minw = M_SQRT2 * bsx;
        const double minh = M_SQRT2 * bsy;
        w = sx > minw ? sx : minw;
        h = sy > minh ? sy : minh;
        x = px + 0.5 * (sx - w);
        y = py + 0.5 * (sy - h);
        ratio = (sx * sy) / (w * h);
    }
    const double ibx = 1.0 / bsx, iby = 1.0 / bsy;
    double fxl = oracle_floor_bin(x, xl, bsx, ibx);
    double fxh = oracle_floor_bin(x + w, xl, bsx, ibx);
    double fyl = oracle_floor_bin(y, yl, bsy, iby);
    double fyh = oracle_floor_bin(y + h, yl, bsy, iby);
    if (fxl < 0.0) fxl = 0.0;
    if (fyl < 0.0) fyl = 0.0;
    if (fxh > M - 1) fxh = M - 1;
    if (fyh > N - 1) fyh = N - 1;
    if (fxl > fxh || fyl > fyh)
        return 0;
    g->x = x; g->y = y; g->w = w; g->h = h; g->ratio = ratio;
    g->bxl = (int)fxl; g->bxh = (int)fxh;
    g->byl = (int)fyl; g->byh = (int)fyh;
    return 1;
}

static inline double overlap_1d(double lo, double ext, double origin,
                                double bs, int k)
{
    const double bl = origin + k * bs;
    const double br = origin + (k + 1) * bs;
    const double hi = lo + ext;
    const double a = lo > bl ? lo : bl;
    const double b = hi < br ? hi : br;
    const double o = b - a;
    return o > 0.0 ? o : 0.0;
}

/* ------------------------------------------------------------------------- */
/* Density scatter                                                            */
/* ------------------------------------------------------------------------- */

int oracle_density(const double* px, const double* py, const double* sx,
                   const double* sy, long nc, int M, int N, double xl,
                   double yl, double xh, double yh, int stretch,
                   const double* d0n, double* out)
{
    if (M <= 0 || N <= 0 || nc < 0 || !out || !(xh > xl) || !(yh > yl))
        return ORACLE_ERR_ARG;
    const long MN = (long)M * N;
    const double bsx = (xh - xl) / M, bsy = (yh - yl) / N;
    const double inv_ba = 1.0 / (bsx * bsy);
    for (long i = 0; i < MN; ++i) out[i] = 0.0;
    for (long i = 0; i < nc; ++i) {
        cell_geom g;
        if (!oracle_cell_geom(px[i], py[i], sx[i], sy[i], M, N, xl, yl, xh,
                              yh, stretch, &g))
            continue;
        const double s = g.ratio * inv_ba;
        for (int k = g.bxl; k <= g.bxh; ++k) {
            const double tx = overlap_1d(g.x, g.w, xl, bsx, k);
            if (tx <= 0.0) continue;
            for (int h = g.byl; h <= g.byh; ++h) {
                const double ty = overlap_1d(g.y, g.h, yl, bsy, h);
                if (ty <= 0.0) continue;
                out[(long)k * N + h] += s * tx * ty;
            }
        }
    }
    if (d0n)
        for (long i = 0; i < MN; ++i) out[i] += d0n[i];
    return ORACLE_OK;
}

/* Brute force over every bin for every cell: O(nc*M*N).  Used only on tiny
 * inputs to pin oracle_density's bin-span logic.                           */
int oracle_density_bruteforce(const double* px, const double* py,
                              const double* sx, const double* sy, long nc,
                              int M, int N, double xl, double yl, double xh,
                              double yh, int stretch, double* out)
{
    if (M <= 0 || N <= 0 || !out) return ORACLE_ERR_ARG;
    const double bsx = (xh - xl) / M, bsy = (yh - yl) / N;
    const double inv_ba = 1.0 / (bsx * bsy);
    for (long i = 0; i < (long)M * N; ++i) out[i] = 0.0;
    for (long i = 0; i < nc; ++i) {
        if (!(isfinite(px[i]) && isfinite(py[i]) && isfinite(sx[i]) &&
              isfinite(sy[i])) || !(sx[i] > 0.0 && sy[i] > 0.0))
            continue;
        double w = sx[i], h = sy[i], x = px[i], y = py[i], ratio = 1.0;
        if (stretch) {
            w = fmax(sx[i], M_SQRT2 * bsx);
            h = fmax(sy[i], M_SQRT2 * bsy);
            x = px[i] + 0.5 * (sx[i] - w);
            y = py[i] + 0.5 * (sy[i] - h);
            ratio = sx[i] * sy[i] / (w * h);
        }
        for (int k = 0; k < M; ++k) {
            const double tx = overlap_1d(x, w, xl, bsx, k);
            for (int hh = 0; hh < N; ++hh) {
                const double ty = overlap_1d(y, h, yl, bsy, hh);
                out[(long)k * N + hh] += ratio * tx * ty * inv_ba;
            }
        }
    }
    return ORACLE_OK;
}

/* ------------------------------------------------------------------------- */
/* Per-cell gather                                                            */
/* ------------------------------------------------------------------------- */

int oracle_gather(const double* px, const double* py, const double* sx,
                  const double* sy, long nc, int M, int N, double xl,
                  double yl, double xh, double yh, int stretch,
                  const double* fx, const double* fy, double* gx, double* gy)
{
    if (M <= 0 || N <= 0 || nc < 0 || !fx || !fy || !gx || !gy)
        return ORACLE_ERR_ARG;
    const double bsx = (xh - xl) / M, bsy = (yh - yl) / N;
#pragma omp parallel for schedule(static)
    for (long i = 0; i < nc; ++i) {
        cell_geom g;
        double ax = 0.0, ay = 0.0;
        if (oracle_cell_geom(px[i], py[i], sx[i], sy[i], M, N, xl, yl, xh,
                             yh, stretch, &g)) {
            for (int k = g.bxl; k <= g.bxh; ++k) {
                const double tx = overlap_1d(g.x, g.w, xl, bsx, k);
                if (tx <= 0.0) continue;
                for (int h = g.byl; h <= g.byh; ++h) {
                    const double ty = overlap_1d(g.y, g.h, yl, bsy, h);
                    if (ty <= 0.0) continue;
                    ax += tx * ty * fx[(long)k * N + h];
                    ay += tx * ty * fy[(long)k * N + h];
                }
            }
            ax *= g.ratio;
            ay *= g.ratio;
        }
        gx[i] = ax;
        gy[i] = ay;
    }
    return ORACLE_OK;
}

/* ------------------------------------------------------------------------- */
/* Spectral solve, direct matrices (reference host code's 6-matmul chain)     */
/* ------------------------------------------------------------------------- */

/* C_K[k,n] = (2/K) cos(pi k (n+1/2) / K)                                    */
static void mat_dct2(int K, double* m)
{
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < K; ++n)
            m[(long)k * K + n] = (2.0 / K) * cos(M_PI * k * (n + 0.5) / K);
}
/* I_K[k,0] = 1, I_K[k,n] = 2 cos(pi n (k+1/2) / K)                          */
static void mat_idct(int K, double* m)
{
    for (int k = 0; k < K; ++k) {
        m[(long)k * K] = 1.0;
        for (int n = 1; n < K; ++n)
            m[(long)k * K + n] = 2.0 * cos(M_PI * n * (k + 0.5) / K);
    }
}
/* S_K[k,n] = sin(pi n (k+1/2) / K)                                          */
static void mat_idxst(int K, double* m)
{
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < K; ++n)
            m[(long)k * K + n] = sin(M_PI * n * (k + 0.5) / K);
}

/* out[M,N] = L[M,M] * X[M,N] * R[N,N]^T                                     */
static void sandwich(const double* Lm, const double* X, const double* Rm,
                     int M, int N, double* tmp, double* out)
{
    /* tmp = X * R^T : tmp[a,b] = sum_c X[a,c] R[b,c] */
#pragma omp parallel for schedule(static)
    for (int a = 0; a < M; ++a)
        for (int b = 0; b < N; ++b) {
            double s = 0.0;
            for (int c = 0; c < N; ++c) s += X[(long)a * N + c] * Rm[(long)b * N + c];
            tmp[(long)a * N + b] = s;
        }
#pragma omp parallel for schedule(static)
    for (int a = 0; a < M; ++a)
        for (int b = 0; b < N; ++b) {
            double s = 0.0;
            for (int c = 0; c < M; ++c) s += Lm[(long)a * M + c] * tmp[(long)c * N + b];
            out[(long)a * N + b] = s;
        }
}

/* Spectral weights, reference host code :251-263.  kind 0: Wx, 1: Wy, 2: 1/D */
static double weight(int kind, int u, int v, int M, int N, double bsx,
                     double bsy)
{
    if (u == 0 && v == 0) return 0.0;
    const double wu = 2.0 * M_PI * u / M;
    const double wv = 2.0 * M_PI * v / N * (bsx / bsy);
    const double d = wu * wu + wv * wv;
    if (kind == 0) return wu / d * 0.5;
    if (kind == 1) return wv / d * 0.5;
    return 1.0 / d;
}

int oracle_solve_direct(const double* rho, int M, int N, double bsx,
                        double bsy, double* phi, double* fx, double* fy)
{
    if (M <= 0 || N <= 0 || !rho) return ORACLE_ERR_ARG;
    const long MN = (long)M * N;
    double* CM = malloc(sizeof(double) * M * M);
    double* CN = malloc(sizeof(double) * N * N);
    double* IM = malloc(sizeof(double) * M * M);
    double* IN = malloc(sizeof(double) * N * N);
    double* SM = malloc(sizeof(double) * M * M);
    double* SN = malloc(sizeof(double) * N * N);
    double* A = malloc(sizeof(double) * MN);
    double* B = malloc(sizeof(double) * MN);
    double* tmp = malloc(sizeof(double) * MN);
    int rc = ORACLE_OK;
    if (!CM || !CN || !IM || !IN || !SM || !SN || !A || !B || !tmp) {
        rc = ORACLE_ERR_NOMEM;
        goto done;
    }
    mat_dct2(M, CM); mat_dct2(N, CN);
    mat_idct(M, IM); mat_idct(N, IN);
    mat_idxst(M, SM); mat_idxst(N, SN);
    for (long i = 0; i < (long)M * M; ++i) SM[i] *= 2.0; /* 2*S_M */
    sandwich(CM, rho, CN, M, N, tmp, A);                  /* A = C_M rho C_N^T */
    if (fx) {
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(0, u, v, M, N, bsx, bsy);
        sandwich(SM, B, IN, M, N, tmp, fx);
    }
    if (fy) {
        for (long i = 0; i < (long)M * M; ++i) SM[i] = 2.0 * IM[i]; /* 2*I_M */
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(1, u, v, M, N, bsx, bsy);
        sandwich(SM, B, SN, M, N, tmp, fy);
    }
    if (phi) {
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(2, u, v, M, N, bsx, bsy);
        sandwich(IM, B, IN, M, N, tmp, phi);
    }
done:
    free(CM); free(CN); free(IM); free(IN); free(SM); free(SN);
    free(A); free(B); free(tmp);
    return rc;
}

/* ------------------------------------------------------------------------- */
/* Spectral solve through zero-padded FFTs                                    */
/* ------------------------------------------------------------------------- */

typedef struct { double re, im; } cpx;

static int is_pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }

/* In-place iterative radix-2 FFT, sign -1 forward, +1 inverse, no scaling. */
static void fft_radix2(cpx* a, int n, int sign)
{
    for (int i = 1, j = 0; i < n; ++i) {
        int bit = n >> 1;
        for (; j & bit; bit >>= 1) j ^= bit;
        j ^= bit;
        if (i < j) { cpx t = a[i]; a[i] = a[j]; a[j] = t; }
    }
    for (int len = 2; len <= n; len <<= 1) {
        const double ang = sign * 2.0 * M_PI / len;
        for (int i = 0; i < n; i += len) {
            for (int k = 0; k < len / 2; ++k) {
                const double c = cos(ang * k), s = sin(ang * k);
                cpx u = a[i + k], v = a[i + k + len / 2];
                cpx t = { v.re * c - v.im * s, v.re * s + v.im * c };
                a[i + k].re = u.re + t.re; a[i + k].im = u.im + t.im;
                a[i + k + len / 2].re = u.re - t.re;
                a[i + k + len / 2].im = u.im - t.im;
            }
        }
    }
}

/* Length-K transforms along a strided line, all unscaled:
 *   kind 0  X[k] = sum_n x[n] cos(pi k (2n+1) / 2K)          (DCT-II)
 *   kind 1  y[n] = sum_k c_k X[k] cos(pi k (2n+1) / 2K)      (I_K, c_0=1, c_k=2)
 *   kind 2  y[n] = sum_k X[k] sin(pi k (2n+1) / 2K)          (S_K)
 * buf holds 2K complex values of scratch.                                   */
static void line_transform(int kind, const double* in, long stride, int K,
                           double* out, long ostride, cpx* buf)
{
    if (!is_pow2(K)) {
        for (int a = 0; a < K; ++a) {
            double s = 0.0;
            for (int b = 0; b < K; ++b) {
                if (kind == 0)
                    s += in[b * stride] * cos(M_PI * a * (2.0 * b + 1) / (2.0 * K));
                else if (kind == 1)
                    s += (b ? 2.0 : 1.0) * in[b * stride] *
                         cos(M_PI * b * (2.0 * a + 1) / (2.0 * K));
                else
                    s += in[b * stride] * sin(M_PI * b * (2.0 * a + 1) / (2.0 * K));
            }
            out[a * ostride] = s;
        }
        return;
    }
    const int P = 2 * K;
    if (kind == 0) {
        for (int n = 0; n < P; ++n) { buf[n].re = n < K ? in[n * stride] : 0.0; buf[n].im = 0.0; }
        fft_radix2(buf, P, -1);
        for (int k = 0; k < K; ++k) {
            const double c = cos(M_PI * k / P), s = -sin(M_PI * k / P);
            out[k * ostride] = buf[k].re * c - buf[k].im * s;
        }
    } else {
        for (int k = 0; k < P; ++k) {
            if (k < K) {
                const double ck = (kind == 1 && k) ? 2.0 : 1.0;
                const double c = cos(M_PI * k / P), s = sin(M_PI * k / P);
                buf[k].re = ck * in[k * stride] * c;
                buf[k].im = ck * in[k * stride] * s;
            } else {
                buf[k].re = buf[k].im = 0.0;
            }
        }
        fft_radix2(buf, P, +1);
        for (int n = 0; n < K; ++n)
            out[n * ostride] = kind == 1 ? buf[n].re : buf[n].im;
    }
}

/* Applies transform kx along x (rows index) and ky along y to X (M x N).   */
static int separable(const double* X, int M, int N, int kx, int ky,
                     double scale, double* out)
{
    const long MN = (long)M * N;
    double* tmp = malloc(sizeof(double) * MN);
    if (!tmp) return ORACLE_ERR_NOMEM;
    int fail = 0;
#pragma omp parallel
    {
        cpx* buf = malloc(sizeof(cpx) * 2 * (M > N ? M : N));
        if (!buf) {
#pragma omp atomic write
            fail = 1;
        } else {
#pragma omp for schedule(static)
            for (int x = 0; x < M; ++x)
                line_transform(ky, X + (long)x * N, 1, N, tmp + (long)x * N, 1, buf);
#pragma omp for schedule(static)
            for (int y = 0; y < N; ++y)
                line_transform(kx, tmp + y, N, M, out + y, N, buf);
            free(buf);
        }
    }
    if (!fail)
        for (long i = 0; i < MN; ++i) out[i] *= scale;
    free(tmp);
    return fail ? ORACLE_ERR_NOMEM : ORACLE_OK;
}

int oracle_solve_fft(const double* rho, int M, int N, double bsx, double bsy,
                     double* phi, double* fx, double* fy)
{
    if (M <= 0 || N <= 0 || !rho) return ORACLE_ERR_ARG;
    const long MN = (long)M * N;
    double* A = malloc(sizeof(double) * MN);
    double* B = malloc(sizeof(double) * MN);
    int rc = ORACLE_OK;
    if (!A || !B) { rc = ORACLE_ERR_NOMEM; goto done; }
    /* A = C_M rho C_N^T = (2/M)(2/N) DCT2_x DCT2_y rho */
    rc = separable(rho, M, N, 0, 0, 4.0 / ((double)M * N), A);
    if (rc) goto done;
    if (fx) {
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(0, u, v, M, N, bsx, bsy);
        rc = separable(B, M, N, 2, 1, 2.0, fx); /* 2 S_M (.) I_N^T */
        if (rc) goto done;
    }
    if (fy) {
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(1, u, v, M, N, bsx, bsy);
        rc = separable(B, M, N, 1, 2, 2.0, fy); /* 2 I_M (.) S_N^T */
        if (rc) goto done;
    }
    if (phi) {
        for (int u = 0; u < M; ++u)
            for (int v = 0; v < N; ++v)
                B[(long)u * N + v] = A[(long)u * N + v] * weight(2, u, v, M, N, bsx, bsy);
        rc = separable(B, M, N, 1, 1, 1.0, phi); /* I_M (.) I_N^T */
    }
done:
    free(A);
    free(B);
    return rc;
}

/* Single 1-D transform, exposed so tests can pin line_transform against
 * scipy.fft golden vectors.                                                 */
int oracle_line_transform(int kind, const double* in, int K, double* out)
{
    if (K <= 0 || kind < 0 || kind > 2) return ORACLE_ERR_ARG;
    cpx* buf = malloc(sizeof(cpx) * 2 * K);
    if (!buf) return ORACLE_ERR_NOMEM;
    line_transform(kind, in, 1, K, out, 1, buf);
    free(buf);
    return ORACLE_OK;
}

int oracle_num_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
