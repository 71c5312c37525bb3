/*
 * cpu_baseline.c -- float32 OpenMP CPU implementation of the electric-potential
 * step, timed by bench.py as the reported CPU baseline ("port").
 *
 * TEST / MEASUREMENT INFRASTRUCTURE ONLY: never linked into the product.
 *
 * It follows DREAMPlace's CPU path as the reference repository restates it:
 * float32 cell geometry with the sqrt2*bin stretch (tools/
 * v13_offset_ratio_stats.py:54-67), a parallel-for over cells with atomic
 * float adds into the bin map (integration/scatter_ttnn_client.py:55-93 is the
 * vectorised restatement), the D0 fold (host/density_scatter_ttnn_server_host.
 * cpp:1770-1777), FFT-based DCT-II / IDCT / IDXST with the normalisation of
 * the reference's matrices (same file :124-181, :281-295), and a parallel-for
 * per-cell force gather.  FFTW is absent from this image, so the FFT is an
 * in-house table-driven radix-2 transform; two real rows are packed into one
 * complex FFT and the column transforms run on a blocked transpose.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#ifdef _OPENMP
#include <omp.h>
#endif

#ifndef M_PI
#define M_PI 3.14159265358979323846
#endif

typedef struct { float re, im; } cf;

typedef struct {
    int K;            /* transform length (power of two) */
    int* rev;         /* bit reversal permutation        */
    cf* tw;           /* exp(-2 pi i m / K), m < K/2     */
    cf* post;         /* exp(-i pi k / (2K)), k < K      */
} plan1d;

typedef struct {
    int M, N;
    float xl, yl, xh, yh;
    plan1d px, py;    /* along x (length M) and y (length N) */
    float *T, *Tt, *Ux, *Uy, *Up, *Uxt, *Uyt, *Upt;
} cpu_base;

static double now_ms(void)
{
    struct timespec ts;
    clock_gettime(CLOCK_MONOTONIC, &ts);
    return ts.tv_sec * 1e3 + ts.tv_nsec * 1e-6;
}

static int plan_init(plan1d* p, int K)
{
    p->K = K;
    p->rev = malloc(sizeof(int) * K);
    p->tw = malloc(sizeof(cf) * (K / 2 + 1));
    p->post = malloc(sizeof(cf) * K);
    if (!p->rev || !p->tw || !p->post) return 1;
    int lg = 0;
    while ((1 << lg) < K) ++lg;
    for (int i = 0; i < K; ++i) {
        int r = 0;
        for (int b = 0; b < lg; ++b) r |= ((i >> b) & 1) << (lg - 1 - b);
        p->rev[i] = r;
    }
    for (int m = 0; m <= K / 2; ++m) {
        p->tw[m].re = (float)cos(2.0 * M_PI * m / K);
        p->tw[m].im = (float)-sin(2.0 * M_PI * m / K);
    }
    for (int k = 0; k < K; ++k) {
        p->post[k].re = (float)cos(M_PI * k / (2.0 * K));
        p->post[k].im = (float)-sin(M_PI * k / (2.0 * K));
    }
    return 0;
}

static void plan_free(plan1d* p)
{
    free(p->rev); free(p->tw); free(p->post);
}

/* in-place radix-2 FFT; inv conjugates the twiddles; unscaled */
static void fft(const plan1d* p, cf* a, int inv)
{
    const int K = p->K;
    for (int i = 0; i < K; ++i) {
        int j = p->rev[i];
        if (i < j) { cf t = a[i]; a[i] = a[j]; a[j] = t; }
    }
    for (int len = 2; len <= K; len <<= 1) {
        const int step = K / len;
        for (int i = 0; i < K; i += len)
            for (int k = 0; k < len / 2; ++k) {
                cf w = p->tw[k * step];
                if (inv) w.im = -w.im;
                cf u = a[i + k], v = a[i + k + len / 2];
                cf t = { v.re * w.re - v.im * w.im, v.re * w.im + v.im * w.re };
                a[i + k].re = u.re + t.re; a[i + k].im = u.im + t.im;
                a[i + k + len / 2].re = u.re - t.re;
                a[i + k + len / 2].im = u.im - t.im;
            }
    }
}

/* Forward unscaled DCT-II of two real rows r1, r2 (length K) -> o1, o2.    */
static void dct2_pair(const plan1d* p, const float* r1, const float* r2,
                      float* o1, float* o2, float scale, cf* z)
{
    const int K = p->K;
    for (int n = 0; n < K / 2; ++n) {
        z[n].re = r1[2 * n]; z[n].im = r2 ? r2[2 * n] : 0.f;
        z[K - 1 - n].re = r1[2 * n + 1]; z[K - 1 - n].im = r2 ? r2[2 * n + 1] : 0.f;
    }
    fft(p, z, 0);
    for (int k = 0; k < K; ++k) {
        cf a = z[k], b = z[(K - k) & (K - 1)];
        /* V1 = (a + conj b)/2, V2 = -i (a - conj b)/2 */
        cf v1 = { 0.5f * (a.re + b.re), 0.5f * (a.im - b.im) };
        cf v2 = { 0.5f * (a.im + b.im), -0.5f * (a.re - b.re) };
        cf t = p->post[k];
        o1[k] = scale * (t.re * v1.re - t.im * v1.im);
        if (o2) o2[k] = scale * (t.re * v2.re - t.im * v2.im);
    }
}

/* y = I_K X (c_0 = 1, c_k = 2) for two real spectra packed in one IFFT.
 * rev{1,2}: use X'[k] = X[K-k], X'[0] = 0 (the S_K identity).               */
static void idct_pair(const plan1d* p, const float* X1, int rev1,
                      const float* X2, int rev2, float* y1, float* y2,
                      float s1, float s2, int alt1, int alt2, cf* z)
{
    const int K = p->K;
    for (int k = 0; k < K; ++k) {
        float a1, b1, a2 = 0.f, b2 = 0.f;   /* X[k], X[K-k] */
        if (rev1) { a1 = k ? X1[K - k] : 0.f; b1 = k ? X1[k] : 0.f; }
        else      { a1 = X1[k]; b1 = k ? X1[K - k] : 0.f; }
        if (X2) {
            if (rev2) { a2 = k ? X2[K - k] : 0.f; b2 = k ? X2[k] : 0.f; }
            else      { a2 = X2[k]; b2 = k ? X2[K - k] : 0.f; }
        }
        cf t = p->post[k];           /* conj gives exp(+i pi k / 2K) */
        const float c = t.re, s = -t.im;
        /* V = e^{i th} (a - i b) = (c a + s b) + i (s a - c b) */
        cf v1 = { c * a1 + s * b1, s * a1 - c * b1 };
        cf v2 = { c * a2 + s * b2, s * a2 - c * b2 };
        z[k].re = v1.re - v2.im;
        z[k].im = v1.im + v2.re;
    }
    fft(p, z, 1);
    for (int n = 0; n < K / 2; ++n) {
        const int m0 = 2 * n, m1 = 2 * n + 1;
        cf e = z[n], o = z[K - 1 - n];
        y1[m0] = s1 * e.re * (alt1 ? 1.f : 1.f);
        y1[m1] = s1 * o.re * (alt1 ? -1.f : 1.f);
        if (y2) {
            y2[m0] = s2 * e.im;
            y2[m1] = s2 * o.im * (alt2 ? -1.f : 1.f);
        }
    }
}

static void transpose(const float* in, int R, int C, float* out)
{
#pragma omp parallel for schedule(static) collapse(2)
    for (int r0 = 0; r0 < R; r0 += 32)
        for (int c0 = 0; c0 < C; c0 += 32)
            for (int r = r0; r < r0 + 32 && r < R; ++r)
                for (int c = c0; c < c0 + 32 && c < C; ++c)
                    out[(long)c * R + r] = in[(long)r * C + c];
}

void cpu_baseline_destroy(void* h)
{
    cpu_base* b = h;
    if (!b) return;
    plan_free(&b->px); plan_free(&b->py);
    free(b->T); free(b->Tt); free(b->Ux); free(b->Uy); free(b->Up);
    free(b->Uxt); free(b->Uyt); free(b->Upt);
    free(b);
}

void* cpu_baseline_create(int M, int N, float xl, float yl, float xh, float yh)
{
    if (M < 4 || N < 4 || (M & (M - 1)) || (N & (N - 1))) return NULL;
    cpu_base* b = calloc(1, sizeof(cpu_base));
    if (!b) return NULL;
    b->M = M; b->N = N; b->xl = xl; b->yl = yl; b->xh = xh; b->yh = yh;
    const size_t MN = (size_t)M * N;
    int bad = plan_init(&b->px, M) | plan_init(&b->py, N);
    b->T = malloc(4 * MN); b->Tt = malloc(4 * MN);
    b->Ux = malloc(4 * MN); b->Uy = malloc(4 * MN); b->Up = malloc(4 * MN);
    b->Uxt = malloc(4 * MN); b->Uyt = malloc(4 * MN); b->Upt = malloc(4 * MN);
    if (bad || !b->T || !b->Tt || !b->Ux || !b->Uy || !b->Up || !b->Uxt ||
        !b->Uyt || !b->Upt) {
        cpu_baseline_destroy(b);
        return NULL;
    }
    return b;
}

/* One step.  stage_ms[0..2] = scatter, spectral solve, gather.             */
int cpu_baseline_step(void* h, const float* px, const float* py,
                      const float* sx, const float* sy, long nc,
                      const float* d0n, float* density, float* phi, float* fx,
                      float* fy, float* gx, float* gy, double* stage_ms)
{
    cpu_base* b = h;
    if (!b || !density || !fx || !fy) return 1;
    const int M = b->M, N = b->N;
    const size_t MN = (size_t)M * N;
    const float bsx = (b->xh - b->xl) / M, bsy = (b->yh - b->yl) / N;
    const float inv_ba = 1.0f / (bsx * bsy);
    const float minw = (float)M_SQRT2 * bsx, minh = (float)M_SQRT2 * bsy;
    const float xl = b->xl, yl = b->yl;

    double t0 = now_ms();
    /* ---- scatter ---- */
#pragma omp parallel for schedule(static)
    for (size_t i = 0; i < MN; ++i) density[i] = d0n ? d0n[i] : 0.f;
#pragma omp parallel for schedule(dynamic, 4096)
    for (long i = 0; i < nc; ++i) {
        const float w0 = sx[i], h0 = sy[i];
        if (!(w0 > 0.f && h0 > 0.f)) continue;
        const float w = w0 > minw ? w0 : minw, hh = h0 > minh ? h0 : minh;
        const float x = px[i] + 0.5f * (w0 - w), y = py[i] + 0.5f * (h0 - hh);
        const float s = (w0 * h0) / (w * hh) * inv_ba;
        int bxl = (int)floorf((x - xl) / bsx), bxh = (int)floorf((x + w - xl) / bsx);
        int byl = (int)floorf((y - yl) / bsy), byh = (int)floorf((y + hh - yl) / bsy);
        if (bxl < 0) bxl = 0;
        if (byl < 0) byl = 0;
        if (bxh > M - 1) bxh = M - 1;
        if (byh > N - 1) byh = N - 1;
        for (int k = bxl; k <= bxh; ++k) {
            const float bl = xl + k * bsx;
            const float tx = fminf(x + w, bl + bsx) - fmaxf(x, bl);
            if (tx <= 0.f) continue;
            for (int q = byl; q <= byh; ++q) {
                const float bb = yl + q * bsy;
                const float ty = fminf(y + hh, bb + bsy) - fmaxf(y, bb);
                if (ty <= 0.f) continue;
#pragma omp atomic
                density[(size_t)k * N + q] += s * tx * ty;
            }
        }
    }
    double t1 = now_ms();

    /* ---- spectral solve ---- */
    /* rows (along y): T[x,:] = (2/N) DCT2(rho[x,:]) */
#pragma omp parallel
    {
        cf* z = malloc(sizeof(cf) * (M > N ? M : N));
#pragma omp for schedule(static)
        for (int x = 0; x < M; x += 2)
            dct2_pair(&b->py, density + (size_t)x * N, density + (size_t)(x + 1) * N,
                      b->T + (size_t)x * N, b->T + (size_t)(x + 1) * N, 2.0f / N, z);
        free(z);
    }
    transpose(b->T, M, N, b->Tt);     /* Tt is N x M */
#pragma omp parallel
    {
        cf* z = malloc(sizeof(cf) * (M > N ? M : N));
        float* A = malloc(sizeof(float) * M);
        float* B1 = malloc(sizeof(float) * M);
        float* B2 = malloc(sizeof(float) * M);
        const double r = (double)(b->xh - b->xl) / M / ((double)(b->yh - b->yl) / N);
#pragma omp for schedule(static)
        for (int v = 0; v < N; ++v) {
            dct2_pair(&b->px, b->Tt + (size_t)v * M, NULL, A, NULL, 2.0f / M, z);
            const double wv = 2.0 * M_PI * v / N * r;
            for (int u = 0; u < M; ++u) {
                const double wu = 2.0 * M_PI * u / M, d = wu * wu + wv * wv;
                const float inv = (u == 0 && v == 0) ? 0.f : (float)(1.0 / d);
                B1[u] = A[u] * (float)wu * inv * 0.5f;   /* Wx */
                B2[u] = A[u] * (float)wv * inv * 0.5f;   /* Wy */
            }
            /* Ux = 2 S_M Bx = (-1)^x I(Bx'); Uy = 2 I_M By */
            idct_pair(&b->px, B1, 1, B2, 0, b->Uxt + (size_t)v * M,
                      b->Uyt + (size_t)v * M, 1.0f, 2.0f, 1, 0, z);
            if (phi) {
                for (int u = 0; u < M; ++u) {
                    const double wu = 2.0 * M_PI * u / M, d = wu * wu + wv * wv;
                    B1[u] = (u == 0 && v == 0) ? 0.f : A[u] * (float)(1.0 / d);
                }
                idct_pair(&b->px, B1, 0, NULL, 0, b->Upt + (size_t)v * M, NULL,
                          1.0f, 0.f, 0, 0, z);
            }
        }
        free(z); free(A); free(B1); free(B2);
    }
    transpose(b->Uxt, N, M, b->Ux);
    transpose(b->Uyt, N, M, b->Uy);
    if (phi) transpose(b->Upt, N, M, b->Up);
#pragma omp parallel
    {
        cf* z = malloc(sizeof(cf) * (M > N ? M : N));
#pragma omp for schedule(static)
        for (int x = 0; x < M; ++x) {
            /* fx = I_N Ux ; fy = S_N Uy = (-1)^y 1/2 I(Uy') */
            idct_pair(&b->py, b->Ux + (size_t)x * N, 0, b->Uy + (size_t)x * N, 1,
                      fx + (size_t)x * N, fy + (size_t)x * N, 1.0f, 0.5f, 0, 1, z);
        }
        if (phi) {
#pragma omp for schedule(static)
            for (int x = 0; x < M; x += 2)
                idct_pair(&b->py, b->Up + (size_t)x * N, 0, b->Up + (size_t)(x + 1) * N, 0,
                          phi + (size_t)x * N, phi + (size_t)(x + 1) * N, 1.0f, 1.0f, 0, 0, z);
        }
        free(z);
    }
    double t2 = now_ms();

    /* ---- per-cell gather ---- */
    if (gx && gy) {
#pragma omp parallel for schedule(dynamic, 4096)
        for (long i = 0; i < nc; ++i) {
            const float w0 = sx[i], h0 = sy[i];
            float ax = 0.f, ay = 0.f;
            if (w0 > 0.f && h0 > 0.f) {
                const float w = w0 > minw ? w0 : minw, hh = h0 > minh ? h0 : minh;
                const float x = px[i] + 0.5f * (w0 - w), y = py[i] + 0.5f * (h0 - hh);
                int bxl = (int)floorf((x - xl) / bsx), bxh = (int)floorf((x + w - xl) / bsx);
                int byl = (int)floorf((y - yl) / bsy), byh = (int)floorf((y + hh - yl) / bsy);
                if (bxl < 0) bxl = 0;
                if (byl < 0) byl = 0;
                if (bxh > M - 1) bxh = M - 1;
                if (byh > N - 1) byh = N - 1;
                for (int k = bxl; k <= bxh; ++k) {
                    const float bl = xl + k * bsx;
                    const float tx = fminf(x + w, bl + bsx) - fmaxf(x, bl);
                    if (tx <= 0.f) continue;
                    for (int q = byl; q <= byh; ++q) {
                        const float bb = yl + q * bsy;
                        const float ty = fminf(y + hh, bb + bsy) - fmaxf(y, bb);
                        if (ty <= 0.f) continue;
                        ax += tx * ty * fx[(size_t)k * N + q];
                        ay += tx * ty * fy[(size_t)k * N + q];
                    }
                }
                const float ratio = (w0 * h0) / (w * hh);
                ax *= ratio; ay *= ratio;
            }
            gx[i] = ax; gy[i] = ay;
        }
    }
    double t3 = now_ms();
    if (stage_ms) {
        stage_ms[0] = t1 - t0;
        stage_ms[1] = t2 - t1;
        stage_ms[2] = t3 - t2;
    }
    return 0;
}

int cpu_baseline_threads(void)
{
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}
