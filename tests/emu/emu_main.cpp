// CPU emulation of one electric-potential step with libdpep's kernel source
// (csrc/dpep_bin.h, csrc/dpep_spectral.h) under AddressSanitizer.
// Every global buffer is malloc'd at its exact size and the LDS tail beyond
// the launch's dynamic size is poisoned, so any out-of-bounds index aborts
// with a report.  Results are compared with the float64 oracle.
// Usage: emu_main <f32|f64> M N ncells [det] [nopot] [ch=<entries>] [tall] [stage] [off]
//        emu_main blocks   (host logic of the cell blocks)
#include <sanitizer/asan_interface.h>
#include <stdio.h>
#include <stdlib.h>

#include <functional>
#include <random>
#include <thread>
#include <memory>
#include <vector>

#include "dpep_bin.h"
#include "dpep_spectral.h"

thread_local dim3 threadIdx, blockIdx;
dim3 blockDim, gridDim;
std::barrier<>* emu_barrier = nullptr;
namespace dpep {
alignas(16) unsigned char smem[163840];
int spectral_fpw(int L, int dtype) { return dtype == 0 ? fpw<float>(L) : fpw<double>(L); }
}

extern "C" {
int oracle_density(const double*, const double*, const double*, const double*, long, int, int,
                   double, double, double, double, int, const double*, double*);
int oracle_solve_fft(const double*, int, int, double, double, double*, double*, double*);
int oracle_gather(const double*, const double*, const double*, const double*, long, int, int,
                  double, double, double, double, int, const double*, const double*, double*,
                  double*);
}

// shuffle groups of the current launch: teams of 16 lanes and waves of 64
static std::vector<std::unique_ptr<std::barrier<>>> emu_groups16, emu_groups64;
double emu_shfl_slot[1024];
std::barrier<>* emu_group_barrier(unsigned group, int width)
{
    auto& gs = width == 16 ? emu_groups16 : emu_groups64;
    if ((width != 16 && width != 64) || group >= gs.size()) {
        fprintf(stderr, "shuffle width %d / group %u not emulated\n", width, group);
        abort();
    }
    return gs[group].get();
}

static void launch(unsigned grid, unsigned block, size_t shm, const std::function<void()>& body)
{
    blockDim = dim3(block);
    gridDim = dim3(grid);
    emu_groups16.clear();
    emu_groups64.clear();
    for (unsigned q = 0; q < block / 16; ++q)
        emu_groups16.push_back(std::make_unique<std::barrier<>>(16));
    for (unsigned q = 0; q < (block + 63) / 64; ++q)
        emu_groups64.push_back(std::make_unique<std::barrier<>>(block - 64 * q < 64 ? block - 64 * q : 64));
    if (shm > sizeof(dpep::smem)) { fprintf(stderr, "LDS %zu too big\n", shm); abort(); }
    // One OS thread per GPU thread of a block, created once per launch; the
    // blocks run one after another, fenced by barriers, with the LDS
    // scribbled over and its tail re-poisoned between blocks.
    std::barrier<> bar(block);
    emu_barrier = &bar;
    std::vector<std::thread> ts;
    ts.reserve(block);
    for (unsigned t = 0; t < block; ++t)
        ts.emplace_back([&, t] {
            threadIdx = dim3(t);
            for (unsigned b = 0; b < grid; ++b) {
                if (t == 0) {
                    ASAN_UNPOISON_MEMORY_REGION(dpep::smem, sizeof(dpep::smem));
                    memset(dpep::smem, 0xA5, sizeof(dpep::smem));
                    ASAN_POISON_MEMORY_REGION(dpep::smem + shm, sizeof(dpep::smem) - shm);
                }
                bar.arrive_and_wait();
                blockIdx = dim3(b);
                body();
                bar.arrive_and_wait();
            }
        });
    for (auto& th : ts) th.join();
    ASAN_UNPOISON_MEMORY_REGION(dpep::smem, sizeof(dpep::smem));
}

template <typename T>
static T* exact(size_t n) { return (T*)malloc(n * sizeof(T) + (n == 0)); }

template <typename T>
static std::vector<T> table(int L, bool post)
{
    const int n = post ? L / 2 + 1 : L;
    std::vector<T> v(2 * (size_t)n);
    for (int m = 0; m < n; ++m) {
        const double a = post ? M_PI * m / (2.0 * L) : 2.0 * M_PI * m / L;
        v[2 * m] = (T)cos(a);
        v[2 * m + 1] = (T)-sin(a);
    }
    return v;
}

// The spectral passes in the form launch_col_pass / launch_row_inv pick:
// tile extents compiled in for square grids of kSquareMin and more.
template <typename T, int L, int F>
static void col_pass_as_launched(const dpep::SpectralArgs& a, const T* Tt, T* Ux, T* Uy)
{
    using namespace dpep;
    if (square_form<T, L>(a)) k_col_pass<T, L, F, true>(a, Tt, Ux, Uy);
    else k_col_pass<T, L, F, false>(a, Tt, Ux, Uy);
}

template <typename T, int L, int F>
static void row_inv_as_launched(const dpep::SpectralArgs& a, const T* Ux, const T* Uy, T* fx,
                                T* fy, T* phi)
{
    using namespace dpep;
    if (square_form<T, L>(a)) k_row_inv<T, L, F, true>(a, Ux, Uy, fx, fy, phi);
    else k_row_inv<T, L, F, false>(a, Ux, Uy, fx, fy, phi);
}

template <typename T, int LM, int LN>
static int run(int nc, bool det, bool pot, int ch, bool tall, bool force_stage, bool off)
{
    using namespace dpep;
    const int M = LM, N = LN;
    const size_t mn = (size_t)M * N;
    // off: a die whose lower-left corner is not the origin
    const double xl = off ? -1234.5 : 0.0, yl = off ? 777.25 : 0.0;
    const double xh = xl + 100.0 * M / 8, yh = yl + 80.0 * N / 8;
    Grid g{};
    g.M = M; g.N = N; g.xl = xl; g.yl = yl; g.xh = xh; g.yh = yh;
    g.bsx = (xh - xl) / M; g.bsy = (yh - yl) / N; g.inv_ba = 1.0 / (g.bsx * g.bsy);
    g.inv_bsx = 1.0 / g.bsx; g.inv_bsy = 1.0 / g.bsy;
    g.minw = M_SQRT2 * g.bsx; g.minh = M_SQRT2 * g.bsy; g.stretch = 1;
    g.fix_scale = ldexp(1.0, fix_exponent_of(nc, (int)sizeof(T)));
    (void)det;
    std::mt19937_64 rng(1234);
    std::uniform_real_distribution<double> U(0, 1);
    T* px = exact<T>(nc); T* py = exact<T>(nc); T* sx = exact<T>(nc); T* sy = exact<T>(nc);
    for (int i = 0; i < nc; ++i) {
        sx[i] = (T)(g.bsx * (0.3 + 3 * U(rng)));
        sy[i] = (T)(g.bsy * (0.3 + 2 * U(rng)));
        px[i] = (T)(xl + (xh - xl) * (1.1 * U(rng) - 0.05));   // some outside the die
        py[i] = (T)(yl + (yh - yl) * (1.1 * U(rng) - 0.05));
    }
    if (nc > 2) { sx[0] = 0; sy[1] = -1; sx[2] = (T)(3 * (xh - xl)); px[2] = (T)(xl - (xh - xl)); }
    if (tall)   // a tenth of the cells spans 3..40 rows
        for (int i = 3; i < nc; i += 10) sx[i] = (T)(g.bsx * (3 + 37 * U(rng)));
    T* d0n = exact<T>(mn); T* dens = exact<T>(mn); T* phi = pot ? exact<T>(mn) : nullptr;
    T* fx = exact<T>(mn); T* fy = exact<T>(mn); T* Tt = exact<T>(mn); T* Ux = exact<T>(mn);
    T* Uy = exact<T>(mn); T* gx = exact<T>(nc); T* gy = exact<T>(nc);
    for (size_t i = 0; i < mn; ++i) d0n[i] = (T)(0.5 * U(rng));
    auto twM = table<T>(M, false), twN = table<T>(N, false);
    auto poM = table<T>(M, true), poN = table<T>(N, true);
    T* d_twM = exact<T>(twM.size()); memcpy(d_twM, twM.data(), twM.size() * sizeof(T));
    T* d_twN = exact<T>(twN.size()); memcpy(d_twN, twN.data(), twN.size() * sizeof(T));
    T* d_poM = exact<T>(poM.size()); memcpy(d_poM, poM.data(), poM.size() * sizeof(T));
    T* d_poN = exact<T>(poN.size()); memcpy(d_poN, poN.data(), poN.size() * sizeof(T));
    SpectralArgs a{};
    a.M = M; a.N = N;
    a.tiles.TX = 2 * fpw<T>(N); a.tiles.TV = 2 * fpw<T>(M);
    a.tiles.TXT = t_tile_rows(strip_rows(N), a.tiles.TX, a.tiles.TV, sizeof(T), M);
    a.wu_step = 2 * M_PI / M; a.wv_step = 2 * M_PI / N * (g.bsx / g.bsy);
    a.potential = pot; a.twM = d_twM; a.postM = d_poM; a.twN = d_twN; a.postN = d_poN;

    // strip binning buffers, exact sizes
    BinPlan p = make_bin_plan(M, N, nc, sizeof(T));
    BinArgs b{};
    b.S = p.S; b.R = p.R; b.lgR = p.lgR;
    if (ch > 0) {   // fixed chunks: every list can hold all of them
        b.ch_force = ch;
        b.Pacc = b.Pgat = p.S + (int)((p.reg_cap + ch - 1) / ch) + 1;
        b.Wacc = b.Wgat = b.Pacc;
    } else {        // chosen per step, as on the device, for a 2-CU "device"
        set_item_grids(b, 2, 3, 2);
    }
    b.G1 = count_grid_max(nc);          // rows of cnt; set per step below
    const size_t nslot = (size_t)kCountSlots * p.S;
    b.cnt = exact<unsigned>((size_t)b.G1 * p.S);
    b.xtot = exact<unsigned>(2 * nslot);           // two sets, by step parity
    memset(b.xtot, 0, 2 * nslot * sizeof(unsigned));
    b.pbase = exact<unsigned>(nslot);
    b.pcap = exact<unsigned>(nslot);
    b.pool_n = exact<unsigned>(2);
    b.pool_n[0] = b.pool_n[1] = 0u;
    b.reg_cap = (unsigned)p.reg_cap;
    b.pool0 = (unsigned)p.reg_cap;
    b.pool_cap = (unsigned)p.cap;
    b.ovst = exact<unsigned long long>(2 * (size_t)p.S);
    memset(b.ovst, 0, 2 * (size_t)p.S * sizeof(unsigned long long));
    b.rmax = run_capacity(nc);
    b.oruns = exact<uint2>((size_t)p.S * b.rmax);
    const size_t nrec = p.reg_cap + p.cap;
    b.items = exact<uint4>(b.Wacc);
    b.items_g = exact<uint4>(b.Wgat);
    b.nitems = exact<unsigned>(2);
    b.chunk = exact<unsigned>(2);
    if (sizeof(vec4_t<T>) != p.geo_bytes) { fprintf(stderr, "record size mismatch\n"); return 4; }
    b.recg = malloc(nrec * p.geo_bytes);
    b.recm = exact<unsigned>(nrec);
    b.done = exact<unsigned>(p.S);
    memset(b.done, 0, p.S * sizeof(unsigned));
    b.pos = exact<unsigned long long>(nc > 0 ? nc : 1);
    b.gtmp = exact<vec2_t<T>>(nrec);
    b.bigflag = exact<unsigned>(kSideWords * p.S);
    b.raw = exact<T>(mn);        // the scatter density without D0, checked below
    b.B = malloc(mn * 8);
    memset(b.B, 0, mn * 8);
    memset(b.bigflag, 0, kSideWords * p.S * sizeof(unsigned));
    const size_t hist = (size_t)p.S * sizeof(unsigned);
    // the library stages K3's records from kStageMinStrips strips on; "stage"
    // forces the staged form on any grid
    const bool stage = force_stage || p.S >= kStageMinStrips;
    unsigned pool_seen = 0;
    // one step: fresh (K1 + K3) or in one pass on the previous step's counts
    auto step = [&](bool once) -> int {
        const OnceBlocks ob = once_blocks(nc, b.cus, sizeof(T));   // as launch_bin_scatter
        set_count_blocks(b, ob);
        if (once) {
            with_cpt(ob.cpt, [&](auto c) -> hipError_t {
                constexpr int CPT = decltype(c)::value;
                launch((unsigned)ob.grid, kOnceThreads, fill_once_lds<T>(p.S),
                       [&] { k_bin_fill_once<T, CPT>(px, py, sx, sy, nc, g, b); });
                return hipSuccess;
            });
        } else {
            launch(b.G1, kBinThreads, hist, [&] { k_bin_count<T>(px, py, sx, sy, nc, g, b); });
            if (stage)
                launch(b.G1, kBinThreads, fill_lds_staged<T>(p.S),
                       [&] { k_bin_fill_staged<T>(px, py, sx, sy, nc, g, b); });
            else
                launch(b.G1, kBinThreads,
                       (size_t)(2 * p.S + kBinThreads + kChunkCands) * sizeof(unsigned),
                       [&] { k_bin_fill_direct<T>(px, py, sx, sy, nc, g, b); });
        }
        pool_seen = b.pool_n[b.par];
        launch(b.Wacc, kAccThreads, acc_lds_bytes<T, LN>(),
               [&] { k_strip_acc<T, LN>(g, b, a, d0n, dens, Tt); });
        for (int s2 = 0; s2 < p.S; ++s2)
            if (b.done[s2]) { fprintf(stderr, "strip chunk counter left set\n"); return 4; }
        for (int s2 = 0; s2 < kSideWords * p.S; ++s2)
            if (b.bigflag[s2]) { fprintf(stderr, "bigflag left set\n"); return 4; }
        {
            constexpr int F = fpw<T>(LM);
            const size_t shm = (size_t)F * lds_len(LM) * sizeof(vec2_t<T>);
            launch(N / (2 * F), col_threads<T>(LM), shm, [&] { col_pass_as_launched<T, LM, F>(a, Tt, Ux, Uy); });
        }
        {
            constexpr int F = fpw<T>(LN);
            const size_t shm = (size_t)F * lds_len(LN) * sizeof(vec2_t<T>);
            const unsigned grid = (M / (2 * F)) * (pot ? 3 : 2);
            launch(grid, row_threads<T>(LN), shm, [&] { row_inv_as_launched<T, LN, F>(a, Ux, Uy, fx, fy, phi); });
        }
        if (nc > 0) {
            const size_t glds = gather_lds<T>(p.R, N);
            if (b.Wgat == b.S)       // as launch_bin_gather
                launch(b.Wgat, kAccThreads, glds, [&] { k_gather_bin<T, true>(g, b, fx, fy); });
            else
                launch(b.Wgat, kAccThreads, glds, [&] { k_gather_bin<T, false>(g, b, fx, fy); });
            with_cpt(ob.cpt, [&](auto c) -> hipError_t {   // as launch_bin_gather
                constexpr int CPT = decltype(c)::value;
                launch((unsigned)ob.grid, kOnceThreads, gather_out_lds<kOnceThreads, CPT>(), [&] {
                    k_gather_out<T, kOnceThreads, CPT>(px, py, sx, sy, nc, g, b, fx, fy, gx, gy);
                });
                return hipSuccess;
            });
        }
        // the older set of counts is zero again for the next step
        const unsigned* older = b.xtot + (size_t)(b.par ^ 1) * nslot;
        for (size_t s2 = 0; s2 < nslot; ++s2)
            if (older[s2]) { fprintf(stderr, "previous counts left set\n"); return 4; }
        if (b.pool_n[b.par ^ 1]) { fprintf(stderr, "previous overflow count left set\n"); return 4; }
        for (int s2 = 0; s2 < p.S; ++s2)
            if (b.ovst[(size_t)(b.par ^ 1) * p.S + s2]) { fprintf(stderr, "previous overflow runs left set\n"); return 4; }
        b.par ^= 1;
        const unsigned char* Bb = (const unsigned char*)b.B;
        for (size_t i = 0; i < mn * 8; ++i)
            if (Bb[i]) { fprintf(stderr, "side map B not re-zeroed at byte %zu (row %zu)\n", i, i / 8 / N); return 4; }
        return 0;
    };
    // step 1 counts first; step 2 sorts in one pass into regions sized
    // from step 1's counts (no overflow: same cells); step 3 sizes them at
    // half of step 2's counts, so it overflows about half its records --
    // and must give bitwise step 2's results
    int rc = step(false);
    if (rc) return rc;
    if (pool_seen) { fprintf(stderr, "fresh step used the pool\n"); return 4; }
    rc = step(true);
    if (rc) return rc;
    if (pool_seen) { fprintf(stderr, "one-pass step on the same cells overflowed (%u)\n", pool_seen); return 4; }
    std::vector<T> keep[7];
    T* outs[7] = {dens, fx, fy, gx, gy, (T*)b.raw, phi};
    const size_t lens[7] = {mn, mn, mn, (size_t)nc, (size_t)nc, mn, pot ? mn : 0};
    for (int k = 0; k < 7; ++k) keep[k].assign(outs[k], outs[k] + lens[k]);
    b.tight = 1;                  // regions at half of step 2's counts
    rc = step(true);
    b.tight = 0;
    if (rc) return rc;
    const unsigned pool_tight = pool_seen;
    for (int k = 0; k < 7; ++k)
        if (lens[k] && memcmp(keep[k].data(), outs[k], lens[k] * sizeof(T))) {
            fprintf(stderr, "overflowing step differs from the planned one in output %d\n", k);
            return 4;
        }
    printf("emu plan S=%d R=%d chunks=%u/%u items=%u/%u of %d/%d block=%d overflow=%u\n", p.S,
           p.R, b.chunk[0], b.chunk[1], b.nitems[0], b.nitems[1], b.Wacc, b.Wgat, b.qcells,
           pool_tight);

    // oracle
    std::vector<double> dpx(nc), dpy(nc), dsx(nc), dsy(nc), dd0(mn), rho(mn), rphi(mn), rfx(mn), rfy(mn), rgx(nc), rgy(nc);
    for (int i = 0; i < nc; ++i) { dpx[i] = px[i]; dpy[i] = py[i]; dsx[i] = sx[i]; dsy[i] = sy[i]; }
    for (size_t i = 0; i < mn; ++i) dd0[i] = d0n[i];
    std::vector<double> rraw(mn);
    oracle_density(dpx.data(), dpy.data(), dsx.data(), dsy.data(), nc, M, N, xl, yl, xh, yh, 1, nullptr, rraw.data());
    oracle_density(dpx.data(), dpy.data(), dsx.data(), dsy.data(), nc, M, N, xl, yl, xh, yh, 1, dd0.data(), rho.data());
    oracle_solve_fft(rho.data(), M, N, g.bsx, g.bsy, rphi.data(), rfx.data(), rfy.data());
    oracle_gather(dpx.data(), dpy.data(), dsx.data(), dsy.data(), nc, M, N, xl, yl, xh, yh, 1, rfx.data(), rfy.data(), rgx.data(), rgy.data());
    auto linf = [](const T* x, const double* r, size_t n) {
        double m = 0, d = 0;
        for (size_t i = 0; i < n; ++i) { m = fmax(m, fabs(r[i])); d = fmax(d, fabs((double)x[i] - r[i])); }
        return d / (m > 0 ? m : 1);
    };
    auto l2 = [](const T* x, const double* r, size_t n) {
        double m = 0, d = 0;
        for (size_t i = 0; i < n; ++i) { m += r[i] * r[i]; d += ((double)x[i] - r[i]) * ((double)x[i] - r[i]); }
        return sqrt(d) / (m > 0 ? sqrt(m) : 1);
    };
    const double e_d = linf(dens, rho.data(), mn), e_p = pot ? linf(phi, rphi.data(), mn) : 0.0;
    const double e_r = nc ? linf((const T*)b.raw, rraw.data(), mn) : 0.0;
    const double e_fx = l2(fx, rfx.data(), mn), e_fy = l2(fy, rfy.data(), mn);
    const double e_gx = nc ? l2(gx, rgx.data(), nc) : 0.0, e_gy = nc ? l2(gy, rgy.data(), nc) : 0.0;
    printf("emu %s M=%d N=%d nc=%d det=%d pot=%d: density %.2e scatter density %.2e potential %.2e fx %.2e fy %.2e gx %.2e gy %.2e\n",
           sizeof(T) == 4 ? "f32" : "f64", M, N, nc, det, pot, e_d, e_r, e_p, e_fx, e_fy, e_gx, e_gy);
    const double tl = sizeof(T) == 4 ? 1e-5 : 1e-10, tf = sizeof(T) == 4 ? 1e-4 : 1e-9;
    const bool ok = e_d <= tl && e_r <= tl && e_p <= tl && e_fx <= tf && e_fy <= tf && e_gx <= tf && e_gy <= tf;
    return ok ? 0 : 3;
}

// The spectral passes alone (P2 k_col_pass, P3 k_row_inv) on a random
// density, at any grid including the largest lengths: T, the row DCT-II of
// rho along y (the first pass, which K4 runs on its strip tile), is computed
// here in float64 and laid out in T's tiles as K4 writes them; the fields and
// the potential are compared with the oracle's FFT solve of rho.
template <typename T, int LM, int LN>
static int run_spectral()
{
    using namespace dpep;
    const int M = LM, N = LN;
    const size_t mn = (size_t)M * N;
    const double bsx = 70.0 / M, bsy = 50.0 / N;   // a 70 x 50 die, as the GPU solve tests
    std::mt19937_64 rng(4321);
    std::uniform_real_distribution<double> U(0, 1);
    std::vector<double> rho(mn);
    for (auto& r : rho) r = U(rng);
    auto twM = table<T>(M, false), twN = table<T>(N, false);
    auto poM = table<T>(M, true), poN = table<T>(N, true);
    T* d_twM = exact<T>(twM.size()); memcpy(d_twM, twM.data(), twM.size() * sizeof(T));
    T* d_twN = exact<T>(twN.size()); memcpy(d_twN, twN.data(), twN.size() * sizeof(T));
    T* d_poM = exact<T>(poM.size()); memcpy(d_poM, poM.data(), poM.size() * sizeof(T));
    T* d_poN = exact<T>(poN.size()); memcpy(d_poN, poN.data(), poN.size() * sizeof(T));
    SpectralArgs a{};
    a.M = M; a.N = N;
    a.tiles.TX = 2 * fpw<T>(N); a.tiles.TV = 2 * fpw<T>(M);
    a.tiles.TXT = t_tile_rows(strip_rows(N), a.tiles.TX, a.tiles.TV, sizeof(T), M);
    a.wu_step = 2 * M_PI / M; a.wv_step = 2 * M_PI / N * (bsx / bsy);
    a.potential = 1; a.twM = d_twM; a.postM = d_poM; a.twN = d_twN; a.postN = d_poN;
    // T[x][v] = (2 / N) sum_y rho[x][y] cos(pi v (y + 1/2) / N), in T's tiles
    const int TXT = a.tiles.TXT, TV = a.tiles.TV;
    const int lgTXT = __builtin_ctz(TXT), lgTV = __builtin_ctz(TV);
    const int lgNBV = __builtin_ctz(N) - lgTV, lgTET = lgTXT + lgTV;
    T* Tt = exact<T>(mn);
    std::vector<double> cosv((size_t)N * N);
    for (int v = 0; v < N; ++v)
        for (int y = 0; y < N; ++y) cosv[(size_t)v * N + y] = cos(M_PI * v * (y + 0.5) / N);
    for (int x = 0; x < M; ++x)
        for (int v = 0; v < N; ++v) {
            double t = 0;
            for (int y = 0; y < N; ++y) t += rho[(size_t)x * N + y] * cosv[(size_t)v * N + y];
            const size_t at = ((((size_t)(x >> lgTXT) << lgNBV) + (size_t)(v >> lgTV)) << lgTET) +
                              ((size_t)(x & (TXT - 1)) << lgTV) + (size_t)(v & (TV - 1));
            Tt[at] = (T)(2.0 / N * t);
        }
    T* Ux = exact<T>(mn); T* Uy = exact<T>(mn);
    T* fx = exact<T>(mn); T* fy = exact<T>(mn); T* phi = exact<T>(mn);
    {
        constexpr int F = fpw<T>(LM);
        const size_t shm = (size_t)F * lds_len(LM) * sizeof(vec2_t<T>);
        launch(N / (2 * F), col_threads<T>(LM), shm, [&] { col_pass_as_launched<T, LM, F>(a, Tt, Ux, Uy); });
    }
    {
        constexpr int F = fpw<T>(LN);
        const size_t shm = (size_t)F * lds_len(LN) * sizeof(vec2_t<T>);
        launch((M / (2 * F)) * 3, row_threads<T>(LN), shm,
               [&] { row_inv_as_launched<T, LN, F>(a, Ux, Uy, fx, fy, phi); });
    }
    std::vector<double> rphi(mn), rfx(mn), rfy(mn);
    oracle_solve_fft(rho.data(), M, N, bsx, bsy, rphi.data(), rfx.data(), rfy.data());
    auto err = [&](const T* x, const std::vector<double>& r, bool inf) {
        double m = 0, d = 0;
        for (size_t i = 0; i < mn; ++i) {
            const double e = (double)x[i] - r[i];
            if (inf) { m = fmax(m, fabs(r[i])); d = fmax(d, fabs(e)); }
            else { m += r[i] * r[i]; d += e * e; }
        }
        return inf ? d / (m > 0 ? m : 1) : sqrt(d) / (m > 0 ? sqrt(m) : 1);
    };
    const double e_p = err(phi, rphi, true), e_fx = err(fx, rfx, false), e_fy = err(fy, rfy, false);
    printf("emu spectral %s M=%d N=%d: potential %.2e fx %.2e fy %.2e\n",
           sizeof(T) == 4 ? "f32" : "f64", M, N, e_p, e_fx, e_fy);
    const double tl = sizeof(T) == 4 ? 1e-5 : 1e-10, tf = sizeof(T) == 4 ? 1e-4 : 1e-9;
    return (e_p <= tl && e_fx <= tf && e_fy <= tf) ? 0 : 3;
}

template <typename T>
static int dispatch_spectral(int M, int N)
{
#define CASE(a, b) if (M == a && N == b) return run_spectral<T, a, b>();
    CASE(2048, 16) CASE(4096, 32) CASE(16, 2048) CASE(32, 4096) CASE(1024, 64)
    CASE(512, 512) CASE(1024, 1024)
    if constexpr (sizeof(T) == 4) { CASE(8192, 8) CASE(8, 8192) }
#undef CASE
    fprintf(stderr, "unsupported shape\n");
    return 2;
}

template <typename T>
static int dispatch(int M, int N, int nc, bool det, bool pot, int ch, bool tall, bool stage,
                    bool off)
{
#define CASE(a, b) if (M == a && N == b) return run<T, a, b>(nc, det, pot, ch, tall, stage, off);
    CASE(8, 8) CASE(16, 16) CASE(8, 32) CASE(64, 64) CASE(16, 128) CASE(128, 16)
    CASE(256, 32) CASE(32, 256) CASE(32, 2048) CASE(16, 4096)
    if constexpr (sizeof(T) == 4) { CASE(8, 8192) }
#undef CASE
    fprintf(stderr, "unsupported shape\n");
    return 2;
}

// Host logic of the cell blocks (once_blocks, set_count_blocks, count_cells):
// every cell in exactly one one-pass block and one counting part, no part
// straddling two blocks, no empty block, the kernels' limits and the cnt
// rows (count_grid_max) respected, for many cell counts and CU counts.
static int check_blocks()
{
    using namespace dpep;
    std::mt19937_64 rng(7);
    std::vector<long long> ncs = {0, 1, 63, 64, 1023, 1024, 1025, 2047, 2048, 2049, 4096,
                                  210000, 256000, 1100000, 2000000, 2600000, 1 << 26};
    const int cuss[] = {1, 2, 80, 256, 304};
    for (int c : cuss)
        for (int k = 1; k <= 3; ++k)
            for (long long q : {2048LL, 2560LL})
                for (long long d = -70; d <= 70; d += 35)
                    ncs.push_back(k * c * q + d);
    for (int r = 0; r < 300; ++r) ncs.push_back((long long)(rng() % 3000000));
    long long checked = 0;
    for (int cus : cuss)
        for (int esz : {4, 8})
            for (long long ncl : ncs) {
                if (ncl < 0) continue;
                const int nc = (int)ncl;
                const OnceBlocks o = once_blocks(nc, cus, (size_t)esz);
                const int cmax = kOnceMaxCpt;
                auto fail = [&](const char* what) {
                    fprintf(stderr, "blocks: %s (nc %d cus %d esz %d: grid %d q %d cpt %d)\n",
                            what, nc, cus, esz, o.grid, o.q, o.cpt);
                    return 1;
                };
                if (o.q % 64 || o.q < kOnceMinCells) return fail("block size");
                if (o.cpt < 2 || o.cpt > cmax || o.cpt * kOnceThreads < o.q ||
                    (o.cpt - 1) * kOnceThreads >= o.q)
                    return fail("cells per thread");
                if (o.grid < 1 || (long long)o.grid * o.q < nc ||
                    (nc > 0 && (long long)(o.grid - 1) * o.q >= nc))
                    return fail("grid");
                BinArgs b{};
                set_count_blocks(b, o);
                if (b.qsub > kCellsPerGroup || b.qsub % 64 || (b.sub - 1) * b.qsub >= o.q)
                    return fail("parts");
                if (b.G1 != o.grid * b.sub || b.G1 > count_grid_max(nc)) return fail("cnt rows");
                long long next = 0;     // parts in order tile [0, nc) exactly
                for (int w = 0; w < b.G1; ++w) {
                    blockIdx = dim3((unsigned)w);
                    int c0, cend;
                    const int slot = count_cells(b, nc, c0, cend);
                    const int ob = w / b.sub;
                    if (slot != (ob & (kCountSlots - 1))) return fail("slot");
                    if (cend < c0 || c0 < ob * o.q || (c0 < nc && cend > (ob + 1) * o.q))
                        return fail("part outside its block");
                    if (cend > c0) {
                        if (c0 != next) return fail("parts leave a gap or overlap");
                        next = cend;
                    }
                }
                if (next != nc) return fail("parts do not cover the cells");
                ++checked;
            }
    blockIdx = dim3(0);
    printf("blocks ok (%lld cases)\n", checked);
    return 0;
}

// The float32 record word (rec_geo / rec_put / rec_view): for random cells,
// including those whose stretched corner lies below the die's lower x or y
// edge (offset in [-1, 0), first row or column 0) and the second-strip copy
// of a cell that spans two strips, the decoded record gives the encoded
// geometry: the same absolute first row, offsets within 2^-23 of a bin, the
// same first column, extents and area ratio, and row / column counts that
// reach the far edge.
static int check_records()
{
    using namespace dpep;
    std::mt19937_64 rng(11);
    std::uniform_real_distribution<double> u01(0.0, 1.0);
    const int Rs[] = {1, 2, 4, 8};
    const int N = 8192;
    long long checked = 0;
    for (int it = 0; it < 400000; ++it) {
        const int R = Rs[it % 4];
        const int s0 = (int)(rng() % 64);
        const int k0 = s0 * R;
        const bool xedge = (it % 7) == 0, yedge = (it % 5) == 0;
        const int rel0 = xedge ? 0 : (int)(rng() % R);
        const int byl = yedge ? 0 : (int)(rng() % N);
        const double ex = xedge ? -u01(rng) : u01(rng) * (1.0 - 1e-9);
        const double ey = yedge ? -u01(rng) : u01(rng) * (1.0 - 1e-9);
        const int stretch = (int)(rng() & 1);
        // extents in bins; an edge cell is stretched (its corner moved left)
        const double wb = (xedge || stretch) ? u01(rng) * 1.4 + 1e-3 : u01(rng) * 3.0 + 1e-3;
        const double hb = (yedge || stretch) ? u01(rng) * 1.4 + 1e-3 : u01(rng) * 3.0 + 1e-3;
        const int st = (xedge || yedge) ? 1 : stretch;
        BinArgs b{};
        b.R = R;
        float4 rec[2];
        const float4 geo = rec_geo<float>(ex, ey, wb, hb, byl, rel0);
        rec_put<float>(b, rec, 0u, geo, rec_span<float>(rel0, 0, 0, byl, false));
        // a cell starting in strip s0 that reaches strip s0 + 1 (never an
        // x-edge cell: it would span more than R rows)
        const bool second = !xedge && R > 1;
        if (second) rec_put<float>(b, rec, 1u, geo, rec_span<float>(rel0 - R, 0, 0, byl, true));
        for (int copy = 0; copy < (second ? 2 : 1); ++copy) {
            const int kc = copy ? k0 + R : k0;       // the strip the copy is in
            const RecView<float> v = rec_view<float>(rec[copy], 0u, kc, st, N);
            const double x_abs = (double)v.bxl + (double)v.dx;
            const double x_want = (double)(k0 + rel0) + ex;
            const double tol = 1.2e-7;
            bool ok = fabs(x_abs - x_want) <= tol && fabs((double)v.dy - ey) <= tol &&
                      v.byl == byl && v.bxl == k0 + rel0 - (xedge ? 1 : 0);
            const float w = (float)wb, h = (float)hb;
            float wc = w, hc = h, rat = 1.f;
            if (st) {
                const float m = 1.41421356237309504880f;
                wc = w > m ? w : m;
                hc = h > m ? h : m;
                rat = (w * h) * fast_rcp(wc * hc);
            }
            ok = ok && v.rat == rat && v.xr == v.dx + wc && v.yr == v.dy + hc;
            ok = ok && v.nx == (int)v.xr && v.ny == std::min((int)v.yr, N - 1 - byl) &&
                 v.bxl + v.nx + 1 > x_want + wc - 1e-6 && v.ny >= 0;
            if (!ok) {
                fprintf(stderr, "record mismatch it=%d R=%d copy=%d ex=%.9f ey=%.9f byl=%d rel0=%d: "
                        "bxl %d dx %.9f dy %.9f byl %d nx %d ny %d\n", it, R, copy, ex, ey, byl,
                        rel0, v.bxl, v.dx, v.dy, v.byl, v.nx, v.ny);
                return 1;
            }
            ++checked;
        }
    }
    printf("records ok (%lld records)\n", checked);
    return 0;
}

int main(int argc, char** argv)
{
    if (argc == 2 && !strcmp(argv[1], "blocks")) return check_blocks();
    if (argc == 2 && !strcmp(argv[1], "records")) return check_records();
    if (argc == 5 && !strcmp(argv[1], "spectral"))
        return !strcmp(argv[2], "f64") ? dispatch_spectral<double>(atoi(argv[3]), atoi(argv[4]))
                                       : dispatch_spectral<float>(atoi(argv[3]), atoi(argv[4]));
    if (argc < 5) { fprintf(stderr, "usage: %s f32|f64 M N nc [det] [nopot]\n", argv[0]); return 2; }
    const bool f64 = !strcmp(argv[1], "f64");
    const int M = atoi(argv[2]), N = atoi(argv[3]), nc = atoi(argv[4]);
    bool det = false, pot = true, tall = false, stage = false, off = false;
    int ch = 0;
    for (int i = 5; i < argc; ++i) {
        if (!strcmp(argv[i], "det")) det = true;
        if (!strcmp(argv[i], "nopot")) pot = false;
        if (!strcmp(argv[i], "tall")) tall = true;
        if (!strcmp(argv[i], "stage")) stage = true;
        if (!strcmp(argv[i], "off")) off = true;
        if (!strncmp(argv[i], "ch=", 3)) ch = atoi(argv[i] + 3);
    }
    return f64 ? dispatch<double>(M, N, nc, det, pot, ch, tall, stage, off)
               : dispatch<float>(M, N, nc, det, pot, ch, tall, stage, off);
}
