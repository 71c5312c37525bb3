// dpep_api.hip -- the C ABI of libdpep.so (declared in include/dpep.h).
//
// A context owns every device buffer of one (M, N, nc_max, dtype) problem,
// allocated once at creation; a step allocates nothing.  Launch sequence of
// one step on the context's stream:
//   k_bin_count, k_bin_fill               counting sort of cells into strips
//   k_strip_acc                           LDS strip accumulation, D0 fold,
//                                         and P1 (row DCT) of each strip
//   k_col_pass  P2
//   k_row_inv   P3  -> field_x, field_y, potential
//   k_gather_bin, k_gather_out   per-cell forces <- fields
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <new>

#include <mutex>
#include <string>
#include <vector>

#include "dpep.h"
#include "dpep_internal.h"

using namespace dpep;

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

#define HIP_TRY(expr)                                                        \
    do {                                                                     \
        hipError_t e_ = (expr);                                              \
        if (e_ != hipSuccess)                                                \
            return fail(DPEP_ERR_HIP, "%s failed: %s", #expr,                 \
                        hipGetErrorString(e_));                              \
    } while (0)

// strip count (+ table), strip fill, strip accumulate (+ row DCT), column
// pass, row inverse, gather
constexpr int kNumStages = 7;

// the context's output buffers, for the validity mask
constexpr unsigned kOutDensity = 1u, kOutPotential = 2u, kOutFx = 4u, kOutFy = 8u,
                   kOutGx = 16u, kOutGy = 32u, kOutRaw = 64u;

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

}  // namespace

struct dpep_ctx {
    int M = 0, N = 0, nc_max = 0, dtype = 0;
    unsigned flags = 0;
    int device = 0;
    size_t esz = 4;
    Grid grid{};
    SpectralArgs sargs{};
    void *d_px = nullptr, *d_py = nullptr, *d_sx = nullptr, *d_sy = nullptr;
    void *d_d0n = nullptr, *d_density = nullptr, *d_potential = nullptr;
    void *d_fx = nullptr, *d_fy = nullptr, *d_gx = nullptr, *d_gy = nullptr;
    void *d_T = nullptr, *d_Ux = nullptr, *d_Uy = nullptr;
    void* d_raw = nullptr;       // scatter density without D0 (DPEP_FLAG_SCATTER_DENSITY)
    BinPlan plan{};
    BinArgs bins{};
    void *d_twM = nullptr, *d_postM = nullptr, *d_twN = nullptr,
         *d_postN = nullptr;
    hipStream_t stream = nullptr;
    hipEvent_t ev[kNumStages + 1] = {};
    hipEvent_t ev_x0 = nullptr, ev_x1 = nullptr;
    // per-kernel profiling: a ring of `prof_slots` event sets, one per step,
    // a (start, end) pair per kernel stamped by its own dispatch
    std::vector<hipEvent_t> prof_ev;   // prof_slots * 2 * kNumStages
    std::vector<unsigned char> prof_mask;   // per slot: the stages that step launched
    int profiling = 0;
    int prof_slots = 0;
    long prof_steps = 0;               // steps recorded since enabling
    int nc = -1;                 // resident cells (-1: none uploaded)
    int nc_sizes = 0;            // cells whose sizes are resident in d_sx, d_sy
    int last_nc = 0;             // cells of the last computed step
    int stepped = 0;
    // the last step left its counts for this one (parity par ^ 1): fill in
    // one pass.  A failed step leaves the counts in an unknown state: the
    // next one re-zeroes both sets and counts first.
    int planned = 0;
    int scrub = 0;
    int par = 0;                 // parity of the next step's set of counts
    int last_par = 0;            // parity of the last step's set of counts
    int last_once = 0;           // the last step sorted in one pass
    hipStream_t last_stream = nullptr;   // the stream the last step ran on
    // which of the context's own output buffers hold the last step's results
    // (kOut* bits): a step on caller-owned outputs leaves the others stale,
    // and new cells uploaded after the step make every output stale
    unsigned valid = 0;
    float h2d_ms = 0.f, d2h_den_ms = 0.f, d2h_out_ms = 0.f;
};

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
static int check_ctx(const dpep_ctx* c)
{
    if (!c) return fail(DPEP_ERR_ARG, "null context");
    return DPEP_OK;
}

// Twiddle tables on the device (the kernel the no-alloc entry point runs
// too, so both paths use bitwise the same tables).
template <typename T>
static int make_tables(dpep_ctx* c)
{
    HIP_TRY(hipMalloc(&c->d_twM, twiddle_elems(c->M) * sizeof(T)));
    HIP_TRY(hipMalloc(&c->d_twN, twiddle_elems(c->N) * sizeof(T)));
    HIP_TRY(hipMalloc(&c->d_postM, post_elems(c->M) * sizeof(T)));
    HIP_TRY(hipMalloc(&c->d_postN, post_elems(c->N) * sizeof(T)));
    HIP_TRY(launch_tables<T>(c->M, (T*)c->d_twM, (T*)c->d_postM, c->stream));
    HIP_TRY(launch_tables<T>(c->N, (T*)c->d_twN, (T*)c->d_postN, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    c->sargs.twM = c->d_twM;
    c->sargs.postM = c->d_postM;
    c->sargs.twN = c->d_twN;
    c->sargs.postN = c->d_postN;
    return DPEP_OK;
}

static void release(dpep_ctx* c)
{
    const BinArgs& b = c->bins;
    void* bufs[] = {c->d_px, c->d_py, c->d_sx, c->d_sy, c->d_d0n,
                    c->d_density, c->d_potential, c->d_fx, c->d_fy, c->d_gx,
                    c->d_gy, c->d_T, c->d_Ux, c->d_Uy, c->d_twM,
                    c->d_postM, c->d_twN, c->d_postN, b.cnt, b.xtot, b.pbase,
                    b.pcap, b.pool_n, b.ovst, b.oruns, b.items, b.nitems, b.done, b.recg,
                    b.recm, b.pos, b.gtmp,
                    b.bigflag, b.B, b.chunk, b.items_g, c->d_raw};
    for (void* p : bufs)
        if (p) (void)hipFree(p);
    for (auto& e : c->ev)
        if (e) (void)hipEventDestroy(e);
    for (auto& e : c->prof_ev)
        if (e) (void)hipEventDestroy(e);
    c->prof_ev.clear();
    if (c->ev_x0) (void)hipEventDestroy(c->ev_x0);
    if (c->ev_x1) (void)hipEventDestroy(c->ev_x1);
    if (c->stream) (void)hipStreamDestroy(c->stream);
}

template <typename T>
static int run_step(dpep_ctx* c, const T* px, const T* py, const T* sx,
                    const T* sy, int nc, T* fx, T* fy, T* dens, T* phi,
                    T* gx, T* gy, hipStream_t s)
{
    const bool gather = !(c->flags & DPEP_FLAG_NO_GATHER);
    const bool prof = c->profiling != 0;
    const T* d0n = (const T*)c->d_d0n;

    // Every pointer a kernel dereferences must be set: a null here is a bug
    // of this library, reported as an error instead of a device fault.
    const SpectralArgs& a = c->sargs;
    const BinArgs& b = c->bins;
    if (!a.twM || !a.postM || !a.twN || !a.postN || !d0n || !dens || !fx ||
        !fy || !c->d_T || !c->d_Ux || !c->d_Uy || (a.potential && !phi) ||
        !b.xtot ||
        (nc > 0 && (!px || !py || !sx || !sy)) ||
        (gather && (!gx || !gy)) || !b.cnt || !b.pbase || !b.pcap ||
        !b.pool_n || !b.ovst || !b.oruns || !b.items || !b.nitems || !b.done || !b.recg ||
        !b.recm || !b.pos ||
        !b.gtmp || !b.bigflag || !b.B || !b.chunk || !b.items_g)
        return fail(DPEP_ERR_STATE, "internal: a kernel argument is NULL");
    if (nc > c->nc_max)
        return fail(DPEP_ERR_ARG, "nc=%d exceeds nc_max=%d", nc, c->nc_max);
    if (c->scrub) {
        HIP_TRY(hipMemsetAsync(b.xtot, 0, 2 * (size_t)kCountSlots * b.S * sizeof(unsigned), s));
        HIP_TRY(hipMemsetAsync(b.pool_n, 0, 2 * sizeof(unsigned), s));
        HIP_TRY(hipMemsetAsync(b.ovst, 0, 2 * (size_t)b.S * sizeof(unsigned long long), s));
        c->scrub = 0;
    }
    // one pass over the cells when the previous step left its counts
    const bool once = c->planned && !(c->flags & DPEP_FLAG_TWO_PASS);
    c->bins.par = c->par;
    c->planned = 0;
    c->scrub = 1;                 // until the step's last launch succeeds

    // with profiling on, each kernel's dispatch stamps its (start, end) pair
    // in one ring slot; the mask says which kernels this step launched
    const size_t slot = prof ? (size_t)(c->prof_steps % c->prof_slots) : 0;
    const hipEvent_t* pe = prof ? &c->prof_ev[slot * 2 * kNumStages] : nullptr;
    if (prof)
        c->prof_mask[slot] = (unsigned char)((once ? 0u : 1u) | 0x1Eu |
                                             (gather && nc > 0 ? 0x60u : 0u));
    // a recorded event costs GPU time (a few us per step on MI355X): only
    // when the caller asked for per-step timings
    const bool timed = (c->flags & DPEP_FLAG_STEP_TIMINGS) != 0;
    if (timed) HIP_TRY(hipEventRecord(c->ev[0], s));
    HIP_TRY(launch_bin_scatter<T>(px, py, sx, sy, nc, c->grid, c->bins, c->sargs, d0n,
                                  dens, (T*)c->d_T, once, s, pe));

    HIP_TRY(launch_col_pass<T>(c->sargs, (T*)c->d_T, (T*)c->d_Ux, (T*)c->d_Uy, s,
                               pe ? pe + 6 : nullptr));
    HIP_TRY(launch_row_inv<T>(c->sargs, (const T*)c->d_Ux, (const T*)c->d_Uy, fx, fy,
                              phi, s, pe ? pe + 8 : nullptr));
    if (gather)
        HIP_TRY(launch_bin_gather<T>(px, py, sx, sy, nc, c->grid, c->bins, fx, fy,
                                     gx, gy, s, pe ? pe + 10 : nullptr));
    c->planned = 1;
    c->scrub = 0;
    c->last_par = c->par;
    c->last_once = once ? 1 : 0;
    c->last_stream = s;
    c->par ^= 1;
    if (timed) HIP_TRY(hipEventRecord(c->ev[kNumStages], s));
    if (prof) c->prof_steps++;
    c->last_nc = nc;
    c->stepped = 1;
    return DPEP_OK;
}

static int step_dispatch(dpep_ctx* c, const void* px, const void* py,
                         const void* sx, const void* sy, int nc, void* fx,
                         void* fy, void* dens, void* phi, void* gx, void* gy,
                         hipStream_t s)
{
    // outputs the caller does not supply land in the context's buffers
    unsigned valid = kOutRaw;
    if (!fx) { fx = c->d_fx; valid |= kOutFx; }
    if (!fy) { fy = c->d_fy; valid |= kOutFy; }
    if (!dens) { dens = c->d_density; valid |= kOutDensity; }
    if (!phi) { phi = c->d_potential; valid |= kOutPotential; }
    if (!gx) { gx = c->d_gx; valid |= kOutGx; }
    if (!gy) { gy = c->d_gy; valid |= kOutGy; }
    int rc;
    if (c->dtype == DPEP_DTYPE_F32)
        rc = run_step<float>(c, (const float*)px, (const float*)py,
                             (const float*)sx, (const float*)sy, nc,
                             (float*)fx, (float*)fy, (float*)dens,
                             (float*)phi, (float*)gx, (float*)gy, s);
    else
        rc = run_step<double>(c, (const double*)px, (const double*)py,
                              (const double*)sx, (const double*)sy, nc,
                              (double*)fx, (double*)fy, (double*)dens,
                              (double*)phi, (double*)gx, (double*)gy, s);
    c->valid = rc == DPEP_OK ? valid : 0u;
    return rc;
}

static float elapsed(hipEvent_t a, hipEvent_t b)
{
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, a, b) != hipSuccess) return 0.f;
    return ms;
}

int dpep::report_error(int code, const char* msg)
{
    g_last_error = msg;
    return code;
}

hipError_t dpep::prepare_kernels()
{
    static std::once_flag once;
    static hipError_t err = hipSuccess;
    std::call_once(once, [] {
        err = spectral_prepare();
        if (err == hipSuccess) err = bin_prepare();
    });
    return err;
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" {

int dpep_abi_version(void) { return DPEP_ABI_VERSION; }

const char* dpep_build_info(void)
{
    return "dpep abi 6; HIP kernels for gfx950; scatter/P1/P2/P3/gather";
}

const char* dpep_last_error(void) { return g_last_error.c_str(); }

int dpep_create(int M, int N, int nc_max, double xl, double yl, double xh,
                double yh, int dtype, unsigned flags, dpep_ctx** out)
{
    if (!out) return fail(DPEP_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (dtype != DPEP_DTYPE_F32 && dtype != DPEP_DTYPE_F64)
        return fail(DPEP_ERR_ARG, "dtype must be DPEP_DTYPE_F32 or DPEP_DTYPE_F64");
    const int maxL = dtype == DPEP_DTYPE_F32 ? 8192 : 4096;
    if (!is_pow2(M) || !is_pow2(N) || M < 8 || N < 8 || M > maxL || N > maxL)
        return fail(DPEP_ERR_UNSUPPORTED,
                    "num_bins_x=%d num_bins_y=%d: both must be powers of two in [8, %d]",
                    M, N, maxL);
    if (nc_max < 0 || nc_max > kMaxCells)
        return fail(DPEP_ERR_ARG, "nc_max=%d must be in [0, %d]", nc_max, kMaxCells);
    if (!(xh > xl) || !(yh > yl) || !isfinite(xl) || !isfinite(yl) ||
        !isfinite(xh) || !isfinite(yh))
        return fail(DPEP_ERR_ARG, "die [%g,%g]x[%g,%g] is empty or not finite",
                    xl, xh, yl, yh);
    if (flags & ~(DPEP_FLAG_DETERMINISTIC | DPEP_FLAG_NO_POTENTIAL |
                  DPEP_FLAG_NO_STRETCH | DPEP_FLAG_NO_GATHER | DPEP_FLAG_STEP_TIMINGS |
                  DPEP_FLAG_SCATTER_DENSITY | DPEP_FLAG_TWO_PASS))
        return fail(DPEP_ERR_ARG, "unknown flag bits 0x%x", flags);

    if (const hipError_t e = prepare_kernels())
        return fail(DPEP_ERR_HIP, "kernel attribute set-up failed: %s", hipGetErrorString(e));

    dpep_ctx* c = new (std::nothrow) dpep_ctx();
    if (!c) return fail(DPEP_ERR_NOMEM, "host allocation failed");
    c->M = M; c->N = N; c->nc_max = nc_max; c->dtype = dtype; c->flags = flags;
    c->esz = dtype == DPEP_DTYPE_F32 ? 4 : 8;
    make_grid(c->grid, M, N, xl, yl, xh, yh, !(flags & DPEP_FLAG_NO_STRETCH), nc_max,
              (int)c->esz);
    make_spectral_args(c->sargs, c->grid, dtype, !(flags & DPEP_FLAG_NO_POTENTIAL));
    const SpectralArgs& a = c->sargs;

    int rc = DPEP_OK;
    auto step = [&]() -> int {
        HIP_TRY(hipGetDevice(&c->device));
        HIP_TRY(hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking));
        // timing only (read after a stream synchronisation): no system-scope
        // fence when recorded, which would write back and invalidate the
        // caches between the kernels it brackets
        for (auto& e : c->ev) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
        HIP_TRY(hipEventCreate(&c->ev_x0));
        HIP_TRY(hipEventCreate(&c->ev_x1));
        const size_t mnb = (size_t)M * N * c->esz;
        const size_t ncb = (size_t)(nc_max > 0 ? nc_max : 1) * c->esz;
        void** cellbufs[] = {&c->d_px, &c->d_py, &c->d_sx, &c->d_sy, &c->d_gx, &c->d_gy};
        for (void** p : cellbufs) HIP_TRY(hipMalloc(p, ncb));
        void** mapbufs[] = {&c->d_d0n, &c->d_density, &c->d_fx, &c->d_fy,
                            &c->d_T, &c->d_Ux, &c->d_Uy};
        for (void** p : mapbufs) HIP_TRY(hipMalloc(p, mnb));
        if (a.potential) HIP_TRY(hipMalloc(&c->d_potential, mnb));
        if (flags & DPEP_FLAG_SCATTER_DENSITY) HIP_TRY(hipMalloc(&c->d_raw, mnb));
        HIP_TRY(hipMemset(c->d_d0n, 0, mnb));
        // strip binning
        const size_t accb = sizeof(unsigned long long);
        BinPlan& p = c->plan;
        p = make_bin_plan(M, N, nc_max, c->esz);
        BinArgs& b = c->bins;
        b.S = p.S; b.R = p.R; b.lgR = p.lgR; b.G1 = 1; b.ch_force = 0;
        b.raw = c->d_raw;
        {
            int acc = 0, gat = 0, cus = 0;
            HIP_TRY(dtype == DPEP_DTYPE_F32 ? bin_occupancy<float>(N, p.R, acc, gat)
                                            : bin_occupancy<double>(N, p.R, acc, gat));
            HIP_TRY(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount,
                                          c->device));
            set_item_grids(b, acc, gat, cus);
        }
        HIP_TRY(hipMalloc((void**)&b.cnt, (size_t)p.G1max * p.S * sizeof(unsigned)));
        // two sets of (slot, strip) counts: this step's and the last one's
        HIP_TRY(hipMalloc((void**)&b.xtot, 2 * (size_t)kCountSlots * p.S * sizeof(unsigned)));
        HIP_TRY(hipMemset(b.xtot, 0, 2 * (size_t)kCountSlots * p.S * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.pbase, (size_t)kCountSlots * p.S * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.pcap, (size_t)kCountSlots * p.S * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.pool_n, 2 * sizeof(unsigned)));
        HIP_TRY(hipMemset(b.pool_n, 0, 2 * sizeof(unsigned)));
        // records: the plan's regions, then an overflow pool of one slot per
        // possible record
        b.reg_cap = (unsigned)p.reg_cap;
        b.pool0 = (unsigned)p.reg_cap;
        b.pool_cap = (unsigned)p.cap;
        const size_t nrec = p.reg_cap + p.cap;
        HIP_TRY(hipMalloc((void**)&b.ovst, 2 * (size_t)p.S * sizeof(unsigned long long)));
        HIP_TRY(hipMemset(b.ovst, 0, 2 * (size_t)p.S * sizeof(unsigned long long)));
        b.rmax = run_capacity(nc_max);
        HIP_TRY(hipMalloc((void**)&b.oruns, (size_t)p.S * b.rmax * sizeof(uint2)));
        HIP_TRY(hipMalloc((void**)&b.items, (size_t)b.Wacc * sizeof(uint4)));
        HIP_TRY(hipMalloc((void**)&b.items_g, (size_t)b.Wgat * sizeof(uint4)));
        HIP_TRY(hipMalloc((void**)&b.nitems, 2 * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.chunk, 2 * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.done, (size_t)p.S * sizeof(unsigned)));
        HIP_TRY(hipMemset(b.done, 0, (size_t)p.S * sizeof(unsigned)));
        HIP_TRY(hipMalloc(&b.recg, nrec * p.geo_bytes));
        HIP_TRY(hipMalloc((void**)&b.recm, (p.span_bytes ? nrec : 1) * sizeof(unsigned)));
        HIP_TRY(hipMalloc((void**)&b.pos, (size_t)(nc_max > 0 ? nc_max : 1) * sizeof(unsigned long long)));
        HIP_TRY(hipMalloc(&b.gtmp, nrec * 2 * c->esz));
        HIP_TRY(hipMalloc((void**)&b.bigflag, (size_t)kSideWords * p.S * sizeof(unsigned)));
        HIP_TRY(hipMalloc(&b.B, (size_t)M * N * accb));
        // B and the strip flags must start at zero; each step leaves them so.
        HIP_TRY(hipMemset(b.B, 0, (size_t)M * N * accb));
        HIP_TRY(hipMemset(b.bigflag, 0, (size_t)kSideWords * p.S * sizeof(unsigned)));
        HIP_TRY(hipDeviceSynchronize());
        return dtype == DPEP_DTYPE_F32 ? make_tables<float>(c) : make_tables<double>(c);
    };
    rc = step();
    if (rc != DPEP_OK) {
        release(c);
        delete c;
        return rc;
    }
    *out = c;
    return DPEP_OK;
}

int dpep_destroy(dpep_ctx* c)
{
    if (!c) return DPEP_OK;
    if (c->stream) (void)hipStreamSynchronize(c->stream);
    release(c);
    delete c;
    return DPEP_OK;
}

int dpep_set_initial_density(dpep_ctx* c, const void* d0n)
{
    if (int rc = check_ctx(c)) return rc;
    if (!d0n) return fail(DPEP_ERR_ARG, "initial density pointer is NULL");
    const size_t bytes = (size_t)c->M * c->N * c->esz;
    HIP_TRY(hipMemcpyAsync(c->d_d0n, d0n, bytes, hipMemcpyHostToDevice, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return DPEP_OK;
}

int dpep_set_fixed_cells(dpep_ctx* c, const void* px, const void* py,
                         const void* sx, const void* sy, int n,
                         double target_density)
{
    if (int rc = check_ctx(c)) return rc;
    if (n < 0) return fail(DPEP_ERR_ARG, "n=%d must be >= 0", n);
    if (n > 0 && (!px || !py || !sx || !sy))
        return fail(DPEP_ERR_ARG, "fixed-cell array is NULL");
    if (!isfinite(target_density) || target_density < 0.0)
        return fail(DPEP_ERR_ARG, "target_density=%g must be finite and >= 0",
                    target_density);
    // one-time set-up: the fixed cells get their own device copy for the call
    void* buf = nullptr;
    const size_t bytes = (size_t)(n > 0 ? n : 1) * c->esz;
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMalloc(&buf, 4 * bytes));
    char* d = static_cast<char*>(buf);
    int rc = DPEP_OK;
    auto run = [&]() -> int {
        if (n > 0) {
            HIP_TRY(hipMemcpyAsync(d, px, (size_t)n * c->esz, hipMemcpyHostToDevice, c->stream));
            HIP_TRY(hipMemcpyAsync(d + bytes, py, (size_t)n * c->esz, hipMemcpyHostToDevice,
                                   c->stream));
            HIP_TRY(hipMemcpyAsync(d + 2 * bytes, sx, (size_t)n * c->esz,
                                   hipMemcpyHostToDevice, c->stream));
            HIP_TRY(hipMemcpyAsync(d + 3 * bytes, sy, (size_t)n * c->esz,
                                   hipMemcpyHostToDevice, c->stream));
        }
        if (c->dtype == DPEP_DTYPE_F32)
            HIP_TRY(launch_fixed_density<float>((const float*)d, (const float*)(d + bytes),
                                                (const float*)(d + 2 * bytes),
                                                (const float*)(d + 3 * bytes), n, c->grid,
                                                target_density, c->bins.B,
                                                (float*)c->d_d0n, c->stream));
        else
            HIP_TRY(launch_fixed_density<double>((const double*)d, (const double*)(d + bytes),
                                                 (const double*)(d + 2 * bytes),
                                                 (const double*)(d + 3 * bytes), n, c->grid,
                                                 target_density, c->bins.B,
                                                 (double*)c->d_d0n, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
        return DPEP_OK;
    };
    rc = run();
    (void)hipFree(buf);
    return rc;
}

int dpep_set_cells(dpep_ctx* c, const void* px, const void* py,
                   const void* sx, const void* sy, int nc)
{
    if (int rc = check_ctx(c)) return rc;
    if (nc < 0 || nc > c->nc_max)
        return fail(DPEP_ERR_ARG, "nc=%d outside [0, nc_max=%d]", nc, c->nc_max);
    const bool keep_sizes = !sx && !sy;      // positions only
    if (nc > 0 && (!px || !py || (!keep_sizes && (!sx || !sy))))
        return fail(DPEP_ERR_ARG, "cell array is NULL");
    if (keep_sizes && nc > c->nc_sizes)
        return fail(DPEP_ERR_STATE,
                    "sizes kept (sx, sy NULL) for nc=%d cells, but only %d have resident sizes",
                    nc, c->nc_sizes);
    const size_t bytes = (size_t)nc * c->esz;
    HIP_TRY(hipEventRecord(c->ev_x0, c->stream));
    if (nc > 0) {
        HIP_TRY(hipMemcpyAsync(c->d_px, px, bytes, hipMemcpyHostToDevice, c->stream));
        HIP_TRY(hipMemcpyAsync(c->d_py, py, bytes, hipMemcpyHostToDevice, c->stream));
        if (!keep_sizes) {
            // the sizes change: none stay valid until the copies are in
            c->nc_sizes = 0;
            HIP_TRY(hipMemcpyAsync(c->d_sx, sx, bytes, hipMemcpyHostToDevice, c->stream));
            HIP_TRY(hipMemcpyAsync(c->d_sy, sy, bytes, hipMemcpyHostToDevice, c->stream));
        }
    }
    HIP_TRY(hipEventRecord(c->ev_x1, c->stream));
    HIP_TRY(hipEventSynchronize(c->ev_x1));
    c->h2d_ms = elapsed(c->ev_x0, c->ev_x1);
    if (!keep_sizes) c->nc_sizes = nc;
    c->nc = nc;
    c->valid = 0u;          // the outputs no longer describe the resident cells
    return DPEP_OK;
}

int dpep_compute(dpep_ctx* c)
{
    if (int rc = check_ctx(c)) return rc;
    if (c->nc < 0) return fail(DPEP_ERR_STATE, "dpep_set_cells was not called");
    return step_dispatch(c, c->d_px, c->d_py, c->d_sx, c->d_sy, c->nc, nullptr,
                         nullptr, nullptr, nullptr, nullptr, nullptr, c->stream);
}

int dpep_sync(dpep_ctx* c)
{
    if (int rc = check_ctx(c)) return rc;
    HIP_TRY(hipStreamSynchronize(c->stream));
    return DPEP_OK;
}

int dpep_get_outputs(dpep_ctx* c, void* density, void* potential,
                     void* field_x, void* field_y, void* grad_x, void* grad_y)
{
    if (int rc = check_ctx(c)) return rc;
    if (!c->stepped) return fail(DPEP_ERR_STATE, "no step has been computed");
    if (potential && !c->d_potential)
        return fail(DPEP_ERR_STATE, "context was created with DPEP_FLAG_NO_POTENTIAL");
    if ((grad_x || grad_y) && (c->flags & DPEP_FLAG_NO_GATHER))
        return fail(DPEP_ERR_STATE, "context was created with DPEP_FLAG_NO_GATHER");
    {
        const unsigned want = (density ? kOutDensity : 0u) | (potential ? kOutPotential : 0u) |
                              (field_x ? kOutFx : 0u) | (field_y ? kOutFy : 0u) |
                              (grad_x ? kOutGx : 0u) | (grad_y ? kOutGy : 0u);
        if (want & ~c->valid)
            return fail(DPEP_ERR_STATE,
                        "the context's outputs are stale: cells were uploaded after the "
                        "last step, or the last step wrote to caller-owned device buffers "
                        "(requested mask 0x%x, valid 0x%x)", want, c->valid);
    }
    const size_t mnb = (size_t)c->M * c->N * c->esz;
    const size_t ncb = (size_t)c->last_nc * c->esz;
    hipStream_t s = c->stream;
    HIP_TRY(hipEventRecord(c->ev_x0, s));
    if (density) HIP_TRY(hipMemcpyAsync(density, c->d_density, mnb, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipEventRecord(c->ev_x1, s));
    HIP_TRY(hipEventSynchronize(c->ev_x1));
    c->d2h_den_ms = elapsed(c->ev_x0, c->ev_x1);
    HIP_TRY(hipEventRecord(c->ev_x0, s));
    if (potential) HIP_TRY(hipMemcpyAsync(potential, c->d_potential, mnb, hipMemcpyDeviceToHost, s));
    if (field_x) HIP_TRY(hipMemcpyAsync(field_x, c->d_fx, mnb, hipMemcpyDeviceToHost, s));
    if (field_y) HIP_TRY(hipMemcpyAsync(field_y, c->d_fy, mnb, hipMemcpyDeviceToHost, s));
    if (grad_x && ncb) HIP_TRY(hipMemcpyAsync(grad_x, c->d_gx, ncb, hipMemcpyDeviceToHost, s));
    if (grad_y && ncb) HIP_TRY(hipMemcpyAsync(grad_y, c->d_gy, ncb, hipMemcpyDeviceToHost, s));
    HIP_TRY(hipEventRecord(c->ev_x1, s));
    HIP_TRY(hipEventSynchronize(c->ev_x1));
    c->d2h_out_ms = elapsed(c->ev_x0, c->ev_x1);
    return DPEP_OK;
}

int dpep_get_scatter_density(dpep_ctx* c, void* out)
{
    if (int rc = check_ctx(c)) return rc;
    if (!out) return fail(DPEP_ERR_ARG, "out is NULL");
    if (!c->d_raw)
        return fail(DPEP_ERR_STATE, "context was created without DPEP_FLAG_SCATTER_DENSITY");
    if (!c->stepped || !(c->valid & kOutRaw))
        return fail(DPEP_ERR_STATE, "no step has been computed on the resident cells");
    HIP_TRY(hipMemcpyAsync(out, c->d_raw, (size_t)c->M * c->N * c->esz,
                           hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    return DPEP_OK;
}

int dpep_host_alloc(size_t bytes, void** out)
{
    if (!out) return fail(DPEP_ERR_ARG, "out is NULL");
    *out = nullptr;
    if (bytes == 0) bytes = 1;
    const hipError_t e = hipHostMalloc(out, bytes, hipHostMallocDefault);
    if (e != hipSuccess) {
        *out = nullptr;
        return fail(DPEP_ERR_NOMEM, "hipHostMalloc(%zu) failed: %s", bytes,
                    hipGetErrorString(e));
    }
    return DPEP_OK;
}

int dpep_host_free(void* p)
{
    if (p) HIP_TRY(hipHostFree(p));
    return DPEP_OK;
}

int dpep_step(dpep_ctx* c, const void* px, const void* py, const void* sx,
              const void* sy, int nc, void* field_x, void* field_y,
              void* density, void* potential, void* grad_x, void* grad_y)
{
    int rc = dpep_set_cells(c, px, py, sx, sy, nc);
    if (rc) return rc;
    if ((rc = dpep_compute(c))) return rc;
    return dpep_get_outputs(c, density, potential, field_x, field_y, grad_x,
                            grad_y);
}

int dpep_step_device(dpep_ctx* c, const void* d_px, const void* d_py,
                     const void* d_sx, const void* d_sy, int nc,
                     void* d_field_x, void* d_field_y, void* d_density,
                     void* d_potential, void* d_grad_x, void* d_grad_y,
                     void* stream)
{
    if (int rc = check_ctx(c)) return rc;
    if (nc < 0 || nc > c->nc_max)
        return fail(DPEP_ERR_ARG, "nc=%d outside [0, nc_max=%d]", nc, c->nc_max);
    if (nc > 0 && (!d_px || !d_py || !d_sx || !d_sy))
        return fail(DPEP_ERR_ARG, "cell array is NULL");
    if (d_potential && !c->sargs.potential)
        return fail(DPEP_ERR_STATE, "context was created with DPEP_FLAG_NO_POTENTIAL");
    hipStream_t s = stream ? (hipStream_t)stream : c->stream;
    return step_dispatch(c, d_px, d_py, d_sx, d_sy, nc, d_field_x, d_field_y,
                         d_density, d_potential, d_grad_x, d_grad_y, s);
}

int dpep_get_timings(dpep_ctx* c, float* out)
{
    if (int rc = check_ctx(c)) return rc;
    if (!out) return fail(DPEP_ERR_ARG, "out is NULL");
    if (!c->stepped) return fail(DPEP_ERR_STATE, "no step has been computed");
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (int i = 0; i < DPEP_NUM_TIMINGS; ++i) out[i] = 0.f;
    const float total = (c->flags & DPEP_FLAG_STEP_TIMINGS)
                            ? elapsed(c->ev[0], c->ev[kNumStages]) : 0.f;
    out[0] = c->h2d_ms;
    if (c->profiling && c->prof_steps > 0) {
        const size_t slot = (size_t)((c->prof_steps - 1) % c->prof_slots);
        const hipEvent_t* pe = &c->prof_ev[slot * 2 * kNumStages];
        const unsigned mask = c->prof_mask[slot];
        // binning (from K1, or K3 on a one-pass step), accumulation and P1
        out[1] = elapsed(pe[(mask & 1u) ? 0 : 2], pe[5]);
        out[5] = elapsed(pe[6], pe[9]);              // P2 + P3
        out[2] = (mask & 0x60u) ? elapsed(pe[10], pe[13]) : 0.f;   // gather
    } else {
        out[5] = total;
    }
    out[3] = c->d2h_den_ms;
    out[6] = c->d2h_out_ms;
    out[8] = c->h2d_ms + total + c->d2h_den_ms + c->d2h_out_ms;
    return DPEP_OK;
}

int dpep_get_binning_stats(dpep_ctx* c, long long* out, int n)
{
    if (int rc = check_ctx(c)) return rc;
    if (!out || n < 0) return fail(DPEP_ERR_ARG, "bad output buffer");
    if (!c->stepped) return fail(DPEP_ERR_STATE, "no step has been computed");
    HIP_TRY(hipStreamSynchronize(c->last_stream ? c->last_stream : c->stream));
    const BinArgs& b = c->bins;
    // the last step's set of counts and pool count stay until the next
    // step's accumulation re-zeroes them
    std::vector<unsigned> tot((size_t)kCountSlots * b.S);
    std::vector<unsigned long long> ost((size_t)b.S);
    unsigned pool = 0, items[2] = {0, 0}, chunk[2] = {0, 0};
    HIP_TRY(hipMemcpy(tot.data(), b.xtot + (size_t)(c->last_par & 1) * kCountSlots * b.S,
                      tot.size() * sizeof(unsigned), hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(ost.data(), b.ovst + (size_t)(c->last_par & 1) * b.S,
                      ost.size() * sizeof(unsigned long long), hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(&pool, b.pool_n + (c->last_par & 1), sizeof(unsigned),
                      hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(items, b.nitems, sizeof items, hipMemcpyDeviceToHost));
    HIP_TRY(hipMemcpy(chunk, b.chunk, sizeof chunk, hipMemcpyDeviceToHost));
    long long recs = 0, runs = 0;
    for (unsigned t : tot) recs += t;
    for (unsigned long long o : ost) runs = (long long)(o >> 32) > runs ? (long long)(o >> 32) : runs;
    const long long v[DPEP_NUM_BIN_STATS] = {c->last_once, recs, c->last_once ? (long long)pool : 0,
                                             items[0], items[1], chunk[0], chunk[1],
                                             c->last_once ? runs : 0};
    for (int i = 0; i < n; ++i) out[i] = i < DPEP_NUM_BIN_STATS ? v[i] : 0;
    return DPEP_OK;
}

int dpep_get_kernel_times(dpep_ctx* c, float* out, int n)
{
    if (int rc = check_ctx(c)) return rc;
    if (!out || n < 0) return fail(DPEP_ERR_ARG, "bad output buffer");
    if (!c->stepped) return fail(DPEP_ERR_STATE, "no step has been computed");
    if (!c->profiling || c->prof_steps == 0)
        return fail(DPEP_ERR_STATE,
                    "no profiled step: call dpep_set_profiling(ctx, slots) first");
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (int i = 0; i < n; ++i) out[i] = 0.f;
    const long steps = c->prof_steps < c->prof_slots ? c->prof_steps : c->prof_slots;
    for (long k = 0; k < steps; ++k) {
        const hipEvent_t* pe = &c->prof_ev[(size_t)k * 2 * kNumStages];
        const unsigned mask = c->prof_mask[(size_t)k];
        // each kernel's own (start, end); a kernel the step did not launch
        // (K1 on a one-pass step, the gather when off) adds nothing
        int first = -1, last = -1;
        for (int i = 0; i < kNumStages; ++i) {
            if (!((mask >> i) & 1u)) continue;
            if (first < 0) first = i;
            last = i;
            if (i < n) out[i] += 1000.f * elapsed(pe[2 * i], pe[2 * i + 1]);
        }
        if (n > kNumStages && first >= 0)
            out[kNumStages] += 1000.f * elapsed(pe[2 * first], pe[2 * last + 1]);
    }
    for (int i = 0; i < n && i <= kNumStages; ++i) out[i] /= (float)steps;
    return DPEP_OK;
}

int dpep_set_profiling(dpep_ctx* c, int slots)
{
    if (int rc = check_ctx(c)) return rc;
    if (slots < 0 || slots > 65536)
        return fail(DPEP_ERR_ARG, "slots=%d outside [0, 65536]", slots);
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (auto& e : c->prof_ev)
        if (e) (void)hipEventDestroy(e);
    c->prof_ev.clear();
    c->profiling = 0;
    c->prof_slots = 0;
    c->prof_steps = 0;
    if (slots == 0) return DPEP_OK;
    c->prof_ev.assign((size_t)slots * 2 * kNumStages, nullptr);
    c->prof_mask.assign((size_t)slots, 0);
    for (auto& e : c->prof_ev)      // timing only, as the step's events
        HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    c->prof_slots = slots;
    c->profiling = 1;
    return DPEP_OK;
}

}  // extern "C"
