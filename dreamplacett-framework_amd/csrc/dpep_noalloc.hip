// dpep_noalloc.hip -- dpep_step_device_noalloc: one electric-potential step
// on caller-owned device memory that allocates nothing, for callers that
// cannot call hipMalloc (code under HIP graph capture, fixed serving loops).
//
// Every scratch buffer of the step (twiddle tables, the transform
// intermediates T / Ux / Uy, the side map B, the strip tables and work-item
// lists, the strip-sorted records, the cell-to-record map and the partial
// forces) is carved from `scratch`, a file-scope device array of
// kScratchBytes, of which each GPU the library runs on holds its own copy
// until the process ends.  Its device address is looked up once per device
// (hipGetSymbolAddress, on the first call with that device current) and
// only that address is handed to kernels and fills.  Every call on one GPU
// shares the array: calls that overlap on one GPU (two streams, two
// threads) race and must be serialised by the caller.  The regions that must
// start at zero are cleared by a fill kernel on the caller's stream at the
// start of each call (no hipMemsetAsync, so the call can be captured).
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "dpep.h"
#include "dpep_internal.h"

using namespace dpep;

namespace {

constexpr size_t kScratchBytes = (size_t)64 << 20;
constexpr int kMaxDevices = 64;

}  // namespace

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

namespace {

std::mutex g_mu;
void* g_base[kMaxDevices];       // device address of `scratch` per GPU
int g_cus[kMaxDevices];          // compute units per GPU

int failf(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int failf(int code, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    return report_error(code, buf);
}

#define NA_TRY(expr)                                                          \
    do {                                                                      \
        const hipError_t e_ = (expr);                                         \
        if (e_ != hipSuccess)                                                 \
            return failf(DPEP_ERR_HIP, "dpep_step_device_noalloc: %s failed: %s", \
                         #expr, hipGetErrorString(e_));                        \
    } while (0)

// Offsets into the scratch array, each region 256-byte aligned.
struct Carve {
    size_t end = 0;
    size_t take(size_t bytes)
    {
        const size_t at = end;
        end += (bytes + 255) & ~(size_t)255;
        return at;
    }
};

// The scratch layout of one call.  The regions that must start at zero (slot
// totals, the overflow counts, chunk tickets, side-map marks, the side map,
// and the zero initial density when the caller passes none) come first, in
// one run.  Every call counts before it sorts (no counts survive between
// calls), so the records need no overflow pool.
struct Layout {
    size_t xtot, pool_n, ovst, done, bigflag, B, d0zero, zero_end;
    size_t twM, postM, twN, postN, T, Ux, Uy;
    size_t cnt, pbase, pcap, oruns, items, items_g, nitems, chunk;
    size_t recg, recm, pos, gtmp;
    size_t total;
};

Layout plan_layout(int M, int N, int nc, size_t esz, const BinPlan& p, const BinArgs& b,
                   bool zero_d0)
{
    const size_t mn = (size_t)M * N;
    const size_t ncs = (size_t)(nc > 0 ? nc : 1);
    Carve c;
    Layout l{};
    l.xtot = c.take(2 * (size_t)kCountSlots * p.S * sizeof(unsigned));
    l.pool_n = c.take(2 * sizeof(unsigned));
    l.ovst = c.take(2 * (size_t)p.S * sizeof(unsigned long long));
    l.done = c.take((size_t)p.S * sizeof(unsigned));
    l.bigflag = c.take((size_t)kSideWords * p.S * sizeof(unsigned));
    l.B = c.take(mn * sizeof(unsigned long long));
    l.d0zero = zero_d0 ? c.take(mn * esz) : 0;
    l.zero_end = c.end;
    l.twM = c.take(twiddle_elems(M) * esz);
    l.postM = c.take(post_elems(M) * esz);
    l.twN = c.take(twiddle_elems(N) * esz);
    l.postN = c.take(post_elems(N) * esz);
    l.T = c.take(mn * esz);
    l.Ux = c.take(mn * esz);
    l.Uy = c.take(mn * esz);
    l.cnt = c.take((size_t)p.G1max * p.S * sizeof(unsigned));
    l.pbase = c.take((size_t)kCountSlots * p.S * sizeof(unsigned));
    l.pcap = c.take((size_t)kCountSlots * p.S * sizeof(unsigned));
    l.oruns = c.take(sizeof(uint2));
    l.items = c.take((size_t)b.Wacc * sizeof(uint4));
    l.items_g = c.take((size_t)b.Wgat * sizeof(uint4));
    l.nitems = c.take(2 * sizeof(unsigned));
    l.chunk = c.take(2 * sizeof(unsigned));
    l.recg = c.take(p.cap * p.geo_bytes);
    l.recm = c.take((p.span_bytes ? p.cap : 1) * sizeof(unsigned));
    l.pos = c.take(ncs * sizeof(unsigned long long));
    l.gtmp = c.take(p.cap * 2 * esz);
    l.total = c.end;
    return l;
}

__global__ __launch_bounds__(256) void k_zero(uint4* __restrict__ p, size_t n16)
{
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16;
         i += (size_t)gridDim.x * 256)
        p[i] = uint4{0u, 0u, 0u, 0u};
}

template <typename T>
int run(int M, int N, const Grid& g, int dtype, bool potential, bool gather, int nc,
        const void* d0n, const void* px, const void* py, const void* sx, const void* sy,
        void* fx, void* fy, void* dens, void* phi, void* gx, void* gy, hipStream_t s)
{
    int dev = 0;
    NA_TRY(hipGetDevice(&dev));
    if (dev < 0 || dev >= kMaxDevices)
        return failf(DPEP_ERR_UNSUPPORTED, "dpep_step_device_noalloc: device %d beyond %d",
                     dev, kMaxDevices);
    void* base = nullptr;
    int cus = 0;
    {
        std::lock_guard<std::mutex> lock(g_mu);
        if (!g_base[dev]) {
            // once per device, with it current: the array's address on it
            void* p = nullptr;
            NA_TRY(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
            int n = 0;
            NA_TRY(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
            g_cus[dev] = n;
            g_base[dev] = p;
        }
        base = g_base[dev];
        cus = g_cus[dev];
    }
    NA_TRY(prepare_kernels());

    const size_t esz = sizeof(T);
    const BinPlan p = make_bin_plan(M, N, nc, esz);
    BinArgs b{};
    b.S = p.S; b.R = p.R; b.lgR = p.lgR; b.G1 = 1; b.ch_force = 0;
    {
        int acc = 0, gat = 0;
        NA_TRY(bin_occupancy<T>(N, p.R, acc, gat));
        set_item_grids(b, acc, gat, cus);
    }
    const Layout l = plan_layout(M, N, nc, esz, p, b, d0n == nullptr);
    if (l.total > kScratchBytes)
        return failf(DPEP_ERR_ARG,
                     "dpep_step_device_noalloc: %dx%d bins and %d cells (%s) need %.1f MiB "
                     "of scratch, above the %zu MiB it holds; use dpep_create and "
                     "dpep_step_device", M, N, nc, esz == 4 ? "float32" : "float64",
                     (double)l.total / 1048576.0, kScratchBytes >> 20);
    char* sc = static_cast<char*>(base);
    b.xtot = (unsigned*)(sc + l.xtot);
    b.done = (unsigned*)(sc + l.done);
    b.bigflag = (unsigned*)(sc + l.bigflag);
    b.B = sc + l.B;
    b.cnt = (unsigned*)(sc + l.cnt);
    b.pool_n = (unsigned*)(sc + l.pool_n);
    b.pbase = (unsigned*)(sc + l.pbase);
    b.pcap = (unsigned*)(sc + l.pcap);
    b.ovst = (unsigned long long*)(sc + l.ovst);
    b.oruns = (uint2*)(sc + l.oruns);
    b.rmax = 1;
    b.reg_cap = (unsigned)p.cap;
    b.pool0 = (unsigned)p.cap;
    b.pool_cap = 0u;
    b.par = 0;
    b.items = (uint4*)(sc + l.items);
    b.items_g = (uint4*)(sc + l.items_g);
    b.nitems = (unsigned*)(sc + l.nitems);
    b.chunk = (unsigned*)(sc + l.chunk);
    b.recg = sc + l.recg;
    b.recm = (unsigned*)(sc + l.recm);
    b.pos = (unsigned long long*)(sc + l.pos);
    b.gtmp = sc + l.gtmp;
    b.raw = nullptr;
    const T* d0 = d0n ? (const T*)d0n : (const T*)(sc + l.d0zero);
    T* Tt = (T*)(sc + l.T);
    T* Ux = (T*)(sc + l.Ux);
    T* Uy = (T*)(sc + l.Uy);

    SpectralArgs a;
    make_spectral_args(a, g, dtype, potential);
    a.twM = sc + l.twM;
    a.postM = sc + l.postM;
    a.twN = sc + l.twN;
    a.postN = sc + l.postN;

    // the zero-start regions, then the tables, then the step
    const size_t n16 = l.zero_end / 16;
    const size_t blocks = (n16 + 255) / 256;
    k_zero<<<(unsigned)(blocks < 4096 ? (blocks > 0 ? blocks : 1) : 4096), 256, 0, s>>>(
        (uint4*)sc, n16);
    NA_TRY(hipGetLastError());
    NA_TRY(launch_tables<T>(M, (T*)(sc + l.twM), (T*)(sc + l.postM), s));
    NA_TRY(launch_tables<T>(N, (T*)(sc + l.twN), (T*)(sc + l.postN), s));
    NA_TRY(launch_bin_scatter<T>((const T*)px, (const T*)py, (const T*)sx, (const T*)sy, nc,
                                 g, b, a, d0, (T*)dens, Tt, false, s, nullptr));
    NA_TRY(launch_col_pass<T>(a, Tt, Ux, Uy, s));
    NA_TRY(launch_row_inv<T>(a, Ux, Uy, (T*)fx, (T*)fy, (T*)phi, s));
    if (gather)
        NA_TRY(launch_bin_gather<T>((const T*)px, (const T*)py, (const T*)sx, (const T*)sy, nc,
                                    g, b, (const T*)fx, (const T*)fy, (T*)gx, (T*)gy, s,
                                    nullptr));
    return DPEP_OK;
}

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

}  // namespace

extern "C" int dpep_step_device_noalloc(int num_bins_x, int num_bins_y, double xl,
                                        double yl, double xh, double yh, int dtype,
                                        unsigned flags, int nc_max,
                                        const void* d_initial_density, const void* d_px,
                                        const void* d_py, const void* d_sx,
                                        const void* d_sy, int nc, void* d_field_x,
                                        void* d_field_y, void* d_density,
                                        void* d_potential, void* d_grad_x,
                                        void* d_grad_y, void* stream)
{
    const int M = num_bins_x, N = num_bins_y;
    if (dtype != DPEP_DTYPE_F32 && dtype != DPEP_DTYPE_F64)
        return failf(DPEP_ERR_ARG, "dtype must be DPEP_DTYPE_F32 or DPEP_DTYPE_F64");
    const int maxL = dtype == DPEP_DTYPE_F32 ? 8192 : 4096;
    if (!is_pow2(M) || !is_pow2(N) || M < 8 || N < 8 || M > maxL || N > maxL)
        return failf(DPEP_ERR_UNSUPPORTED,
                     "num_bins_x=%d num_bins_y=%d: both must be powers of two in [8, %d]", M,
                     N, maxL);
    if (flags & ~(DPEP_FLAG_DETERMINISTIC | DPEP_FLAG_NO_POTENTIAL | DPEP_FLAG_NO_STRETCH |
                  DPEP_FLAG_NO_GATHER))
        return failf(DPEP_ERR_ARG, "flag bits 0x%x are not available without a context",
                     flags);
    if (nc_max < 0 || nc < 0 || nc > nc_max)
        return failf(DPEP_ERR_ARG, "nc=%d and nc_max=%d: need 0 <= nc <= nc_max", nc, nc_max);
    if (!(xh > xl) || !(yh > yl) || !isfinite(xl) || !isfinite(yl) || !isfinite(xh) ||
        !isfinite(yh))
        return failf(DPEP_ERR_ARG, "die [%g,%g]x[%g,%g] is empty or not finite", xl, xh, yl,
                     yh);
    const bool potential = !(flags & DPEP_FLAG_NO_POTENTIAL);
    const bool gather = !(flags & DPEP_FLAG_NO_GATHER);
    if (nc > 0 && (!d_px || !d_py || !d_sx || !d_sy))
        return failf(DPEP_ERR_ARG, "cell array is NULL");
    if (!d_field_x || !d_field_y || !d_density || (potential && !d_potential) ||
        (gather && (!d_grad_x || !d_grad_y)))
        return failf(DPEP_ERR_ARG, "an output this step computes is NULL (there are no "
                                   "context buffers to fall back on)");
    Grid g;
    const int esz = dtype == DPEP_DTYPE_F32 ? 4 : 8;
    make_grid(g, M, N, xl, yl, xh, yh, !(flags & DPEP_FLAG_NO_STRETCH), nc_max, esz);
    hipStream_t s = (hipStream_t)stream;
    if (dtype == DPEP_DTYPE_F32)
        return run<float>(M, N, g, dtype, potential, gather, nc, d_initial_density, d_px, d_py,
                          d_sx, d_sy, d_field_x, d_field_y, d_density, d_potential, d_grad_x,
                          d_grad_y, s);
    return run<double>(M, N, g, dtype, potential, gather, nc, d_initial_density, d_px, d_py,
                       d_sx, d_sy, d_field_x, d_field_y, d_density, d_potential, d_grad_x,
                       d_grad_y, s);
}
