// dpep_bin.hip -- host launchers of the strip-binned scatter and gather
// (kernels in dpep_bin.h).
#include <math.h>

#include <type_traits>

#include "dpep_bin.h"

namespace dpep {

// k_strip_acc is instantiated per row length N (its row DCT is templated).
template <typename T, typename Fn>
static hipError_t dispatch_n(int N, Fn&& fn)
{
    switch (N) {
    case 8: return fn(std::integral_constant<int, 8>{});
    case 16: return fn(std::integral_constant<int, 16>{});
    case 32: return fn(std::integral_constant<int, 32>{});
    case 64: return fn(std::integral_constant<int, 64>{});
    case 128: return fn(std::integral_constant<int, 128>{});
    case 256: return fn(std::integral_constant<int, 256>{});
    case 512: return fn(std::integral_constant<int, 512>{});
    case 1024: return fn(std::integral_constant<int, 1024>{});
    case 2048: return fn(std::integral_constant<int, 2048>{});
    case 4096: return fn(std::integral_constant<int, 4096>{});
    case 8192:
        if constexpr (sizeof(T) == 4) return fn(std::integral_constant<int, 8192>{});
        else return hipErrorInvalidValue;
    default: return hipErrorInvalidValue;
    }
}

template <typename T>
hipError_t launch_bin_scatter(const T* px, const T* py, const T* sx,
                              const T* sy, int nc, const Grid& g,
                              BinArgs b, const SpectralArgs& a, const T* d0n, T* dens,
                              T* Tt, bool once, hipStream_t s, const hipEvent_t* ev)
{
    const OnceBlocks ob = once_blocks(nc, b.cus, sizeof(T));
    set_count_blocks(b, ob);
    if (b.R != strip_rows(g.N)) return hipErrorInvalidValue;   // the kernel's R
    // a one-pass step needs an overflow pool for all its records and room in
    // every strip's run table for one run per block
    if (once && (b.pool_cap < 2u * (unsigned)(nc > 0 ? nc : 0) || ob.grid > b.rmax))
        return hipErrorInvalidValue;
    hipError_t e;
    const hipEvent_t* ev1 = ev ? ev + 0 : nullptr;     // K1
    const hipEvent_t* ev3 = ev ? ev + 2 : nullptr;     // K3
    const hipEvent_t* ev4 = ev ? ev + 4 : nullptr;     // K4
    if (once) {
        if ((e = with_cpt(ob.cpt, [&](auto c) -> hipError_t {
                 constexpr int CPT = decltype(c)::value;
                 DPEP_LAUNCH(ev3, (k_bin_fill_once<T, CPT>), (unsigned)ob.grid, kOnceThreads,
                             fill_once_lds<T>(b.S), s, px, py, sx, sy, nc, g, b);
                 return hipSuccess;
             })))
            return e;
    } else {
        const size_t count_lds = (size_t)b.S * sizeof(unsigned);
        const bool staged = b.S >= kStageMinStrips;
        const size_t fill_lds =
            staged ? fill_lds_staged<T>(b.S)
                   : (size_t)(2 * b.S + kBinThreads + kChunkCands) * sizeof(unsigned);
        DPEP_LAUNCH(ev1, (k_bin_count<T>), b.G1, kBinThreads, count_lds, s, px, py, sx, sy,
                    nc, g, b);
        if ((e = hipGetLastError())) return e;
        if (staged)
            DPEP_LAUNCH(ev3, (k_bin_fill_staged<T>), b.G1, kBinThreads, fill_lds, s, px, py, sx,
                        sy, nc, g, b);
        else
            DPEP_LAUNCH(ev3, (k_bin_fill_direct<T>), b.G1, kBinThreads, fill_lds, s, px, py, sx,
                        sy, nc, g, b);
    }
    if ((e = hipGetLastError())) return e;
    return dispatch_n<T>(g.N, [&](auto lc) -> hipError_t {
        constexpr int L = decltype(lc)::value;
        DPEP_LAUNCH(ev4, (k_strip_acc<T, L>), b.Wacc, kAccThreads, (acc_lds_bytes<T, L>()), s, g,
                    b, a, d0n, dens, Tt);
        return hipGetLastError();
    });
}

template <typename T>
hipError_t launch_bin_gather(const T* px, const T* py, const T* sx,
                             const T* sy, int nc, const Grid& g,
                             const BinArgs& b, const T* fx, const T* fy,
                             T* gx, T* gy, hipStream_t s, const hipEvent_t* ev)
{
    if (nc <= 0) return hipSuccess;
    const size_t lds = gather_lds<T>(b.R, g.N);
    const hipEvent_t* evg1 = ev ? ev + 0 : nullptr;
    const hipEvent_t* evg2 = ev ? ev + 2 : nullptr;
    if (b.Wgat == b.S)      // one workgroup per strip: item w is mostly strip w
        DPEP_LAUNCH(evg1, (k_gather_bin<T, true>), b.Wgat, kAccThreads, lds, s, g, b, fx, fy);
    else
        DPEP_LAUNCH(evg1, (k_gather_bin<T, false>), b.Wgat, kAccThreads, lds, s, g, b, fx, fy);
    hipError_t e = hipGetLastError();
    if (e) return e;
    // the one-pass K3's cell blocks
    const OnceBlocks ob = once_blocks(nc, b.cus, sizeof(T));
    BinArgs bo = b;
    bo.qcells = ob.q;
    if ((e = with_cpt(ob.cpt, [&](auto c) -> hipError_t {
             constexpr int CPT = decltype(c)::value;
             DPEP_LAUNCH(evg2, (k_gather_out<T, kOnceThreads, CPT>), (unsigned)ob.grid,
                         kOnceThreads, (gather_out_lds<kOnceThreads, CPT>()), s, px, py, sx, sy,
                         nc, g, bo, fx, fy, gx, gy);
             return hipSuccess;
         })))
        return e;
    return hipGetLastError();
}

template <typename T>
hipError_t launch_fixed_density(const T* px, const T* py, const T* sx, const T* sy,
                                int n, const Grid& g, double target_density,
                                void* B, T* d0n, hipStream_t s)
{
    // contributions <= 1 bin area each, at most n of them per bin
    const double scale = ldexp(1.0, fix_exponent(n));
    unsigned long long* Bm = reinterpret_cast<unsigned long long*>(B);
    Grid gn = g;
    gn.stretch = 0;                    // fixed cells keep their own sizes
    if (n > 0) {
        k_fixed_overlap<T><<<(unsigned)n, kFixedThreads, 0, s>>>(px, py, sx, sy, n, gn,
                                                               scale, Bm);
        hipError_t e = hipGetLastError();
        if (e) return e;
    }
    const size_t mn = (size_t)g.M * g.N;
    k_fixed_flush<T><<<(unsigned)((mn + 255) / 256), 256, 0, s>>>(Bm, d0n, mn,
                                                                  target_density / scale);
    return hipGetLastError();
}

template <typename T>
hipError_t bin_occupancy(int N, int R, int& acc_per_cu, int& gat_per_cu)
{
    acc_per_cu = gat_per_cu = 0;
    hipError_t e = dispatch_n<T>(N, [&](auto lc) -> hipError_t {
        constexpr int L = decltype(lc)::value;
        return hipOccupancyMaxActiveBlocksPerMultiprocessor(
            &acc_per_cu, (const void*)k_strip_acc<T, L>, kAccThreads, acc_lds_bytes<T, L>());
    });
    if (e) return e;
    return hipOccupancyMaxActiveBlocksPerMultiprocessor(
        &gat_per_cu, (const void*)k_gather_bin<T, false>, kAccThreads, gather_lds<T>(R, N));
}

template <typename T>
static hipError_t prepare_bin_type()
{
    hipError_t e = hipSuccess;
    for (int N = 8; N <= (sizeof(T) == 4 ? 8192 : 4096) && !e; N *= 2)
        e = dispatch_n<T>(N, [&](auto lc) -> hipError_t {
            constexpr int L = decltype(lc)::value;
            return hipFuncSetAttribute((const void*)k_strip_acc<T, L>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)acc_lds_bytes<T, L>());
        });
    if (e) return e;
    // K3's LDS grows with the strips: at most 8192 / 2 (float32) or 4096 / 4
    if ((e = hipFuncSetAttribute((const void*)k_bin_fill_staged<T>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize,
                                 (int)fill_lds_staged<T>(sizeof(T) == 4 ? 4096 : 1024))))
        return e;
    // the one-pass K3's strip tables: at most 8192 * 8192 bins in 2-row strips
    for (int cpt = 2; cpt <= kOnceMaxCpt && !e; ++cpt)
        e = with_cpt(cpt, [&](auto c) -> hipError_t {
            constexpr int CPT = decltype(c)::value;
            return hipFuncSetAttribute((const void*)k_bin_fill_once<T, CPT>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)fill_once_lds<T>(4096));
        });
    if (e) return e;
    const int glds = (int)(kTileBytes + (size_t)kRunBatch * sizeof(uint2));
    if ((e = hipFuncSetAttribute((const void*)k_gather_bin<T, true>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, glds)))
        return e;
    return hipFuncSetAttribute((const void*)k_gather_bin<T, false>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, glds);
}

hipError_t bin_prepare()
{
    hipError_t e = prepare_bin_type<float>();
    if (e) return e;
    return prepare_bin_type<double>();
}

template hipError_t launch_bin_scatter<float>(const float*, const float*, const float*,
                                              const float*, int, const Grid&, BinArgs,
                                              const SpectralArgs&, const float*, float*,
                                              float*, bool, hipStream_t, const hipEvent_t*);
template hipError_t launch_bin_scatter<double>(const double*, const double*,
                                               const double*, const double*, int,
                                               const Grid&, BinArgs, const SpectralArgs&,
                                               const double*, double*, double*, bool,
                                               hipStream_t, const hipEvent_t*);
template hipError_t bin_occupancy<float>(int, int, int&, int&);
template hipError_t bin_occupancy<double>(int, int, int&, int&);
template hipError_t launch_fixed_density<float>(const float*, const float*, const float*,
                                                const float*, int, const Grid&, double,
                                                void*, float*, hipStream_t);
template hipError_t launch_fixed_density<double>(const double*, const double*,
                                                 const double*, const double*, int,
                                                 const Grid&, double, void*, double*,
                                                 hipStream_t);
template hipError_t launch_bin_gather<float>(const float*, const float*, const float*,
                                             const float*, int, const Grid&,
                                             const BinArgs&, const float*, const float*,
                                             float*, float*, hipStream_t, const hipEvent_t*);
template hipError_t launch_bin_gather<double>(const double*, const double*,
                                              const double*, const double*, int,
                                              const Grid&, const BinArgs&, const double*,
                                              const double*, double*, double*,
                                              hipStream_t, const hipEvent_t*);

}  // namespace dpep
