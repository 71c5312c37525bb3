// dpep_bin.hip -- host launchers of the strip-binned scatter and gather
// (kernels in dpep_bin.h).
#include "dpep_bin.h"

namespace dpep {

static unsigned g1_of(int nc)
{
    const int g = (nc + kCellsPerGroup - 1) / kCellsPerGroup;
    return (unsigned)(g > 0 ? g : 1);
}

template <typename T>
hipError_t launch_bin_scatter(const T* px, const T* py, const T* sx,
                              const T* sy, int nc, const Grid& g,
                              BinArgs b, const T* d0n, T* dens,
                              uint64_t* acc, T* gx, T* gy, hipStream_t s,
                              hipEvent_t* ev)
{
    const bool fixed = acc != nullptr;
    b.G1 = (int)g1_of(nc);
    const size_t acc_bytes = fixed ? 8 : sizeof(T);
    const size_t tile = (size_t)b.R * g.N * acc_bytes;
    const size_t hist = (size_t)b.S * sizeof(unsigned);
    hipError_t e;
    k_bin_count<T><<<b.G1, kBinThreads, hist, s>>>(px, py, sx, sy, nc, g, b);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[0], s))) return e;
    k_bin_scan<<<1, kScanThreads, (size_t)(b.S + 2048) * sizeof(unsigned), s>>>(b);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[1], s))) return e;
    if (fixed)
        k_bin_fill<T, true><<<b.G1, kBinThreads, hist, s>>>(px, py, sx, sy, nc, g, b, gx, gy);
    else
        k_bin_fill<T, false><<<b.G1, kBinThreads, hist, s>>>(px, py, sx, sy, nc, g, b, gx, gy);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[2], s))) return e;
    if (fixed)
        k_strip_acc<T, true><<<b.Wmax, kAccThreads, tile, s>>>(g, b, d0n, dens, acc);
    else
        k_strip_acc<T, false><<<b.Wmax, kAccThreads, tile, s>>>(g, b, d0n, dens, acc);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[3], s))) return e;
    if (fixed)
        k_strip_red<T, true><<<b.S, kAccThreads, 0, s>>>(g, b, d0n, dens, acc);
    else
        k_strip_red<T, false><<<b.S, kAccThreads, 0, s>>>(g, b, d0n, dens, acc);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_bin_gather(const T* px, const T* py, const T* sx,
                             const T* sy, int nc, const Grid& g,
                             const BinArgs& b, const T* fx, const T* fy,
                             T* gx, T* gy, hipStream_t s)
{
    if (nc <= 0) return hipSuccess;
    long long blocks = ((long long)nc * 5 / 4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    k_gather_bin<T><<<(unsigned)blocks, 256, 0, s>>>(px, py, sx, sy, g, b, fx, fy, gx, gy);
    return hipGetLastError();
}

template <typename T>
static hipError_t prepare_bin_type()
{
    hipError_t e;
    if ((e = hipFuncSetAttribute((const void*)k_strip_acc<T, false>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, 65536)))
        return e;
    return hipFuncSetAttribute((const void*)k_strip_acc<T, true>,
                               hipFuncAttributeMaxDynamicSharedMemorySize, 65536);
}

hipError_t bin_prepare()
{
    hipError_t e = prepare_bin_type<float>();
    if (e) return e;
    return prepare_bin_type<double>();
}

template hipError_t launch_bin_scatter<float>(const float*, const float*, const float*,
                                              const float*, int, const Grid&, BinArgs,
                                              const float*, float*, uint64_t*, float*,
                                              float*, hipStream_t, hipEvent_t*);
template hipError_t launch_bin_scatter<double>(const double*, const double*,
                                               const double*, const double*, int,
                                               const Grid&, BinArgs, const double*,
                                               double*, uint64_t*, double*, double*,
                                               hipStream_t, hipEvent_t*);
template hipError_t launch_bin_gather<float>(const float*, const float*, const float*,
                                             const float*, int, const Grid&,
                                             const BinArgs&, const float*, const float*,
                                             float*, float*, hipStream_t);
template hipError_t launch_bin_gather<double>(const double*, const double*,
                                              const double*, const double*, int,
                                              const Grid&, const BinArgs&, const double*,
                                              const double*, double*, double*,
                                              hipStream_t);

}  // namespace dpep
