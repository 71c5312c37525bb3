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
                              BinArgs b, const T* d0n, T* dens, hipStream_t s,
                              hipEvent_t* ev)
{
    b.G1 = (int)g1_of(nc);
    const size_t tile = (size_t)b.R * g.N * sizeof(unsigned long long) + 16;
    const size_t count_lds = (size_t)(b.S + kBinThreads + 1) * sizeof(unsigned);
    const size_t hist = (size_t)b.S * sizeof(unsigned);
    hipError_t e;
    k_bin_count<T><<<b.G1, kBinThreads, count_lds, s>>>(px, py, sx, sy, nc, g, b);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[0], s))) return e;
    if (ev && (e = hipEventRecord(ev[1], s))) return e;
    k_bin_fill<T><<<b.G1, kBinThreads, hist, s>>>(px, py, sx, sy, nc, g, b);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[2], s))) return e;
    k_strip_acc<T><<<b.Wmax, kAccThreads, tile, s>>>(g, b, d0n, dens);
    if ((e = hipGetLastError())) return e;
    if (ev && (e = hipEventRecord(ev[3], s))) return e;
    return hipSuccess;
}

template <typename T>
hipError_t launch_bin_gather(const T* px, const T* py, const T* sx,
                             const T* sy, int nc, const Grid& g,
                             const BinArgs& b, const T* fx, const T* fy,
                             T* gx, T* gy, hipStream_t s)
{
    if (nc <= 0) return hipSuccess;
    const size_t lds = (size_t)gather_rows<T>(b.R, g.N) * g.N * 2 * sizeof(T);
    k_gather_bin<T><<<b.Wmax, kAccThreads, lds, s>>>(g, b, fx, fy);
    hipError_t e = hipGetLastError();
    if (e) return e;
    k_gather_out<T><<<g1_of(nc), kBinThreads, 0, s>>>(px, py, sx, sy, nc, g, b, fx, fy, gx,
                                                      gy);
    return hipGetLastError();
}

template <typename T>
static hipError_t prepare_bin_type()
{
    hipError_t e = hipFuncSetAttribute((const void*)k_strip_acc<T>,
                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                       (int)kAccLds);
    if (e) return e;
    return hipFuncSetAttribute((const void*)k_gather_bin<T>,
                               hipFuncAttributeMaxDynamicSharedMemorySize,
                               (int)kTileBytes);
}

hipError_t bin_prepare()
{
    hipError_t e = prepare_bin_type<float>();
    if (e) return e;
    return prepare_bin_type<double>();
}

template hipError_t launch_bin_scatter<float>(const float*, const float*, const float*,
                                              const float*, int, const Grid&, BinArgs,
                                              const float*, float*, hipStream_t, hipEvent_t*);
template hipError_t launch_bin_scatter<double>(const double*, const double*,
                                               const double*, const double*, int,
                                               const Grid&, BinArgs, const double*,
                                               double*, hipStream_t, hipEvent_t*);
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
