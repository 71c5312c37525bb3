// dpep_scatter.hip -- host launchers of the scatter, init and gather
// kernels (kernels in dpep_scatter.h).
#include "dpep_scatter.h"

namespace dpep {

template <typename T>
hipError_t launch_fill_init(const T* d0n, T* density, uint64_t* acc,
                            size_t mn, hipStream_t s)
{
    const size_t blocks = (mn + 255) / 256;
    const unsigned grid = (unsigned)(blocks < 8192 ? blocks : 8192);
    k_init<T><<<dim3(grid), dim3(256), 0, s>>>(d0n, density, acc, mn);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_scatter(const T* px, const T* py, const T* sx, const T* sy,
                          int nc, const Grid& g, T* density, uint64_t* acc,
                          hipStream_t s)
{
    if (nc <= 0) return hipSuccess;
    const dim3 grid((nc + 255) / 256), block(256);
    if (acc)
        k_scatter<T, true><<<grid, block, 0, s>>>(px, py, sx, sy, nc, g, density, acc);
    else
        k_scatter<T, false><<<grid, block, 0, s>>>(px, py, sx, sy, nc, g, density, acc);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_gather(const T* px, const T* py, const T* sx, const T* sy,
                         int nc, const Grid& g, const T* fx, const T* fy,
                         T* gx, T* gy, hipStream_t s)
{
    if (nc <= 0) return hipSuccess;
    const dim3 grid((nc + 255) / 256), block(256);
    k_gather<T><<<grid, block, 0, s>>>(px, py, sx, sy, nc, g, fx, fy, gx, gy);
    return hipGetLastError();
}

template hipError_t launch_fill_init<float>(const float*, float*, uint64_t*,
                                            size_t, hipStream_t);
template hipError_t launch_fill_init<double>(const double*, double*,
                                             uint64_t*, size_t, hipStream_t);
template hipError_t launch_scatter<float>(const float*, const float*,
                                          const float*, const float*, int,
                                          const Grid&, float*, uint64_t*,
                                          hipStream_t);
template hipError_t launch_scatter<double>(const double*, const double*,
                                           const double*, const double*, int,
                                           const Grid&, double*, uint64_t*,
                                           hipStream_t);
template hipError_t launch_gather<float>(const float*, const float*,
                                         const float*, const float*, int,
                                         const Grid&, const float*,
                                         const float*, float*, float*,
                                         hipStream_t);
template hipError_t launch_gather<double>(const double*, const double*,
                                          const double*, const double*, int,
                                          const Grid&, const double*,
                                          const double*, double*, double*,
                                          hipStream_t);

}  // namespace dpep
