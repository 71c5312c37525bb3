// dpep_internal.h -- host-side context and the kernel launchers shared by the
// translation units of libdpep.so.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dpep_device.h"

namespace dpep {

// Rows per workgroup of the spectral passes are 2*F where F is the number of
// complex FFTs a workgroup holds in LDS.  The intermediate matrices are
// stored in tiles of (2*F_N) x (2*F_M) elements so that every pass moves
// whole tiles (>= 128 contiguous bytes) through HBM.
int spectral_fpw(int L, int dtype);

struct Tiles {
    int TX;   // tile extent along x  (= 2 * F of the length-N passes)
    int TV;   // tile extent along v  (= 2 * F of the length-M pass)
};

struct SpectralArgs {
    int M, N;
    Tiles tiles;
    double wu_step;     // 2 pi / M
    double wv_step;     // 2 pi / N * bsx / bsy
    int potential;      // compute the potential map
    double fix_inv;     // 1 / Grid::fix_scale (deterministic mode)
    const void* twM;    // exp(-2 pi i m / M), m < M
    const void* postM;  // exp(-i pi k / 2M), k <= M/2
    const void* twN;
    const void* postN;
};

// Launchers (return hipError_t of the launch).  T = float or double.
template <typename T>
hipError_t launch_fill_init(const T* d0n, T* density, uint64_t* acc,
                            size_t mn, hipStream_t s);
template <typename T>
hipError_t launch_scatter(const T* px, const T* py, const T* sx, const T* sy,
                          int nc, const Grid& g, T* density, uint64_t* acc,
                          hipStream_t s);
template <typename T>
hipError_t launch_row_dct(const SpectralArgs& a, const T* density_in,
                          const uint64_t* acc, const T* d0n, T* density_out,
                          T* Tt, hipStream_t s);
template <typename T>
hipError_t launch_col_pass(const SpectralArgs& a, T* Tt, T* Ux, T* Uy,
                           hipStream_t s);
template <typename T>
hipError_t launch_row_inv(const SpectralArgs& a, const T* Ux, const T* Uy,
                          const T* Up, T* fx, T* fy, T* phi, hipStream_t s);
template <typename T>
hipError_t launch_gather(const T* px, const T* py, const T* sx, const T* sy,
                         int nc, const Grid& g, const T* fx, const T* fy,
                         T* gx, T* gy, hipStream_t s);

// Sets the dynamic-LDS limits of every spectral kernel instance (once).
hipError_t spectral_prepare();

}  // namespace dpep
