// dpep_scatter.h -- kernels of the cell-to-bin density scatter and the per-cell field
// gather.
//
// Scatter: one thread per cell computes the stretched cell's bin span in
// float64 (reference maths: tools/v13_offset_ratio_stats.py:54-67 stretch,
// kernels/v4_compute.cpp:128-176 overlap, tools/cpu_vs_tt_density.py:45-76
// span loop) and adds ratio * tx * ty / bin_area into every covered bin:
// native float atomics into a map pre-loaded with the fixed-cell density, or
// (deterministic mode) unsigned 64-bit fixed-point atomics into a zeroed map
// that the first spectral pass converts and folds (scale 2^f, f chosen
// per context so the sum cannot overflow; see fix_exponent).
//
// Gather: one thread per cell sums ratio * tx * ty * field over the same span
// (the consumer of ctx.field_map_x/y, integration/scatter_ttnn_client.py:
// 831-855).
#pragma once

#include "dpep_internal.h"

namespace dpep {

template <typename T>
__global__ __launch_bounds__(256) void k_init(const T* __restrict__ d0n,
                                              T* __restrict__ density,
                                              uint64_t* __restrict__ acc,
                                              size_t mn)
{
    const size_t stride = (size_t)gridDim.x * blockDim.x;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < mn;
         i += stride) {
        if (acc) acc[i] = 0ull;
        else density[i] = d0n[i];
    }
}

template <typename T, bool FIXED>
__global__ __launch_bounds__(256) void k_scatter(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    T* __restrict__ density, uint64_t* __restrict__ acc)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nc) return;
    CellSpan c;
    if (!cell_span((double)px[i], (double)py[i], (double)sx[i], (double)sy[i],
                   g, c))
        return;
    const double s = c.ratio * g.inv_ba;
    for (int k = c.bxl; k <= c.bxh; ++k) {
        const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
        if (tx <= 0.0) continue;
        const double stx = s * tx;
        const size_t row = (size_t)k * g.N;
        for (int h = c.byl; h <= c.byh; ++h) {
            const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, h);
            if (ty <= 0.0) continue;
            const double v = stx * ty;
            if constexpr (FIXED) {
                atomicAdd((unsigned long long*)&acc[row + h],
                          (unsigned long long)__double2ull_rn(v * g.fix_scale));
            } else {
                unsafeAtomicAdd(&density[row + h], (T)v);
            }
        }
    }
}

template <typename T>
__global__ __launch_bounds__(256) void k_gather(
    const T* __restrict__ px, const T* __restrict__ py,
    const T* __restrict__ sx, const T* __restrict__ sy, int nc, Grid g,
    const T* __restrict__ fx, const T* __restrict__ fy, T* __restrict__ gx,
    T* __restrict__ gy)
{
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= nc) return;
    CellSpan c;
    double ax = 0.0, ay = 0.0;
    if (cell_span((double)px[i], (double)py[i], (double)sx[i], (double)sy[i],
                  g, c)) {
        for (int k = c.bxl; k <= c.bxh; ++k) {
            const double tx = overlap_1d(c.x, c.w, g.xl, g.bsx, k);
            if (tx <= 0.0) continue;
            const size_t row = (size_t)k * g.N;
            for (int h = c.byl; h <= c.byh; ++h) {
                const double ty = overlap_1d(c.y, c.h, g.yl, g.bsy, h);
                if (ty <= 0.0) continue;
                const double a = tx * ty;
                ax += a * (double)fx[row + h];
                ay += a * (double)fy[row + h];
            }
        }
        ax *= c.ratio;
        ay *= c.ratio;
    }
    gx[i] = (T)ax;
    gy[i] = (T)ay;
}

}  // namespace dpep
