/*
 * dpep.h -- C ABI of libdpep.so, the MI355X (gfx950) electric-potential step
 * of DREAMPlace: cell-to-bin density scatter, DCT-based Poisson solve, field
 * maps and the per-cell field gather.
 *
 * The ABI replaces the device side of the reference's shared-memory server
 * (host/density_scatter_ttnn_server_host.cpp) with plain functions over plain
 * pointers.  Its callers here are the ctypes binding of the Python client
 * (dreamplacett-framework_amd/dpep/_lib.py) and the shm server loop
 * (dreamplacett-framework_amd/csrc/dpep_server.cpp).
 *
 * Conventions
 *   - Maps are x-major: map[bx * N + by], M = num_bins_x rows of N = num_bins_y
 *     (the reference's density layout, kernels/v11_accum_dm.cpp:386-398).
 *   - px, py are lower-left corners; sx, sy are the cells' original sizes
 *     (integration/scatter_ttnn_client.py:628-649).  The library applies
 *     DREAMPlace's small-cell stretch itself (sqrt2 * bin, ratio = area /
 *     stretched area) unless DPEP_FLAG_NO_STRETCH is set.
 *   - Cells with a non-finite coordinate or a non-positive size contribute
 *     nothing and receive zero force (the reference's zero padding,
 *     docs/DREAMPLACE_TT_INTEGRATION.md:233-241).
 *   - Element type of every array is the context's dtype: float for
 *     DPEP_DTYPE_F32, double for DPEP_DTYPE_F64.
 *   - Every function returns DPEP_OK or an error code; dpep_last_error()
 *     gives the text of the calling thread's last error.
 *   - A context is not thread-safe: one in-flight step per context.
 */
#ifndef DPEP_H
#define DPEP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define DPEP_ABI_VERSION 6

/* status codes */
#define DPEP_OK 0
#define DPEP_ERR_ARG 1          /* invalid argument (bad size, NULL, ...)   */
#define DPEP_ERR_HIP 2          /* HIP runtime failure                      */
#define DPEP_ERR_STATE 3        /* call out of order (e.g. no cells yet)    */
#define DPEP_ERR_NOMEM 4        /* device or host allocation failed         */
#define DPEP_ERR_UNSUPPORTED 5  /* grid shape outside the supported set     */

/* element types */
#define DPEP_DTYPE_F32 0
#define DPEP_DTYPE_F64 1

/* flags for dpep_create */
#define DPEP_FLAG_DETERMINISTIC 0x1u /* accepted for compatibility: every
                                        mode accumulates the density in
                                        uint64 fixed point and is bitwise
                                        reproducible run to run           */
#define DPEP_FLAG_NO_POTENTIAL 0x2u  /* skip the potential map             */
#define DPEP_FLAG_NO_STRETCH 0x4u    /* no sqrt2*bin stretch, ratio = 1
                                        (the TT path's semantics,
                                        scatter_ttnn_client.py:628-649)    */
#define DPEP_FLAG_NO_GATHER 0x8u     /* skip the per-cell force gather     */
#define DPEP_FLAG_STEP_TIMINGS 0x10u /* record a HIP event at the start and
                                        end of every step, for the compute
                                        slot of dpep_get_timings (each event
                                        costs a few microseconds of GPU time
                                        per step; without the flag the slot
                                        reads 0 unless profiling is on)    */
#define DPEP_FLAG_SCATTER_DENSITY 0x20u /* also keep the scattered cells'
                                        density without the initial density
                                        (one more M*N map written per step),
                                        for dpep_get_scatter_density       */
#define DPEP_FLAG_TWO_PASS 0x40u     /* count the cells per strip before
                                        sorting them on every step.  By
                                        default a step after the first sorts
                                        in one pass into room the previous
                                        step sized from its own counts (plus
                                        an eighth); cells beyond that room
                                        still land correctly, through device
                                        atomics, but a context stepped with
                                        unrelated placements is faster with
                                        this flag.  Results are bitwise the
                                        same either way.                   */

/* timing slots, the reference's 9-float shm header order
 * (integration/scatter_ttnn_client.py:151-163): h2d, scatter, gather,
 * d2h_den, upload, compute, download, fw, total.  Here: scatter = density
 * scatter kernels, gather = per-cell force gather, compute = spectral solve
 * kernels, h2d = cell upload, d2h_den = density download, download = field /
 * potential / force download, upload = initial-density upload (0 per step),
 * fw = 0 (filled by the shm server), total = sum.  Milliseconds, measured
 * with HIP events on the context's stream.                                 */
#define DPEP_NUM_TIMINGS 9

typedef struct dpep_ctx dpep_ctx;

/* Library version and the gfx target it was built for. */
int dpep_abi_version(void);
const char* dpep_build_info(void);

/* Text of the calling thread's last error ("" if none). */
const char* dpep_last_error(void);

/* Creates a context on the current HIP device: allocates every device buffer
 * for nc_max cells and an M x N grid (no allocation happens per step),
 * builds the twiddle tables and the stream.  M and N must be powers of two in
 * [8, 8192].  Replaces the reference server's start-up: argument parsing
 * (host/density_scatter_ttnn_server_host.cpp:324-339), device buffer set-up
 * (:404-483) and TTNNDCTSolver::init (:236-269). */
int dpep_create(int num_bins_x, int num_bins_y, int nc_max, double xl,
                double yl, double xh, double yh, int dtype, unsigned flags,
                dpep_ctx** out);

/* Releases the context and its device memory. */
int dpep_destroy(dpep_ctx* ctx);

/* Uploads initial_density_map / bin_area (M*N elements, host memory), the
 * fixed-cell density folded into every step's density.  Replaces shm slot 3
 * (integration/scatter_ttnn_client.py:786-795) and the server's host fold
 * (host/density_scatter_ttnn_server_host.cpp:1770-1777).  Until called the
 * initial density is zero. */
int dpep_set_initial_density(dpep_ctx* ctx, const void* d0n);

/* Computes the initial density from n fixed cells (host memory: lower-left
 * corners and sizes, no stretch): D0n = target_density * sum of exact
 * cell/bin overlaps / bin_area, replacing any previous initial density.
 * This is the initial_density_map / bin_area that the reference's client
 * receives from DREAMPlace and uploads once
 * (integration/scatter_ttnn_client.py:786-795), computed on the GPU.
 * A set-up call: it allocates a temporary device copy of the cells. */
int dpep_set_fixed_cells(dpep_ctx* ctx, const void* px, const void* py,
                         const void* sx, const void* sy, int n,
                         double target_density);

/* Uploads nc <= nc_max cells (host memory) into the context's device
 * buffers.  Replaces the server's H2D (:1335-1349).  sx and sy both NULL
 * (new in ABI 5): only the positions are uploaded and the cells keep the
 * sizes resident from the last call that passed them, which must have
 * covered at least nc cells (DPEP_ERR_STATE otherwise).  DREAMPlace's cell
 * sizes do not change between iterations, so a caller that knows this
 * halves the per-step upload. */
int dpep_set_cells(dpep_ctx* ctx, const void* px, const void* py,
                   const void* sx, const void* sy, int nc);

/* Runs one step on the resident cells into the context's device outputs,
 * asynchronously on the context's stream.  Replaces the scatter, accumulate,
 * fold and TTNN solve of the server loop (:1629-1781). */
int dpep_compute(dpep_ctx* ctx);

/* Waits for the context's stream. */
int dpep_sync(dpep_ctx* ctx);

/* Copies the last step's outputs to host memory (waits first).  Any pointer
 * may be NULL.  density, potential, field_x, field_y: M*N; grad_x, grad_y:
 * nc of the last computed step (the per-cell gather ratio * sum
 * tx*ty*field, sign left to the caller).  Fails with DPEP_ERR_STATE when a
 * requested output is stale: cells were uploaded after the last step, or the
 * last step was a dpep_step_device that wrote that output to a caller-owned
 * buffer.  Host memory from dpep_host_alloc copies at the full link rate.
 * Replaces the server's D2H and field write (:1678, :1785-1789). */
int dpep_get_outputs(dpep_ctx* ctx, void* density, void* potential,
                     void* field_x, void* field_y, void* grad_x,
                     void* grad_y);

/* The last step's scattered-cell density alone, M*N elements, without the
 * initial density: the reference server's density read-back
 * (host/density_scatter_ttnn_server_host.cpp:1676-1678), which it dumps to
 * EXPORT_DENSITY_PATH (:1686-1695) and, with CPU_DCT=1, writes to the
 * field_x slot unfolded (:1759, :1786-1788).  Needs a context created with
 * DPEP_FLAG_SCATTER_DENSITY.  Waits for the step. */
int dpep_get_scatter_density(dpep_ctx* ctx, void* out);

/* Page-locked host memory (hipHostMalloc): transfers from and to it run at
 * the link rate, where pageable memory is staged by the runtime.  The
 * reference's server copies through pageable std::vectors
 * (:1335-1349, :1676-1678); the shm server of this library stages through
 * these buffers instead.  Free with dpep_host_free. */
int dpep_host_alloc(size_t bytes, void** out);
int dpep_host_free(void* p);

/* set_cells + compute + get_outputs: one whole step on host buffers, the
 * server loop body (:1326-1815).  sx and sy both NULL keep the resident
 * sizes, as in dpep_set_cells. */
int dpep_step(dpep_ctx* ctx, const void* px, const void* py, const void* sx,
              const void* sy, int nc, void* field_x, void* field_y,
              void* density, void* potential, void* grad_x, void* grad_y);

/* One step on caller-owned device memory, asynchronous on `stream`
 * (a hipStream_t; NULL = the context's stream).  Inputs px..sy hold nc
 * cells.  Outputs may be NULL, in which case they land in the context's own
 * buffers.  No counterpart in the reference (its positions always crossed
 * PCIe); it is the zero-copy entry point for callers already on the GPU. */
int dpep_step_device(dpep_ctx* ctx, const void* d_px, const void* d_py,
                     const void* d_sx, const void* d_sy, int nc,
                     void* d_field_x, void* d_field_y, void* d_density,
                     void* d_potential, void* d_grad_x, void* d_grad_y,
                     void* stream);

/* dpep_step_device without a context, allocating nothing: no counterpart in
 * the reference.  It is for callers that cannot allocate device memory --
 * code under HIP graph capture, fixed serving loops.  Arguments as
 * dpep_create (grid, die, dtype, flags among DETERMINISTIC, NO_POTENTIAL,
 * NO_STRETCH, NO_GATHER; nc_max sizes the fixed-point scale exactly as
 * there) plus the initial density (device, M*N; NULL = zero) and the
 * dpep_step_device arguments; every output the step computes must be given
 * (no context buffers to fall back on).  All scratch comes from one 64 MiB
 * device array per GPU, held until the process ends (e.g. 1024 x 1024 bins
 * with 2^19 float32 cells fit); a larger problem fails with DPEP_ERR_ARG
 * and the size it needs.  Calls that overlap on one GPU share that array and
 * race: serialise them.  Asynchronous on `stream` (NULL = the null stream);
 * launches only kernels (no memset, no allocation, no host wait). */
int dpep_step_device_noalloc(int num_bins_x, int num_bins_y, double xl, double yl,
                             double xh, double yh, int dtype, unsigned flags,
                             int nc_max, const void* d_initial_density,
                             const void* d_px, const void* d_py, const void* d_sx,
                             const void* d_sy, int nc, void* d_field_x,
                             void* d_field_y, void* d_density, void* d_potential,
                             void* d_grad_x, void* d_grad_y, void* stream);

/* Per-stage milliseconds of the last step (DPEP_NUM_TIMINGS floats), the
 * values the reference server wrote into the shm header (:1798-1808). */
int dpep_get_timings(dpep_ctx* ctx, float* out);

/* Per-kernel average durations in microseconds over the steps recorded
 * since profiling was enabled (at most `slots` of them), measured with HIP
 * events around each launch on the stream the kernels run on:
 * [0] strip count (with the strip table; a step that sorts in one pass
 * launches none and adds 0), [1] strip fill, [2] strip
 * accumulate with the row DCT (and the reduction of split strips),
 * [3] column DCT + inverse, [4] row inverse, [5] gather of the partial
 * forces per strip record, [6] forces in cell order, [7] whole step.
 * n = floats in out.  (ABI version 1 had one gather slot at [5] and the
 * step at [6].) */
int dpep_get_kernel_times(dpep_ctx* ctx, float* out, int n);

/* How the last step binned its cells (waits for it): n long longs of
 * [0] 1 if it sorted in one pass on the plan the step before it made from
 *     its counts, 0 if it counted first;
 * [1] strip records of the step (a cell that is not taller than a strip
 *     makes one record per strip it touches: one or two);
 * [2] of them, records that found no room in their region and went to the
 *     overflow pool (their density through device atomics; always 0 on a
 *     counted step);
 * [3] [4] work items of the strip accumulation and of the per-strip gather;
 * [5] [6] records per work item of each (a strip above that is split);
 * [7] the most overflow runs one strip received (one per block of cells
 *     that overflowed there).
 * No counterpart in the reference (its routing dropped records past a page's
 * capacity, kernels/v11_scatter_dm.cpp:235-246, and counted nothing); it
 * shows what the one-pass binning costs when cells move between steps. */
#define DPEP_NUM_BIN_STATS 8
int dpep_get_binning_stats(dpep_ctx* ctx, long long* out, int n);

/* slots > 0 enables per-kernel event timing for a ring of `slots` steps
 * (each kernel of a profiled step is launched with a start/end event pair
 * stamped by its own dispatch); 0 disables (the default). */
int dpep_set_profiling(dpep_ctx* ctx, int slots);

#ifdef __cplusplus
}
#endif

#endif /* DPEP_H */
