// dpep_spectral.hip -- host launchers of the spectral passes (kernels in
// dpep_spectral.h).
#include "dpep_spectral.h"

namespace dpep {

int spectral_fpw(int L, int dtype)
{
    return dtype == 0 ? fpw<float>(L) : fpw<double>(L);
}

// ---------------------------------------------------------------------------
// Host dispatch over the supported lengths.
// ---------------------------------------------------------------------------
template <typename T, int L>
constexpr size_t lds_bytes()
{
    return (size_t)fpw<T>(L) * lds_len(L) * sizeof(vec2_t<T>);
}

template <typename T, typename Fn>
static hipError_t dispatch_len(int L, Fn&& fn)
{
    switch (L) {
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
__global__ __launch_bounds__(256) void k_tables(int L, T* __restrict__ tw,
                                                T* __restrict__ post)
{
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    double s, c;
    if (i < L) {
        sincospi(2.0 * (double)i / (double)L, &s, &c);
        tw[2 * i] = (T)c;
        tw[2 * i + 1] = (T)-s;
    }
    if (i <= L / 2) {
        sincospi((double)i / (2.0 * (double)L), &s, &c);
        post[2 * i] = (T)c;
        post[2 * i + 1] = (T)-s;
    }
}

template <typename T>
hipError_t launch_tables(int L, T* tw, T* post, hipStream_t s)
{
    if (L < 1 || !tw || !post) return hipErrorInvalidValue;
    k_tables<T><<<(unsigned)((L + 255) / 256), 256, 0, s>>>(L, tw, post);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_col_pass(const SpectralArgs& a, const T* Tt, T* Ux, T* Uy,
                           hipStream_t s, const hipEvent_t* ev)
{
    return dispatch_len<T>(a.M, [&](auto lc) -> hipError_t {
        constexpr int L = decltype(lc)::value;
        constexpr int F = fpw<T>(L);
        const dim3 grid(a.N / (2 * F)), block(col_threads<T>(L));
        if (square_form<T, L>(a))
            DPEP_LAUNCH(ev, (k_col_pass<T, L, F, true>), grid, block,
                        (lds_bytes<T, L>()), s, a, Tt, Ux, Uy);
        else
            DPEP_LAUNCH(ev, (k_col_pass<T, L, F, false>), grid, block, (lds_bytes<T, L>()), s,
                        a, Tt, Ux, Uy);
        return hipGetLastError();
    });
}

template <typename T>
hipError_t launch_row_inv(const SpectralArgs& a, const T* Ux, const T* Uy,
                          T* fx, T* fy, T* phi, hipStream_t s, const hipEvent_t* ev)
{
    return dispatch_len<T>(a.N, [&](auto lc) -> hipError_t {
        constexpr int L = decltype(lc)::value;
        constexpr int F = fpw<T>(L);
        const int groups = a.M / (2 * F);
        const dim3 grid(groups * (a.potential ? 3 : 2)), block(row_threads<T>(L));
        if (square_form<T, L>(a))
            DPEP_LAUNCH(ev, (k_row_inv<T, L, F, true>), grid, block,
                        (lds_bytes<T, L>()), s, a, Ux, Uy, fx, fy, phi);
        else
            DPEP_LAUNCH(ev, (k_row_inv<T, L, F, false>), grid, block, (lds_bytes<T, L>()), s, a,
                        Ux, Uy, fx, fy, phi);
        return hipGetLastError();
    });
}

template <typename T, int L>
static hipError_t prepare_len()
{
    constexpr int F = fpw<T>(L);
    const int bytes = (int)lds_bytes<T, L>();
    hipError_t e;
    constexpr bool kSq = L >= kSquareMin;
    if ((e = hipFuncSetAttribute((const void*)k_col_pass<T, L, F, false>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes)) ||
        (e = hipFuncSetAttribute((const void*)k_row_inv<T, L, F, false>,
                                 hipFuncAttributeMaxDynamicSharedMemorySize, bytes)))
        return e;
    if constexpr (kSq) {
        if ((e = hipFuncSetAttribute((const void*)k_col_pass<T, L, F, true>,
                                     hipFuncAttributeMaxDynamicSharedMemorySize, bytes)))
            return e;
        return hipFuncSetAttribute((const void*)k_row_inv<T, L, F, true>,
                                   hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
    }
    return hipSuccess;
}

template <typename T>
static hipError_t prepare_type()
{
    hipError_t e;
    if ((e = prepare_len<T, 8>())) return e;
    if ((e = prepare_len<T, 16>())) return e;
    if ((e = prepare_len<T, 32>())) return e;
    if ((e = prepare_len<T, 64>())) return e;
    if ((e = prepare_len<T, 128>())) return e;
    if ((e = prepare_len<T, 256>())) return e;
    if ((e = prepare_len<T, 512>())) return e;
    if ((e = prepare_len<T, 1024>())) return e;
    if ((e = prepare_len<T, 2048>())) return e;
    if ((e = prepare_len<T, 4096>())) return e;
    if constexpr (sizeof(T) == 4)
        if ((e = prepare_len<T, 8192>())) return e;
    return hipSuccess;
}

hipError_t spectral_prepare()
{
    hipError_t e = prepare_type<float>();
    if (e) return e;
    return prepare_type<double>();
}

template hipError_t launch_tables<float>(int, float*, float*, hipStream_t);
template hipError_t launch_tables<double>(int, double*, double*, hipStream_t);
template hipError_t launch_col_pass<float>(const SpectralArgs&, const float*,
                                           float*, float*, hipStream_t, const hipEvent_t*);
template hipError_t launch_col_pass<double>(const SpectralArgs&, const double*,
                                            double*, double*, hipStream_t, const hipEvent_t*);
template hipError_t launch_row_inv<float>(const SpectralArgs&, const float*,
                                          const float*, float*, float*, float*,
                                          hipStream_t, const hipEvent_t*);
template hipError_t launch_row_inv<double>(const SpectralArgs&, const double*,
                                           const double*, double*, double*,
                                           double*, hipStream_t, const hipEvent_t*);

}  // namespace dpep
