// Host stand-in for <hip/hip_runtime.h>, used ONLY by tests/emu: it lets the
// kernel headers of libdpep (csrc/dpep_*.h) compile as plain C++ so the test
// can run every kernel on the CPU -- one std::thread per GPU thread, a
// std::barrier per __syncthreads -- under AddressSanitizer with exact-size
// buffers.  It is a bounds and logic checker for the kernel source, not an
// execution path of the product.
#pragma once
#include <atomic>
#include <barrier>
#include <cmath>
#include <cstddef>
#include <cstdint>
#include <cstring>
#include <type_traits>
#include <algorithm>
#include <utility>

#define __global__
#define __device__
#define __host__
#define __forceinline__ inline
#define __launch_bounds__(...)
#define __shared__
#define __align__(n) __attribute__((aligned(n)))

struct dim3 {
    unsigned x = 1, y = 1, z = 1;
    dim3() = default;
    dim3(unsigned a, unsigned b = 1, unsigned c = 1) : x(a), y(b), z(c) {}
};
struct float2 { float x, y; };
struct double2 { double x, y; };
struct float4 { float x, y, z, w; };
struct uint2 { unsigned x, y; };
struct uint4 { unsigned x, y, z, w; };
inline float __uint_as_float(unsigned u) { float f; memcpy(&f, &u, 4); return f; }
inline unsigned __float_as_uint(float f) { unsigned u; memcpy(&u, &f, 4); return u; }
struct double4 { double x, y, z, w; };
using std::max;
using std::min;

extern thread_local dim3 threadIdx, blockIdx;
extern dim3 blockDim, gridDim;
extern std::barrier<>* emu_barrier;
inline void __syncthreads() { emu_barrier->arrive_and_wait(); }
inline void __threadfence() { std::atomic_thread_fence(std::memory_order_seq_cst); }
// __shfl_xor within groups of `width` lanes.  Every lane of a group calls it
// together (on the GPU the group runs in lockstep); here the lanes exchange
// values through one slot each, between two waits on the group's barrier.
extern std::barrier<>* emu_group_barrier(unsigned group, int width);
extern double emu_shfl_slot[1024];
template <typename V>
inline V __shfl_xor(V v, int mask, int width)
{
    const unsigned t = threadIdx.x, first = t - t % (unsigned)width;
    std::barrier<>& b = *emu_group_barrier(first / (unsigned)width, width);
    emu_shfl_slot[t] = (double)v;
    b.arrive_and_wait();
    const double r = emu_shfl_slot[first + ((t - first) ^ (unsigned)mask) % (unsigned)width];
    b.arrive_and_wait();
    return (V)r;
}
// __shfl_up: lane l gets lane l - delta's value (its own below delta)
template <typename V>
inline V __shfl_up(V v, unsigned delta, int width)
{
    const unsigned t = threadIdx.x, first = t - t % (unsigned)width;
    std::barrier<>& b = *emu_group_barrier(first / (unsigned)width, width);
    emu_shfl_slot[t] = (double)v;
    b.arrive_and_wait();
    const double r = t - first >= delta ? emu_shfl_slot[t - delta] : (double)v;
    b.arrive_and_wait();
    return (V)r;
}
// __hip_atomic_load is a clang builtin, available to host code as well
#ifndef __HIP_MEMORY_SCOPE_AGENT
#define __HIP_MEMORY_SCOPE_AGENT 3
#endif

using std::floor;
using std::isfinite;

inline unsigned long long __double2ull_rn(double x)
{
    return (unsigned long long)std::nearbyint(x);
}
#define __builtin_amdgcn_rcpf(x) (1.0f / (x))
// a wave vote decided per lane: the kernels only use it to choose between
// forms that give the same results
#define __any(p) (p)
inline unsigned __float2uint_rn(float x)
{
    return (unsigned)std::nearbyint(x);
}
inline unsigned long long __float2ull_rn(float x)
{
    return (unsigned long long)std::nearbyint(x);
}
inline unsigned __umul24(unsigned a, unsigned b)
{
    return (a & 0xFFFFFFu) * (b & 0xFFFFFFu);
}
template <class T>
inline T unsafeAtomicAdd(T* p, T v)
{
    std::atomic_ref<T> r(*p);
    return r.fetch_add(v);
}
inline unsigned long long atomicAdd(unsigned long long* p, unsigned long long v)
{
    return __atomic_fetch_add(p, v, __ATOMIC_RELAXED);
}
inline unsigned atomicExch(unsigned* p, unsigned v)
{
    std::atomic_ref<unsigned> r(*p);
    return r.exchange(v);
}
inline unsigned atomicAdd(unsigned* p, unsigned v)
{
    return __atomic_fetch_add(p, v, __ATOMIC_RELAXED);
}
inline unsigned atomicMax(unsigned* p, unsigned v)
{
    std::atomic_ref<unsigned> r(*p);
    unsigned o = r.load();
    while (o < v && !r.compare_exchange_weak(o, v)) {
    }
    return o;
}
inline unsigned atomicOr(unsigned* p, unsigned v)
{
    return std::atomic_ref<unsigned>(*p).fetch_or(v);
}
inline float atomicAdd(float* p, float v) { return unsafeAtomicAdd(p, v); }
inline double atomicAdd(double* p, double v) { return unsafeAtomicAdd(p, v); }

typedef int hipError_t;
constexpr hipError_t hipSuccess = 0;
constexpr hipError_t hipErrorInvalidValue = 1;
typedef void* hipStream_t;
typedef void* hipEvent_t;
