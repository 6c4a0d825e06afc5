// Global accumulators of the decode step: fp64 (or fp32) sums built with
// relaxed agent-scope atomics by many workgroups, read and cleared in one
// atomic exchange, and cleared in shares by the workgroups of a later
// launch.
#pragma once

#include <hip/hip_runtime.h>

namespace iam {

__device__ __forceinline__ void acc_add(double* p, double v) { unsafeAtomicAdd(p, v); }
__device__ __forceinline__ void acc_add(float* p, float v) { unsafeAtomicAdd(p, v); }

// the value, leaving zero behind
__device__ __forceinline__ double acc_take(double* p)
{
    const unsigned long long b = __hip_atomic_exchange(reinterpret_cast<unsigned long long*>(p), 0ull,
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)b);
}
__device__ __forceinline__ float acc_take(float* p)
{
    const unsigned int b = __hip_atomic_exchange(reinterpret_cast<unsigned int*>(p), 0u, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    return __uint_as_float(b);
}

// the value, read at the point of coherence of the atomics
__device__ __forceinline__ double acc_peek(double* p)
{
    const unsigned long long b = __hip_atomic_load(reinterpret_cast<unsigned long long*>(p), __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT);
    return __longlong_as_double((long long)b);
}
__device__ __forceinline__ float acc_peek(float* p)
{
    return __uint_as_float(__hip_atomic_load(reinterpret_cast<unsigned int*>(p), __ATOMIC_RELAXED,
                                             __HIP_MEMORY_SCOPE_AGENT));
}

// zero n accumulator words, shared out over every workgroup of the grid (x
// and y): each one must call it, including those with no other work
template <typename Acc>
__device__ __forceinline__ void zero_share(void* p, int n, int nt)
{
    if (!p || n <= 0) return;
    const int nb = gridDim.x * gridDim.y;
    const int b = blockIdx.y * gridDim.x + blockIdx.x;
    const int per = (n + nb - 1) / nb;
    const int e = min(n, (b + 1) * per);
    Acc* q = reinterpret_cast<Acc*>(p);
    for (int i = b * per + (int)threadIdx.x; i < e; i += nt) q[i] = (Acc)0;
}

}  // namespace iam
