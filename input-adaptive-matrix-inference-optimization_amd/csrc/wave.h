// Wave64 reductions and scans through DPP (gfx9 encodings): row_shr:n =
// 0x110 + n shifts within 16-lane rows, row_bcast15 / row_bcast31 = 0x142 /
// 0x143 carry lane 15 / 31 of a row group into the next rows (masked by
// row_mask).  Lanes with no source keep `old`.  The results are exact and
// the order of operations is fixed, so they are deterministic.
#pragma once

#include <hip/hip_runtime.h>

namespace iam {

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ int dpp_i(int old, int v)
{
    return __builtin_amdgcn_update_dpp(old, v, CTRL, ROW_MASK, 0xF, false);
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_f(float old, float v)
{
    return __int_as_float(dpp_i<CTRL, ROW_MASK>(__float_as_int(old), __float_as_int(v)));
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_d(double old, double v)
{
    const long long o = __double_as_longlong(old), x = __double_as_longlong(v);
    const int lo = dpp_i<CTRL, ROW_MASK>((int)o, (int)x);
    const int hi = dpp_i<CTRL, ROW_MASK>((int)(o >> 32), (int)(x >> 32));
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}


template <typename T>
__device__ __forceinline__ T lane63(T v);
template <>
__device__ __forceinline__ float lane63<float>(float v)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 63));
}
template <>
__device__ __forceinline__ double lane63<double>(double v)
{
    const long long x = __double_as_longlong(v);
    const int lo = __builtin_amdgcn_readlane((int)x, 63);
    const int hi = __builtin_amdgcn_readlane((int)(x >> 32), 63);
    return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

template <>
__device__ __forceinline__ uint32_t lane63<uint32_t>(uint32_t v)
{
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ uint32_t dpp_t(uint32_t old, uint32_t v)
{
    return (uint32_t)dpp_i<CTRL, ROW_MASK>((int)old, (int)v);
}
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp_t(float old, float v) { return dpp_f<CTRL, ROW_MASK>(old, v); }
template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ double dpp_t(double old, double v) { return dpp_d<CTRL, ROW_MASK>(old, v); }

// op over the 64 lanes (op(v, v) == v for lanes without a source), returned
// in every lane
template <typename T, typename Op>
__device__ __forceinline__ T wave_reduce(T v, Op op)
{
    v = op(v, dpp_t<0x111>(v, v));
    v = op(v, dpp_t<0x112>(v, v));
    v = op(v, dpp_t<0x114>(v, v));
    v = op(v, dpp_t<0x118>(v, v));
    v = op(v, dpp_t<0x142, 0xA>(v, v));
    v = op(v, dpp_t<0x143, 0xC>(v, v));
    return lane63(v);
}

__device__ __forceinline__ float wave_min(float v)
{
    return wave_reduce(v, [](float a, float b) { return fminf(a, b); });
}
__device__ __forceinline__ float wave_max(float v)
{
    return wave_reduce(v, [](float a, float b) { return fmaxf(a, b); });
}
template <typename T>
__device__ __forceinline__ T wave_max_t(T v)
{
    return wave_reduce(v, [](T a, T b) { return a > b ? a : b; });
}

// min / max of unsigned values over the 64 lanes, in every lane: lanes
// without a source see the identity, so each step is one min / max with a
// DPP operand
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v)
{
    v = min(v, dpp_t<0x111>(0xffffffffu, v));
    v = min(v, dpp_t<0x112>(0xffffffffu, v));
    v = min(v, dpp_t<0x114>(0xffffffffu, v));
    v = min(v, dpp_t<0x118>(0xffffffffu, v));
    v = min(v, dpp_t<0x142, 0xA>(0xffffffffu, v));
    v = min(v, dpp_t<0x143, 0xC>(0xffffffffu, v));
    return lane63(v);
}
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v)
{
    v = max(v, dpp_t<0x111>(0u, v));
    v = max(v, dpp_t<0x112>(0u, v));
    v = max(v, dpp_t<0x114>(0u, v));
    v = max(v, dpp_t<0x118>(0u, v));
    v = max(v, dpp_t<0x142, 0xA>(0u, v));
    v = max(v, dpp_t<0x143, 0xC>(0u, v));
    return lane63(v);
}

// sum over the 64 lanes: lanes without a source add zero
template <typename T>
__device__ __forceinline__ T wave_sum(T v)
{
    v += dpp_t<0x111>((T)0, v);
    v += dpp_t<0x112>((T)0, v);
    v += dpp_t<0x114>((T)0, v);
    v += dpp_t<0x118>((T)0, v);
    v += dpp_t<0x142, 0xA>((T)0, v);
    v += dpp_t<0x143, 0xC>((T)0, v);
    return lane63(v);
}

// inclusive prefix sum over the 64 lanes
__device__ __forceinline__ int wave_incl_sum(int v)
{
    v += dpp_i<0x111>(0, v);
    v += dpp_i<0x112>(0, v);
    v += dpp_i<0x114>(0, v);
    v += dpp_i<0x118>(0, v);
    v += dpp_i<0x142, 0xA>(0, v);
    v += dpp_i<0x143, 0xC>(0, v);
    return v;
}

}  // namespace iam
