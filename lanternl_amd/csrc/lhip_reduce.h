// lhip_reduce.h -- wave64 and workgroup reductions (device helpers).
#pragma once

#include <hip/hip_runtime.h>

namespace lhip {

__device__ __forceinline__ float wave_sum(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

__device__ __forceinline__ double wave_sum(double v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

// fmaxf ignores a NaN operand, like the Lua `if v > mx` scan.
__device__ __forceinline__ float wave_max(float v)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
    return v;
}

// Workgroup reductions for NW waves; `red` is LDS scratch of >= NW floats.
// Every thread of the block must call them (they contain barriers).
template <int NW>
__device__ __forceinline__ float block_sum(float v, float* red)
{
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < NW; ++i) s += red[i];
    return s;
}

template <int NW>
__device__ __forceinline__ float block_max(float v, float* red)
{
    v = wave_max(v);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NW; ++i) s = fmaxf(s, red[i]);
    return s;
}

// Row argmax under a strict '>' scan: (bv, bi) is a lane's best value and
// its index (bi < 0: nothing seen, i.e. only -inf/NaN).  A candidate wins on a
// larger value, or on an equal value at a lower index, so the result is the
// first index of the maximum whatever the lane split.
__device__ __forceinline__ void argmax_merge(float& bv, int& bi, float ov, int oi)
{
    if (oi >= 0 && (bi < 0 || ov > bv || (ov == bv && oi < bi))) { bv = ov; bi = oi; }
}

__device__ __forceinline__ void wave_argmax(float& bv, int& bi)
{
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        argmax_merge(bv, bi, ov, oi);
    }
}

// Workgroup argmax for NW waves; redv/redi are LDS scratch of >= NW entries.
// Returns the winning index (-1 if none) in every thread.
template <int NW>
__device__ __forceinline__ int block_argmax(float bv, int bi, float* redv, int* redi)
{
    wave_argmax(bv, bi);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) { redv[w] = bv; redi[w] = bi; }
    __syncthreads();
    float v = redv[0];
    int i = redi[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) argmax_merge(v, i, redv[k], redi[k]);
    return i;
}

}  // namespace lhip
