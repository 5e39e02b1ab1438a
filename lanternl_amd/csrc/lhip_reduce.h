// lhip_reduce.h -- wave64 and workgroup reductions (device helpers).
#pragma once

#include <hip/hip_runtime.h>

namespace lhip {

// Cross-lane moves inside a 16-lane row use DPP (a VALU operand modifier, a
// few cycles) instead of __shfl_xor, which is an LDS permute with an LDS round
// trip per step.  The four row results of a wave are combined with
// v_readlane, which leaves the value wave-uniform.
//   0xB1  quad_perm [1,0,3,2]: lane i <- i^1
//   0x4E  quad_perm [2,3,0,1]: lane i <- i^2
//   0x141 row_half_mirror:     lane i <- 7-i within each 8 lanes
//   0x140 row_mirror:          lane i <- 15-i within each 16 lanes
// After the two quad steps every lane holds its quad's value; the half
// mirror pairs the two quads of each 8 lanes, the mirror the two halves of
// each 16, so four steps reduce a row and leave the result in all 16 lanes
// (each step combines a lane with its partner in both orders; + and max are
// commutative, so the 16 lanes agree bit for bit).
template <int CTRL>
__device__ __forceinline__ int dpp_i(int v)
{
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v)
{
    return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v)));
}

template <int CTRL>
__device__ __forceinline__ double dpp_d(double v)
{
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = dpp_i<CTRL>(static_cast<int>(b));
    const int hi = dpp_i<CTRL>(static_cast<int>(b >> 32));
    return __builtin_bit_cast(double, (static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

__device__ __forceinline__ float lane_f(float v, int l)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), l));
}

__device__ __forceinline__ double lane_d(double v, int l)
{
    const long long b = __builtin_bit_cast(long long, v);
    const int lo = __builtin_amdgcn_readlane(static_cast<int>(b), l);
    const int hi = __builtin_amdgcn_readlane(static_cast<int>(b >> 32), l);
    return __builtin_bit_cast(double, (static_cast<long long>(hi) << 32) | static_cast<unsigned int>(lo));
}

// sum / max over each 16-lane row, result in every lane of the row
__device__ __forceinline__ float row16_sum(float v)
{
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    v += dpp_f<0x141>(v);
    v += dpp_f<0x140>(v);
    return v;
}

__device__ __forceinline__ double row16_sum(double v)
{
    v += dpp_d<0xB1>(v);
    v += dpp_d<0x4E>(v);
    v += dpp_d<0x141>(v);
    v += dpp_d<0x140>(v);
    return v;
}

// fmaxf ignores a NaN operand, like the Lua `if v > mx` scan.
__device__ __forceinline__ float row16_max(float v)
{
    v = fmaxf(v, dpp_f<0xB1>(v));
    v = fmaxf(v, dpp_f<0x4E>(v));
    v = fmaxf(v, dpp_f<0x141>(v));
    v = fmaxf(v, dpp_f<0x140>(v));
    return v;
}

// Whole-wave reductions (every lane active); the result is wave-uniform.
__device__ __forceinline__ float wave_sum(float v)
{
    v = row16_sum(v);
    return (lane_f(v, 0) + lane_f(v, 16)) + (lane_f(v, 32) + lane_f(v, 48));
}

__device__ __forceinline__ double wave_sum(double v)
{
    v = row16_sum(v);
    return (lane_d(v, 0) + lane_d(v, 16)) + (lane_d(v, 32) + lane_d(v, 48));
}

__device__ __forceinline__ float wave_max(float v)
{
    v = row16_max(v);
    return fmaxf(fmaxf(lane_f(v, 0), lane_f(v, 16)), fmaxf(lane_f(v, 32), lane_f(v, 48)));
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

template <int CTRL>
__device__ __forceinline__ void argmax_step(float& bv, int& bi)
{
    const float ov = dpp_f<CTRL>(bv);
    const int oi = dpp_i<CTRL>(bi);
    argmax_merge(bv, bi, ov, oi);
}

// Whole-wave argmax (every lane active); the result is wave-uniform.  The
// merge is a total order (valid beats none, larger value, then lower index),
// so the reduction order does not change the result.
__device__ __forceinline__ void wave_argmax(float& bv, int& bi)
{
    argmax_step<0xB1>(bv, bi);
    argmax_step<0x4E>(bv, bi);
    argmax_step<0x141>(bv, bi);
    argmax_step<0x140>(bv, bi);
    float v = lane_f(bv, 0);
    int i = __builtin_amdgcn_readlane(bi, 0);
#pragma unroll
    for (int r = 16; r < 64; r += 16) argmax_merge(v, i, lane_f(bv, r), __builtin_amdgcn_readlane(bi, r));
    bv = v;
    bi = i;
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

// Column sums of one 32-column block over the NT threads of a workgroup:
// out[c] (+)= sum_b partial[b][c] for c in [c0, c0 + 32) (cols % 4 == 0,
// 16-byte aligned rows).  Thread (g, q) sums column quad q over the partial
// rows g, g + G, ... (G = NT/8 groups; eight loads in flight at a time); the G
// group sums are then added in a fixed tree through red (G x 8 float4 of
// LDS).  Deterministic.  Returns the float4 this thread stored (zeros for
// threads that store nothing).
template <int NT = 256>
__device__ inline float4 colsum4_block(const float* __restrict__ partial, int nparts, float* __restrict__ out,
                                       int cols, int c0, int acc, float4 (*red)[8])
{
    constexpr int G = NT / 8;
    const int q = threadIdx.x & 7, g = threadIdx.x >> 3;
    const int c = c0 + 4 * q;
    float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
    if (c < cols) {
        int b = g;
        for (; b + 7 * G < nparts; b += 8 * G) {
            float4 t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u)
                t[u] = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(b + u * G) * cols + c);
#pragma unroll
            for (int u = 0; u < 8; ++u) { s.x += t[u].x; s.y += t[u].y; s.z += t[u].z; s.w += t[u].w; }
        }
        for (; b < nparts; b += G) {
            const float4 t = *reinterpret_cast<const float4*>(partial + static_cast<size_t>(b) * cols + c);
            s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
        }
    }
    red[g][q] = s;
    __syncthreads();
#pragma unroll
    for (int half = G / 2; half > 0; half >>= 1) {
        if (g < half) {
            const float4 t = red[g + half][q];
            float4 u = red[g][q];
            u.x += t.x; u.y += t.y; u.z += t.z; u.w += t.w;
            red[g][q] = u;
        }
        __syncthreads();
    }
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
    if (g == 0 && c < cols) {
        t = red[0][q];
        float4* o = reinterpret_cast<float4*>(out + c);
        if (acc) {
            const float4 v = *o;
            t.x += v.x; t.y += v.y; t.z += v.z; t.w += v.w;
        }
        *o = t;
    }
    return t;
}
