// lhip_rows.hip -- row-wise bandwidth kernels: RMSNorm fwd/bwd, row softmax fwd/bwd,
// fused softmax + cross-entropy, row argmax.
//
// All are HBM-bound.  Rows up to a few thousand columns are held in registers
// by one wave64 per row (float4 = 128-bit loads, NV float4 per lane), so each
// input byte is read from HBM once and each output byte written once; the
// reductions stay inside the wave (__shfl_xor butterflies lowered to DPP /
// ds_swizzle).  Cross-entropy rows (V up to 32768) are held by a whole
// workgroup.  Shapes outside the register-resident envelope, or unaligned
// operands, take a generic multi-pass kernel with the same semantics.
//
// Semantics follow ai/core/tensor2.lua (the CPU LMTrain path):
//   rmsnorm  :609-666   softmax_rows :332-408   cross_entropy :809-882
// and the reference kernels' batched contracts (cuda/luaTL_train.cu):
//   softmax_ex group-causal mask :545-619, fused CE :837-891, argmax :982-1018.
#include <algorithm>
#include <cmath>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

constexpr int kRowThreads = 256;  // 4 waves, one row each
constexpr int kWavesPerBlock = kRowThreads / 64;

__device__ __forceinline__ float4 f4zero() { return make_float4(0.f, 0.f, 0.f, 0.f); }

__device__ __forceinline__ float f4get(const float4& v, int e)
{
    return e == 0 ? v.x : (e == 1 ? v.y : (e == 2 ? v.z : v.w));
}

__device__ __forceinline__ void f4set(float4& v, int e, float x)
{
    if (e == 0) v.x = x; else if (e == 1) v.y = x; else if (e == 2) v.z = x; else v.w = x;
}

typedef float vf4 __attribute__((ext_vector_type(4)));

// 128-bit load of data this kernel reads exactly once (non-temporal hint)
__device__ __forceinline__ float4 ld_stream(const float4* p)
{
    const vf4 v = __builtin_nontemporal_load(reinterpret_cast<const vf4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}

// Plain 128-bit load.  Which load form streams faster depends on the kernel
// (measured with non-temporal stores): plain loads for the RMSNorm forward
// (4096 x 1024: 65% of HBM against 63%) and the softmax forward (4096 x 4096:
// 70% against 67%); ld_stream for the RMSNorm backward (52% against 46%), the
// softmax backward and the fused CE (71% against 67%).
__device__ __forceinline__ float4 ld_row(const float4* p) { return *p; }

// 128-bit store of data this kernel writes once and does not read back
// (non-temporal hint: streamed to memory instead of being kept dirty in L2,
// which the end-of-kernel L2 write-back would otherwise have to flush).
__device__ __forceinline__ void st_stream(float4* p, const float4& v)
{
    __builtin_nontemporal_store(vf4{v.x, v.y, v.z, v.w}, reinterpret_cast<vf4*>(p));
}

// Waves walk rows grid-stride (row += total waves) and prefetch their next
// row into a second register set while they reduce and store the current
// one, so that reads and writes of different rows overlap.  The grid is
// capped at two workgroups (8 waves) per CU: on 4096 x 4096 softmax rows that
// runs at 68% of HBM against 62% with one row per wave and 16 waves per CU
// (all loads first, then all stores).
inline int row_wave_blocks(int rows)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    int b = ceil_div(rows, kWavesPerBlock);
    if (b > 2 * cus) b = 2 * cus;
    return b < 1 ? 1 : b;
}

// Run body(buf, row) over this wave's rows with a one-row prefetch:
// load(buf, row) fills a register set, body consumes it.
template <class Regs, int WPB = kWavesPerBlock, class Load, class Body>
__device__ __forceinline__ void walk_rows(int rows, Load load, Body body)
{
    const int nw = gridDim.x * WPB;
    int row = blockIdx.x * WPB + (threadIdx.x >> 6);
    if (row >= rows) return;
    Regs a, b;
    load(a, row);
    while (true) {
        int next = row + nw;
        if (next < rows) load(b, next);
        body(a, row);
        if (next >= rows) break;
        row = next;
        next = row + nw;
        if (next < rows) load(a, next);
        body(b, row);
        if (next >= rows) break;
        row = next;
    }
}

template <int NV>
struct Row1 {
    float4 v[NV];
};
template <int NV>
struct Row2 {
    float4 v[NV], g[NV];
    float r;   // per-row scalar loaded with the row (RMSNorm backward: 1/rms)
};

// ------------------------------------------------------------------ RMSNorm
// y = x * r * w, r = 1/sqrt(mean_j x^2 + eps); inv[row] = r (tensor2.lua:609-634).
// One wave per RPW consecutive rows, no walking: the wave issues every load
// of its rows (plain loads; addresses clamped into the matrix, so no load
// sits behind a branch) before the first reduction, then normalises and
// stores the rows one by one.  On 4096 x 1024 (RPW = 2, 512 workgroups) this
// streams at 84% of HBM, against 70% for waves walking rows grid-stride two
// workgroups per CU with a one-row prefetch.
template <int NV, int RPW>
__global__ void __launch_bounds__(kRowThreads)
rmsnorm_fwd_vec(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y,
                float* __restrict__ inv, int rows, int cols, float eps)
{
    const int lane = threadIdx.x & 63;
    const int c4n = cols >> 2;
    const int row0 = (blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6)) * RPW;
    if (row0 >= rows) return;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 v[RPW][NV], g[NV];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = min(row0 + r, rows - 1);
        const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * cols);
#pragma unroll
        for (int i = 0; i < NV; ++i) v[r][i] = ld_row(xr + min(lane + 64 * i, c4n - 1));
    }
    // the gain too, before the first reduction (a load issued after it would
    // stall every row's stores on its latency)
#pragma unroll
    for (int i = 0; i < NV; ++i) g[i] = w4[min(lane + 64 * i, c4n - 1)];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
        const int row = row0 + r;
        float ss = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const float t = v[r][i].x * v[r][i].x + v[r][i].y * v[r][i].y + v[r][i].z * v[r][i].z +
                            v[r][i].w * v[r][i].w;
            ss += lane + 64 * i < c4n ? t : 0.f;
        }
        ss = wave_sum(ss);
        if (row >= rows) break;   // wave-uniform
        const float rs = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
        float4* yr = reinterpret_cast<float4*>(y + static_cast<size_t>(row) * cols);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            if (c < c4n)
                st_stream(yr + c, make_float4(v[r][i].x * rs * g[i].x, v[r][i].y * rs * g[i].y,
                                             v[r][i].z * rs * g[i].z, v[r][i].w * rs * g[i].w));
        }
        if (inv && lane == 0) inv[row] = rs;
    }
}

__global__ void __launch_bounds__(kRowThreads)
rmsnorm_fwd_generic(const float* __restrict__ x, const float* __restrict__ w, float* __restrict__ y,
                    float* __restrict__ inv, int rows, int cols, float eps)
{
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + static_cast<size_t>(row) * cols;
    float ss = 0.f;
    for (int c = lane; c < cols; c += 64) ss += xr[c] * xr[c];
    ss = wave_sum(ss);
    const float r = 1.0f / sqrtf(ss / static_cast<float>(cols) + eps);
    float* yr = y + static_cast<size_t>(row) * cols;
    for (int c = lane; c < cols; c += 64) yr[c] = xr[c] * r * w[c];
    if (inv && lane == 0) inv[row] = r;
}

// dx = g*w*r - x*(r^3/N)*sum_j(g_j w_j x_j)  (+ dres, the incoming residual
// gradient, when given; dres may be dx itself);
// per-block partial dw over the block's rows -> partial[block][cols], skipped
// when partial is NULL (tensor2.lua:641-666).  NW waves per block, one row per
// wave at a time, rows walked grid-stride with a one-row prefetch; the waves'
// dw sums meet in LDS and are added in wave order.
template <int NV, int NW>
__global__ void __launch_bounds__(64 * NW)
rmsnorm_bwd_vec(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ inv,
                const float* __restrict__ dy, float* dx, const float* dres, float* __restrict__ partial,
                int rows, int cols)
{
    extern __shared__ float4 sdw[];   // [NW][cols/4]
    const int wv = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int c4n = cols >> 2;
    const float4* w4 = reinterpret_cast<const float4*>(w);
    float4 wr[NV], dwp[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + 64 * i;
        wr[i] = c < c4n ? w4[c] : f4zero();
        dwp[i] = f4zero();
    }
    const float inv_n = 1.0f / static_cast<float>(cols);
    auto load = [&](Row2<NV>& rr, int row) {
        const size_t base = static_cast<size_t>(row) * cols;
        const float4* xr = reinterpret_cast<const float4*>(x + base);
        const float4* gr = reinterpret_cast<const float4*>(dy + base);
        rr.r = inv[row];
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            rr.v[i] = c < c4n ? ld_stream(xr + c) : f4zero();
            rr.g[i] = c < c4n ? ld_stream(gr + c) : f4zero();
        }
    };
    auto body = [&](const Row2<NV>& rr, int row) {
        const size_t base = static_cast<size_t>(row) * cols;
        const float r = rr.r;
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i)
            dot += rr.g[i].x * wr[i].x * rr.v[i].x + rr.g[i].y * wr[i].y * rr.v[i].y +
                   rr.g[i].z * wr[i].z * rr.v[i].z + rr.g[i].w * wr[i].w * rr.v[i].w;
        dot = wave_sum(dot);
        const float coef = dot * r * r * r * inv_n;
        float4* dxr = reinterpret_cast<float4*>(dx + base);
        const float4* drr = reinterpret_cast<const float4*>(dres + base);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            if (c < c4n) {
                float4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float gg = f4get(rr.g[i], e), xx = f4get(rr.v[i], e);
                    f4set(o, e, gg * f4get(wr[i], e) * r - xx * coef);
                    f4set(dwp[i], e, f4get(dwp[i], e) + gg * xx * r);
                }
                if (dres) {
                    const float4 old = drr[c];
                    o.x += old.x; o.y += old.y; o.z += old.z; o.w += old.w;
                }
                st_stream(dxr + c, o);
            }
        }
    };
    walk_rows<Row2<NV>, NW>(rows, load, body);
    if (!partial) return;   // uniform: no dw wanted
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int c = lane + 64 * i;
        if (c < c4n) sdw[wv * c4n + c] = dwp[i];
    }
    __syncthreads();
    float4* pr = reinterpret_cast<float4*>(partial + static_cast<size_t>(blockIdx.x) * cols);
    for (int c = threadIdx.x; c < c4n; c += 64 * NW) {
        float4 s = sdw[c];
#pragma unroll
        for (int k = 1; k < NW; ++k) {
            const float4 t = sdw[k * c4n + c];
            s.x += t.x; s.y += t.y; s.z += t.z; s.w += t.w;
        }
        pr[c] = s;
    }
}

__global__ void __launch_bounds__(kRowThreads)
rmsnorm_bwd_generic(const float* __restrict__ x, const float* __restrict__ w, const float* __restrict__ inv,
                    const float* __restrict__ dy, float* dx, const float* dres, float* __restrict__ partial,
                    int rows, int cols)
{
    // one wave per row, rows grid-stride; dw partial per block accumulated
    // column by column through LDS-free atomics-free passes: each wave owns
    // its partial row in `partial` ([gridDim.x * waves][cols]), if given.
    const int wv = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int gw = blockIdx.x * kWavesPerBlock + wv;
    float* pw = partial ? partial + static_cast<size_t>(gw) * cols : nullptr;
    if (pw)
        for (int c = lane; c < cols; c += 64) pw[c] = 0.f;
    const float inv_n = 1.0f / static_cast<float>(cols);
    for (int row = gw; row < rows; row += gridDim.x * kWavesPerBlock) {
        const size_t base = static_cast<size_t>(row) * cols;
        float dot = 0.f;
        for (int c = lane; c < cols; c += 64) dot += dy[base + c] * w[c] * x[base + c];
        dot = wave_sum(dot);
        const float r = inv[row];
        const float coef = dot * r * r * r * inv_n;
        for (int c = lane; c < cols; c += 64) {
            const float gg = dy[base + c], xx = x[base + c];
            const float o = gg * w[c] * r - xx * coef;
            dx[base + c] = dres ? dres[base + c] + o : o;
            if (pw) pw[c] += gg * xx * r;
        }
    }
}

// dw[c] = (acc ? dw[c] : 0) + sum_b partial[b][c] in a fixed order: 32 columns
// per block, 8 thread groups each summing every 8th partial row (independent,
// unrolled loads), then the 8 group sums added in a fixed tree.  Deterministic.
// blockIdx.y selects one of up to kColsumJobs independent (partial, out) jobs.
struct ColsumJobs {
    const float* partial[kColsumJobs];
    float* out[kColsumJobs];
    int nparts[kColsumJobs];
};

// Float4 variant (cols % 4 == 0, 16-byte aligned partial rows and outputs):
// 32 columns per block; thread (g, q) sums column quad q over the partial rows
// g, g + 32, ... (eight loads in flight at a time), then the 32 group sums are
// added in a fixed tree.  Deterministic.
__global__ void __launch_bounds__(256)
colsum4_kernel(const ColsumJobs jobs, int cols, int acc)
{
    __shared__ float4 red[32][8];
    colsum4_block(jobs.partial[blockIdx.y], jobs.nparts[blockIdx.y], jobs.out[blockIdx.y], cols, blockIdx.x * 32, acc,
                  red);
}

__global__ void __launch_bounds__(256)
colsum_kernel(const ColsumJobs jobs, int cols, int acc)
{
    // 32 columns per block, 8 thread groups each summing every 8th partial row
    __shared__ float red[8][32];
    const float* __restrict__ partial = jobs.partial[blockIdx.y];
    float* __restrict__ out = jobs.out[blockIdx.y];
    const int nparts = jobs.nparts[blockIdx.y];
    const int cl = threadIdx.x & 31, g = threadIdx.x >> 5;
    const int c = blockIdx.x * 32 + cl;
    float s = 0.f;
    if (c < cols) {
#pragma unroll 8
        for (int b = g; b < nparts; b += 8) s += partial[static_cast<size_t>(b) * cols + c];
    }
    red[g][cl] = s;
    __syncthreads();
    if (g == 0 && c < cols) {
        const float t = ((red[0][cl] + red[1][cl]) + (red[2][cl] + red[3][cl])) +
                        ((red[4][cl] + red[5][cl]) + (red[6][cl] + red[7][cl]));
        out[c] = acc ? out[c] + t : t;
    }
}

// ------------------------------------------------------------- row softmax
// Row r keeps columns [0, lim): lim = cols, or with the (group-)causal mask
// lim = clamp((r % group) + 1 + offset, 1, cols) (tensor2.lua:332-383 with
// Lua's 1-based lim = i + offset; luaTL_softmax_ex's row % group).  Masked
// entries are exactly 0.  y = softmax(scale * x) over the kept prefix.  x and
// y must not overlap (the kernels are compiled with __restrict__).
__device__ __forceinline__ int softmax_lim(int row, int cols, int causal, int offset, int group)
{
    if (!causal) return cols;
    int lim = (row % group) + 1 + offset;
    return lim < 1 ? 1 : (lim > cols ? cols : lim);
}

template <int NV>
__global__ void __launch_bounds__(kRowThreads)
softmax_fwd_vec(const float* __restrict__ x, float* __restrict__ y, int rows, int cols, float scale,
                int causal, int offset, int group)
{
    const int lane = threadIdx.x & 63;
    const int c4n = cols >> 2;
    auto load = [&](Row1<NV>& r, int row) {
        const int lim = softmax_lim(row, cols, causal, offset, group);
        const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * cols);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            r.v[i] = (c < c4n && 4 * c < lim) ? ld_row(xr + c) : f4zero();
        }
    };
    auto body = [&](Row1<NV>& r, int row) {
        const int lim = softmax_lim(row, cols, causal, offset, group);
        float4* v = r.v;                     // transformed in place (register pressure)
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float sv = (4 * c + e < lim) ? scale * f4get(v[i], e) : -INFINITY;
                f4set(v[i], e, sv);
                mx = fmaxf(mx, sv);
            }
        }
        mx = wave_max(mx);
        if (mx == -INFINITY || mx != mx) mx = 0.f;
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ev = (4 * c + e < lim) ? expf(f4get(v[i], e) - mx) : 0.f;
                f4set(v[i], e, ev);
                sum += ev;
            }
        }
        sum = wave_sum(sum);
        if (!(sum > 0.f)) sum = 1.f;
        const float is = 1.0f / sum;
        float4* yr = reinterpret_cast<float4*>(y + static_cast<size_t>(row) * cols);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            if (c < c4n) st_stream(yr + c, make_float4(v[i].x * is, v[i].y * is, v[i].z * is, v[i].w * is));
        }
    };
    walk_rows<Row1<NV>>(rows, load, body);
}

// Long rows (2048 < cols <= 4096, cols % 1024 == 0): one BS-thread workgroup
// per row, NPT float4 per thread (column c4 = thread + BS i), the row max and
// sum meeting in LDS in wave order.  A workgroup per row puts many more rows'
// loads in flight than a wave per row at the same register cost per byte.
// FULL (no causal mask: every row keeps all its columns) loads without a
// condition, so no load waits behind another's select.  At 4096 x 4096, 512
// threads per row stream at 84% of HBM against 80% for 256.
template <int BS, int NPT, bool FULL>
__global__ void __launch_bounds__(BS)
softmax_fwd_blk(const float* __restrict__ x, float* __restrict__ y, int rows, int cols, float scale,
                int causal, int offset, int group)
{
    constexpr int NW = BS / 64;
    __shared__ float red[2][NW];
    const int row = blockIdx.x;
    const int t = threadIdx.x, wv = t >> 6;
    const int lim = FULL ? cols : softmax_lim(row, cols, causal, offset, group);
    const float4* xr = reinterpret_cast<const float4*>(x + static_cast<size_t>(row) * cols);
    float4 v[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
        if (FULL) v[i] = ld_row(xr + c);
        else v[i] = 4 * c < lim ? ld_row(xr + c) : f4zero();
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float sv = (FULL || 4 * c + e < lim) ? scale * f4get(v[i], e) : -INFINITY;
            f4set(v[i], e, sv);
            mx = fmaxf(mx, sv);
        }
    }
    mx = wave_max(mx);
    if ((t & 63) == 0) red[0][wv] = mx;
    __syncthreads();
    mx = red[0][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) mx = fmaxf(mx, red[0][k]);
    if (mx == -INFINITY || mx != mx) mx = 0.f;
    float sum = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float ev = (FULL || 4 * c + e < lim) ? expf(f4get(v[i], e) - mx) : 0.f;
            f4set(v[i], e, ev);
            sum += ev;
        }
    }
    sum = wave_sum(sum);
    if ((t & 63) == 0) red[1][wv] = sum;
    __syncthreads();
    sum = red[1][0];
#pragma unroll
    for (int k = 1; k < NW; ++k) sum += red[1][k];
    if (!(sum > 0.f)) sum = 1.f;
    const float is = 1.0f / sum;
    float4* yr = reinterpret_cast<float4*>(y + static_cast<size_t>(row) * cols);
#pragma unroll
    for (int i = 0; i < NPT; ++i)
        st_stream(yr + t + BS * i, make_float4(v[i].x * is, v[i].y * is, v[i].z * is, v[i].w * is));
}

__global__ void __launch_bounds__(kRowThreads)
softmax_fwd_generic(const float* __restrict__ x, float* __restrict__ y, int rows, int cols, float scale,
                    int causal, int offset, int group)
{
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int lim = softmax_lim(row, cols, causal, offset, group);
    const float* xr = x + static_cast<size_t>(row) * cols;
    float* yr = y + static_cast<size_t>(row) * cols;
    float mx = -INFINITY;
    for (int c = lane; c < lim; c += 64) mx = fmaxf(mx, scale * xr[c]);
    mx = wave_max(mx);
    if (mx == -INFINITY || mx != mx) mx = 0.f;
    float sum = 0.f;
    for (int c = lane; c < lim; c += 64) sum += expf(scale * xr[c] - mx);
    sum = wave_sum(sum);
    if (!(sum > 0.f)) sum = 1.f;
    const float is = 1.0f / sum;
    for (int c = lane; c < cols; c += 64) yr[c] = c < lim ? expf(scale * xr[c] - mx) * is : 0.f;
}

// dx = scale * y * (dy - sum_{j<lim} dy_j y_j) on the kept prefix, 0 beyond
// (+ dx if acc) (tensor2.lua:388-408 followed by the scale node's backward).
template <int NV>
__global__ void __launch_bounds__(kRowThreads)
softmax_bwd_vec(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx,
                int rows, int cols, float scale, int causal, int offset, int group, int acc)
{
    const int lane = threadIdx.x & 63;
    const int c4n = cols >> 2;
    auto load = [&](Row2<NV>& r, int row) {
        const int lim = softmax_lim(row, cols, causal, offset, group);
        const size_t base = static_cast<size_t>(row) * cols;
        const float4* yr = reinterpret_cast<const float4*>(y + base);
        const float4* gr = reinterpret_cast<const float4*>(dy + base);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            const bool in = c < c4n && 4 * c < lim;
            r.v[i] = in ? ld_stream(yr + c) : f4zero();
            r.g[i] = in ? ld_stream(gr + c) : f4zero();
        }
    };
    auto body = [&](const Row2<NV>& r, int row) {
        const int lim = softmax_lim(row, cols, causal, offset, group);
        float dot = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (4 * c + e < lim) dot += f4get(r.g[i], e) * f4get(r.v[i], e);
        }
        dot = wave_sum(dot);
        float4* dr = reinterpret_cast<float4*>(dx + static_cast<size_t>(row) * cols);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = lane + 64 * i;
            if (c < c4n) {
                float4 o;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    f4set(o, e, (4 * c + e < lim) ? scale * (f4get(r.v[i], e) * (f4get(r.g[i], e) - dot)) : 0.f);
                if (acc) {
                    const float4 old = dr[c];
                    o.x += old.x; o.y += old.y; o.z += old.z; o.w += old.w;
                }
                st_stream(dr + c, o);
            }
        }
    };
    walk_rows<Row2<NV>>(rows, load, body);
}

// Long rows as softmax_fwd_blk: one BS-thread workgroup per row; FULL (no
// mask) loads y and dy without a condition (non-temporal: at 4096 x 4096 that
// streams at 80% of HBM, against 69% with the masked loads).
template <int BS, int NPT, bool FULL>
__global__ void __launch_bounds__(BS)
softmax_bwd_blk(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx,
                int rows, int cols, float scale, int causal, int offset, int group, int acc)
{
    constexpr int NW = BS / 64;
    __shared__ float red[NW];
    const int row = blockIdx.x;
    const int t = threadIdx.x, wv = t >> 6;
    const int lim = FULL ? cols : softmax_lim(row, cols, causal, offset, group);
    const size_t base = static_cast<size_t>(row) * cols;
    const float4* yr = reinterpret_cast<const float4*>(y + base);
    const float4* gr = reinterpret_cast<const float4*>(dy + base);
    float4 v[NPT], g[NPT];
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
        if (FULL) {
            v[i] = ld_stream(yr + c);
            g[i] = ld_stream(gr + c);
        } else {
            const bool in = 4 * c < lim;
            v[i] = in ? ld_stream(yr + c) : f4zero();
            g[i] = in ? ld_stream(gr + c) : f4zero();
        }
    }
    float dot = 0.f;
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (FULL || 4 * c + e < lim) dot += f4get(g[i], e) * f4get(v[i], e);
    }
    dot = wave_sum(dot);
    if ((t & 63) == 0) red[wv] = dot;
    __syncthreads();
    dot = red[0];
#pragma unroll
    for (int k = 1; k < NW; ++k) dot += red[k];
    float4* dr = reinterpret_cast<float4*>(dx + base);
#pragma unroll
    for (int i = 0; i < NPT; ++i) {
        const int c = t + BS * i;
        float4 o;
#pragma unroll
        for (int e = 0; e < 4; ++e)
            f4set(o, e, (FULL || 4 * c + e < lim) ? scale * (f4get(v[i], e) * (f4get(g[i], e) - dot)) : 0.f);
        if (acc) {
            const float4 old = dr[c];
            o.x += old.x; o.y += old.y; o.z += old.z; o.w += old.w;
        }
        st_stream(dr + c, o);
    }
}

__global__ void __launch_bounds__(kRowThreads)
softmax_bwd_generic(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx,
                    int rows, int cols, float scale, int causal, int offset, int group, int acc)
{
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const int lim = softmax_lim(row, cols, causal, offset, group);
    const size_t base = static_cast<size_t>(row) * cols;
    float dot = 0.f;
    for (int c = lane; c < lim; c += 64) dot += dy[base + c] * y[base + c];
    dot = wave_sum(dot);
    for (int c = lane; c < cols; c += 64) {
        const float o = c < lim ? scale * (y[base + c] * (dy[base + c] - dot)) : 0.f;
        dx[base + c] = acc ? dx[base + c] + o : o;
    }
}

// ------------------------------------------------- fused softmax + cross-entropy
// Per row r with target t: rows with t < 0, t >= V or t == ignore_index give
// loss 0 and dlogits 0; otherwise loss[r] = logsumexp(x) - x[t] and
// dlogits = gscale * (softmax(x) - onehot(t)).  dlogits may alias logits.
// With row_len (the LM step's windows of `period` rows), a counted row's scale
// is gscale / row_len[row / period]: each window's CE is the mean over its
// own length (tensor2.lua:845-857).
// (tensor2.lua:809-882 per row; cuda/luaTL_train.cu:837-878 contract.)
template <int NT, int NV, bool PF>
__global__ void __launch_bounds__(NT)
ce_fused_vec(const float* logits, const int* __restrict__ tgt, float* __restrict__ losses,
             float* dlogits, int* __restrict__ amax, int rows, int V, int ignore_index, float gscale,
             const int* __restrict__ row_len, int period)
{
    // One workgroup per row at a time.  With PF, rows are walked block-stride
    // and the next row is prefetched into registers while the current one is
    // reduced and its dlogits written (reads and writes of different rows
    // overlap); without PF (rows too long for two register copies) each
    // workgroup takes one row.
    constexpr int NW = NT / 64;
    __shared__ float red[NW];
    __shared__ float redv[NW];
    __shared__ int redi[NW];
    const int c4n = V >> 2;
    auto load = [&](Row1<NV>& r, int row) {
        const float4* xr = reinterpret_cast<const float4*>(logits + static_cast<size_t>(row) * V);
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = threadIdx.x + NT * i;
            r.v[i] = c < c4n ? ld_stream(xr + c) : make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        }
    };
    auto body = [&](Row1<NV>& r, int row) {
        const int t = tgt[row];
        const size_t base = static_cast<size_t>(row) * V;
        if (amax) {   // argmax of the raw logits, for every row (ignored targets included)
            float bv = -INFINITY;
            int bi = -1;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = threadIdx.x + NT * i;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (c < c4n && f4get(r.v[i], e) > bv) { bv = f4get(r.v[i], e); bi = 4 * c + e; }
            }
            const int am = block_argmax<NW>(bv, bi, redv, redi);
            if (threadIdx.x == 0) amax[row] = am < 0 ? 0 : am;
        }
        if (t < 0 || t >= V || t == ignore_index) {      // uniform in the block
            if (losses && threadIdx.x == 0) losses[row] = 0.f;
            if (dlogits) {
                float4* dr = reinterpret_cast<float4*>(dlogits + base);
                for (int c = threadIdx.x; c < c4n; c += NT) st_stream(dr + c, f4zero());
            }
            return;
        }
        const float xt = logits[base + t];   // read before any thread writes this row's dlogits
        float4* v = r.v;                     // transformed in place (register pressure)
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < NV; ++i) mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
        mx = block_max<NW>(mx, red);
        float sum = 0.f;
#pragma unroll
        for (int i = 0; i < NV; ++i) {
            const int c = threadIdx.x + NT * i;
            if (c < c4n) {
                v[i].x = expf(v[i].x - mx); v[i].y = expf(v[i].y - mx);
                v[i].z = expf(v[i].z - mx); v[i].w = expf(v[i].w - mx);
                sum += (v[i].x + v[i].y) + (v[i].z + v[i].w);
            }
        }
        sum = block_sum<NW>(sum, red);
        if (losses && threadIdx.x == 0) losses[row] = (mx + logf(sum)) - xt;
        if (dlogits) {
            const float is = 1.0f / sum;
            const float gs = row_len ? gscale / static_cast<float>(row_len[row / period]) : gscale;
            float4* dr = reinterpret_cast<float4*>(dlogits + base);
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int c = threadIdx.x + NT * i;
                if (c < c4n) {
                    float4 o;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        float p = f4get(v[i], e) * is;
                        if (4 * c + e == t) p -= 1.f;
                        f4set(o, e, gs * p);
                    }
                    st_stream(dr + c, o);
                }
            }
        }
        __syncthreads();   // red[] is reused by the next row's reductions
    };
    int row = blockIdx.x;
    if (row >= rows) return;
    Row1<NV> a;
    load(a, row);
    if (!PF) {
        body(a, row);
        return;
    }
    Row1<NV> b;
    while (true) {
        int next = row + gridDim.x;
        if (next < rows) load(b, next);
        body(a, row);
        if (next >= rows) break;
        row = next;
        next = row + gridDim.x;
        if (next < rows) load(a, next);
        body(b, row);
        if (next >= rows) break;
        row = next;
    }
}

__global__ void __launch_bounds__(256)
ce_fused_generic(const float* logits, const int* __restrict__ tgt, float* __restrict__ losses,
                 float* dlogits, int* __restrict__ amax, int rows, int V, int ignore_index, float gscale,
                 const int* __restrict__ row_len, int period)
{
    __shared__ float red[4];
    __shared__ float redv[4];
    __shared__ int redi[4];
    const int row = blockIdx.x;
    const int t = tgt[row];
    const size_t base = static_cast<size_t>(row) * V;
    if (amax) {
        float bv = -INFINITY;
        int bi = -1;
        for (int c = threadIdx.x; c < V; c += 256)
            if (logits[base + c] > bv) { bv = logits[base + c]; bi = c; }
        const int am = block_argmax<4>(bv, bi, redv, redi);
        if (threadIdx.x == 0) amax[row] = am < 0 ? 0 : am;
    }
    if (t < 0 || t >= V || t == ignore_index) {
        if (losses && threadIdx.x == 0) losses[row] = 0.f;
        if (dlogits) for (int c = threadIdx.x; c < V; c += 256) dlogits[base + c] = 0.f;
        return;
    }
    const float xt = logits[base + t];
    float mx = -INFINITY;
    for (int c = threadIdx.x; c < V; c += 256) mx = fmaxf(mx, logits[base + c]);
    mx = block_max<4>(mx, red);
    float sum = 0.f;
    for (int c = threadIdx.x; c < V; c += 256) sum += expf(logits[base + c] - mx);
    sum = block_sum<4>(sum, red);
    if (losses && threadIdx.x == 0) losses[row] = (mx + logf(sum)) - xt;
    if (dlogits) {
        const float is = 1.0f / sum;
        const float gs = row_len ? gscale / static_cast<float>(row_len[row / period]) : gscale;
        // every element is read before the same thread overwrites it
        for (int c = threadIdx.x; c < V; c += 256) {
            float p = expf(logits[base + c] - mx) * is;
            if (c == t) p -= 1.f;
            dlogits[base + c] = gs * p;
        }
    }
}

// ------------------------------------------------------------------ argmax
// First index of the row maximum under a strict '>' scan from -inf: NaN never
// wins, ties go to the lowest index, a row of only -inf/NaN gives 0
// (lmtrain.lua:1200-1209; cuda/luaTL_train.cu:982-1018).  Bit-exact.
__global__ void __launch_bounds__(kRowThreads)
argmax_rows_kernel(const float* __restrict__ x, int* __restrict__ out, int rows, int cols)
{
    const int row = blockIdx.x * kWavesPerBlock + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= rows) return;
    const float* xr = x + static_cast<size_t>(row) * cols;
    float bv = -INFINITY;
    int bi = -1;
    for (int c = lane; c < cols; c += 64) {
        const float v = xr[c];
        if (v > bv) { bv = v; bi = c; }
    }
    wave_argmax(bv, bi);
    if (lane == 0) out[row] = bi < 0 ? 0 : bi;
}

int nv_for(int cols)  // float4 per lane needed for a wave-resident row
{
    const int per_lane = (cols + 255) / 256;
    if (per_lane <= 1) return 1;
    if (per_lane <= 2) return 2;
    if (per_lane <= 4) return 4;
    if (per_lane <= 8) return 8;
    if (per_lane <= 16) return 16;
    return 0;
}

inline int row_blocks(int rows) { return ceil_div(rows, kWavesPerBlock); }

}  // namespace

// ------------------------------------------------------------------ launchers
int rmsnorm_fwd(const float* x, const float* w, float* y, float* inv, int rows, int cols, float eps,
                hipStream_t s)
{
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "rmsnorm_fwd: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !w || !y) return fail(LHIP_E_NULL, "rmsnorm_fwd: NULL x/w/y");
    if (!(eps >= 0.f)) return fail(LHIP_E_ARG, "rmsnorm_fwd: eps must be >= 0");
    const int nv = nv_for(cols);
    const bool vec = nv && cols % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(y);
    if (!vec) {
        klaunch(rmsnorm_fwd_generic, row_blocks(rows), kRowThreads, 0, s, x, w, y, inv, rows, cols, eps);
        return check_launch("rmsnorm_fwd");
    }
    // two rows per wave once that still gives every CU two workgroups
    // (and the rows fit: NV <= 4); otherwise one
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const int rpw = (nv <= 4 && rows >= 2 * kWavesPerBlock * 2 * cus) ? 2 : 1;
    const dim3 g(ceil_div(rows, kWavesPerBlock * rpw)), b(kRowThreads);
#define LHIP_RMF(NV_, RPW_) klaunch(rmsnorm_fwd_vec<NV_, RPW_>, g, b, 0, s, x, w, y, inv, rows, cols, eps)
    if (nv == 1) { if (rpw == 2) LHIP_RMF(1, 2); else LHIP_RMF(1, 1); }
    else if (nv == 2) { if (rpw == 2) LHIP_RMF(2, 2); else LHIP_RMF(2, 1); }
    else if (nv == 4) { if (rpw == 2) LHIP_RMF(4, 2); else LHIP_RMF(4, 1); }
    else if (nv == 8) LHIP_RMF(8, 1);
    else LHIP_RMF(16, 1);
#undef LHIP_RMF
    return check_launch("rmsnorm_fwd");
}

// Waves per workgroup of the register-resident backward: 8 for rows up to
// 2048 floats, 4 up to 4096 (the waves' dw partials then fill at most 64 KB of
// LDS, and two rows of x and dy -- the prefetch -- plus w and the dw sums fit a
// wave's registers).  With one workgroup per CU, 8 waves walking two rows each
// beat 16 waves taking one row each (all loads first, then all stores) by 25%
// at 4096 x 1024.
int rmsnorm_bwd_waves(int cols)
{
    return nv_for(cols) == 16 ? 4 : 8;
}

// Workgroups of the backward: at most one per CU (which bounds the dw partial
// rows, one per workgroup), each wave taking a row at a time.
int rmsnorm_bwd_blocks(int rows, int waves)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    int blocks = ceil_div(rows, waves);
    if (blocks > cus) blocks = cus;
    return blocks < 1 ? 1 : blocks;
}

// Upper bound on the partial-dw rows the backward uses (workspace = parts * cols
// floats): one per block on the register-resident path, one per wave otherwise.
int rmsnorm_bwd_parts(int rows, int cols)
{
    return std::max(rmsnorm_bwd_blocks(rows, rmsnorm_bwd_waves(cols)),
                    rmsnorm_bwd_blocks(rows, kWavesPerBlock) * kWavesPerBlock);
}

int rmsnorm_bwd_rows(const float* x, const float* w, const float* inv, const float* dy, float* dx,
                     const float* dres, float* partial, size_t partial_floats, int rows, int cols, int* parts_out,
                     hipStream_t s)
{
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "rmsnorm_bwd: rows=%d cols=%d", rows, cols);
    if (parts_out) *parts_out = 0;
    if (rows == 0) return LHIP_OK;
    if (!x || !w || !inv || !dy || !dx) return fail(LHIP_E_NULL, "rmsnorm_bwd: NULL argument");
    const int nv = nv_for(cols);
    const bool vec = nv && cols % 4 == 0 && aligned16(x) && aligned16(w) && aligned16(dy) && aligned16(dx) &&
                     (!dres || aligned16(dres));
    const int nw = vec ? rmsnorm_bwd_waves(cols) : kWavesPerBlock;
    const int blocks = rmsnorm_bwd_blocks(rows, nw);
    const int parts = vec ? blocks : blocks * kWavesPerBlock;
    if (partial && static_cast<size_t>(parts) * cols > partial_floats)
        return fail(LHIP_E_CAPACITY, "rmsnorm_bwd: workspace of %zu floats < %lld needed", partial_floats,
                    static_cast<long long>(parts) * cols);
    const dim3 g(blocks);
    const size_t lds = static_cast<size_t>(nw) * cols * sizeof(float);
#define LHIP_RBV(NV_, NW_) \
    klaunch(rmsnorm_bwd_vec<NV_, NW_>, g, 64 * NW_, lds, s, x, w, inv, dy, dx, dres, partial, rows, cols)
    if (!vec) klaunch(rmsnorm_bwd_generic, g, kRowThreads, 0, s, x, w, inv, dy, dx, dres, partial, rows, cols);
    else if (nv == 1) LHIP_RBV(1, 8);
    else if (nv == 2) LHIP_RBV(2, 8);
    else if (nv == 4) LHIP_RBV(4, 8);
    else if (nv == 8) LHIP_RBV(8, 8);
    else LHIP_RBV(16, 4);
#undef LHIP_RBV
    if (parts_out) *parts_out = parts;
    return check_launch("rmsnorm_bwd");
}

int rmsnorm_bwd_colsum(const float* partial, int parts, float* dw, int cols, int accumulate, hipStream_t s)
{
    return rmsnorm_bwd_colsum_multi(&partial, &parts, &dw, 1, cols, accumulate, s);
}

int rmsnorm_bwd_colsum_multi(const float* const* partials, const int* parts, float* const* dws, int njobs, int cols,
                             int accumulate, hipStream_t s)
{
    if (njobs < 0 || njobs > kColsumJobs) return fail(LHIP_E_ARG, "colsum: %d jobs (at most %d)", njobs, kColsumJobs);
    ColsumJobs jobs{};
    int n = 0;
    for (int i = 0; i < njobs; ++i) {
        if (parts[i] <= 0) continue;
        if (!partials[i] || !dws[i]) return fail(LHIP_E_NULL, "colsum: NULL partials/output");
        jobs.partial[n] = partials[i];
        jobs.out[n] = dws[i];
        jobs.nparts[n] = parts[i];
        ++n;
    }
    if (n == 0) return LHIP_OK;
    bool vec = cols % 4 == 0;
    for (int i = 0; i < n; ++i) vec = vec && aligned16(jobs.partial[i]) && aligned16(jobs.out[i]);
    if (vec) klaunch(colsum4_kernel, dim3(ceil_div(cols, 32), n), 256, 0, s, jobs, cols, accumulate);
    else klaunch(colsum_kernel, dim3(ceil_div(cols, 32), n), 256, 0, s, jobs, cols, accumulate);
    return check_launch("rmsnorm_bwd: dw reduce");
}

int rmsnorm_bwd(const float* x, const float* w, const float* inv, const float* dy, float* dx, float* dw,
                int rows, int cols, int accumulate, float* work, size_t work_floats, hipStream_t s)
{
    if (dw && !work) return fail(LHIP_E_NULL, "rmsnorm_bwd: no workspace for dw");
    int parts = 0;
    int rc = rmsnorm_bwd_rows(x, w, inv, dy, dx, accumulate ? dx : nullptr, dw ? work : nullptr, work_floats,
                              rows, cols, &parts, s);
    if (rc != LHIP_OK || !dw) return rc;
    return rmsnorm_bwd_colsum(work, parts, dw, cols, accumulate, s);
}

int softmax_fwd(const float* x, float* y, int rows, int cols, float scale, int causal, int offset, int group,
                hipStream_t s)
{
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "softmax_fwd: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !y) return fail(LHIP_E_NULL, "softmax_fwd: NULL x/y");
    if (group <= 0) group = rows;
    const int nv = nv_for(cols);
    const bool vec = nv && cols % 4 == 0 && aligned16(x) && aligned16(y);
    dim3 g(vec ? row_wave_blocks(rows) : row_blocks(rows)), b(kRowThreads);
#define LHIP_SMF(NV_) klaunch(softmax_fwd_vec<NV_>, g, b, 0, s, x, y, rows, cols, scale, causal, offset, group)
    if (vec && cols > 2048 && cols <= 4096 && cols % 1024 == 0) {
#define LHIP_SMFB(BS_, NPT_, FULL_) klaunch(softmax_fwd_blk<BS_, NPT_, FULL_>, dim3(rows), dim3(BS_), 0, s, x, y, rows, \
                                            cols, scale, causal, offset, group)
        if (cols == 3072) { if (causal) LHIP_SMFB(256, 3, false); else LHIP_SMFB(256, 3, true); }
        else { if (causal) LHIP_SMFB(512, 2, false); else LHIP_SMFB(512, 2, true); }
#undef LHIP_SMFB
    }
    else if (!vec) klaunch(softmax_fwd_generic, g, b, 0, s, x, y, rows, cols, scale, causal, offset, group);
    else if (nv == 1) LHIP_SMF(1);
    else if (nv == 2) LHIP_SMF(2);
    else if (nv == 4) LHIP_SMF(4);
    else if (nv == 8) LHIP_SMF(8);
    else LHIP_SMF(16);
#undef LHIP_SMF
    return check_launch("softmax_fwd");
}

int softmax_bwd(const float* y, const float* dy, float* dx, int rows, int cols, float scale, int causal,
                int offset, int group, int accumulate, hipStream_t s)
{
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "softmax_bwd: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!y || !dy || !dx) return fail(LHIP_E_NULL, "softmax_bwd: NULL y/dy/dx");
    if (group <= 0) group = rows;
    const int nv = nv_for(cols);
    const bool vec = nv && cols % 4 == 0 && aligned16(y) && aligned16(dy) && aligned16(dx);
    dim3 g(vec ? row_wave_blocks(rows) : row_blocks(rows)), b(kRowThreads);
#define LHIP_SMB(NV_) klaunch(softmax_bwd_vec<NV_>, g, b, 0, s, y, dy, dx, rows, cols, scale, causal, offset, group, accumulate)
    if (vec && cols > 2048 && cols <= 4096 && cols % 1024 == 0) {
#define LHIP_SMBB(BS_, NPT_, FULL_) klaunch(softmax_bwd_blk<BS_, NPT_, FULL_>, dim3(rows), dim3(BS_), 0, s, y, dy, dx, \
                                            rows, cols, scale, causal, offset, group, accumulate)
        if (cols == 3072) { if (causal) LHIP_SMBB(256, 3, false); else LHIP_SMBB(256, 3, true); }
        else { if (causal) LHIP_SMBB(256, 4, false); else LHIP_SMBB(256, 4, true); }
#undef LHIP_SMBB
    }
    else if (!vec) klaunch(softmax_bwd_generic, g, b, 0, s, y, dy, dx, rows, cols, scale, causal, offset, group, accumulate);
    else if (nv == 1) LHIP_SMB(1);
    else if (nv == 2) LHIP_SMB(2);
    else if (nv == 4) LHIP_SMB(4);
    else if (nv == 8) LHIP_SMB(8);
    else LHIP_SMB(16);
#undef LHIP_SMB
    return check_launch("softmax_bwd");
}

int ce_fused(const float* logits, const int* tgt, float* losses, float* dlogits, int rows, int V,
             int ignore_index, float gscale, hipStream_t s, int* amax, const int* row_len, int period)
{
    if (rows < 0 || V <= 0) return fail(LHIP_E_SHAPE, "ce_fused: rows=%d vocab=%d", rows, V);
    if (rows == 0) return LHIP_OK;
    if (!logits || !tgt) return fail(LHIP_E_NULL, "ce_fused: NULL logits/targets");
    if (row_len && period <= 0) return fail(LHIP_E_ARG, "ce_fused: window period %d must be > 0", period);
    const bool vec = V % 4 == 0 && aligned16(logits) && (!dlogits || aligned16(dlogits));
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    // rows walked block-stride: about 2 rows per workgroup once rows exceed the CUs
    const int nb_small = rows < 4 * cus ? rows : 4 * cus;
    if (vec && V <= 256 * 4 * 2)
        klaunch(ce_fused_vec<256, 2, true>, nb_small, 256, 0, s, logits, tgt, losses, dlogits, amax, rows, V, ignore_index, gscale,
                                                          row_len, period);
    else if (vec && V <= 256 * 4 * 8)
        klaunch(ce_fused_vec<256, 8, true>, nb_small, 256, 0, s, logits, tgt, losses, dlogits, amax, rows, V, ignore_index, gscale,
                                                          row_len, period);
    else if (vec && V <= 1024 * 4 * 8)
        klaunch(ce_fused_vec<1024, 8, false>, rows, 1024, 0, s, logits, tgt, losses, dlogits, amax, rows, V, ignore_index, gscale,
                                                          row_len, period);
    else
        klaunch(ce_fused_generic, rows, 256, 0, s, logits, tgt, losses, dlogits, amax, rows, V, ignore_index, gscale,
                                                          row_len, period);
    return check_launch("ce_fused");
}

int argmax_rows(const float* x, int* out, int rows, int cols, hipStream_t s)
{
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "argmax_rows: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !out) return fail(LHIP_E_NULL, "argmax_rows: NULL x/out");
    klaunch(argmax_rows_kernel, row_blocks(rows), kRowThreads, 0, s, x, out, rows, cols);
    return check_launch("argmax_rows");
}

}  // namespace lhip

using lhip::st;

extern "C" {

LHIP_API int lhip_rmsnorm_fwd(const float* x, const float* w, float* y, float* inv, int rows, int cols, float eps)
{
    LHIP_REQUIRE_READY();
    return lhip::rmsnorm_fwd(x, w, y, inv, rows, cols, eps, st().stream);
}

LHIP_API int lhip_rmsnorm_bwd(const float* x, const float* w, const float* inv, const float* dy,
                              float* dx, float* dw, int rows, int cols, int accumulate)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return lhip::fail(LHIP_E_SHAPE, "rmsnorm_bwd: rows=%d cols=%d", rows, cols);
    float* work = nullptr;
    const size_t need = static_cast<size_t>(lhip::rmsnorm_bwd_parts(rows, cols)) * cols;
    if (dw && rows > 0) {
        int rc = lhip::workspace(need * sizeof(float), reinterpret_cast<void**>(&work));
        if (rc != LHIP_OK) return rc;
    }
    return lhip::rmsnorm_bwd(x, w, inv, dy, dx, dw, rows, cols, accumulate, work, need, st().stream);
}

LHIP_API int lhip_softmax_fwd(const float* x, float* y, int rows, int cols, float scale, int causal,
                              int offset, int group)
{
    LHIP_REQUIRE_READY();
    return lhip::softmax_fwd(x, y, rows, cols, scale, causal, offset, group, st().stream);
}

LHIP_API int lhip_softmax_bwd(const float* y, const float* dy, float* dx, int rows, int cols, float scale,
                              int causal, int offset, int group, int accumulate)
{
    LHIP_REQUIRE_READY();
    return lhip::softmax_bwd(y, dy, dx, rows, cols, scale, causal, offset, group, accumulate, st().stream);
}

LHIP_API int lhip_ce_fused(const float* logits, const int* targets, float* losses, float* dlogits,
                           int rows, int vocab, int ignore_index, float grad_scale)
{
    LHIP_REQUIRE_READY();
    return lhip::ce_fused(logits, targets, losses, dlogits, rows, vocab, ignore_index, grad_scale, st().stream);
}

LHIP_API int lhip_argmax_rows(const float* x, int* out, int rows, int cols)
{
    LHIP_REQUIRE_READY();
    return lhip::argmax_rows(x, out, rows, cols, st().stream);
}

}  // extern "C"
