// lhip_optim.hip -- gradient norm and the SGD step of the CPU LMTrain path, on device.
//
// optim2.lua: grad_norm :27-38, scale_grads :40-46, SGD :72-99; the step
// logic of lmtrain.lua:1212-1226 (scale by 1/B, global L2 norm, skip the step
// when the norm is not finite, clip to clip_norm, update).  The norm never
// leaves the device: a deterministic two-stage reduction writes it to device
// memory and the update kernel reads it, so a step needs no host round trip.
#include <cmath>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

constexpr int kRedThreads = 256;
constexpr int kRedMaxBlocks = 1024;

// partial[b] = sum of x^2 over block b's grid-stride share (double accumulation)
__global__ void __launch_bounds__(kRedThreads)
sumsq_stage1(const float* __restrict__ x, long long n, double* __restrict__ partial, int vec)
{
    __shared__ double red[kRedThreads / 64];
    const long long stride = static_cast<long long>(gridDim.x) * kRedThreads;
    const long long t0 = blockIdx.x * static_cast<long long>(kRedThreads) + threadIdx.x;
    double s = 0.0;
    if (vec) {
        // four grid-stride float4 per pass, all loaded before the first add
        // (the summation order is the plain grid-stride order)
        const float4* x4 = reinterpret_cast<const float4*>(x);
        const long long n4 = n >> 2;
        for (long long base = t0; base < n4; base += 4 * stride) {
            float4 v[4];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const long long i = base + k * stride;
                v[k] = i < n4 ? x4[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                if (base + k * stride >= n4) break;
                s += static_cast<double>(v[k].x) * v[k].x + static_cast<double>(v[k].y) * v[k].y +
                     static_cast<double>(v[k].z) * v[k].z + static_cast<double>(v[k].w) * v[k].w;
            }
        }
        for (long long i = 4 * n4 + t0; i < n; i += stride) s += static_cast<double>(x[i]) * x[i];
    } else {
        for (long long i = t0; i < n; i += stride) s += static_cast<double>(x[i]) * x[i];
    }
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
        for (int i = 0; i < kRedThreads / 64; ++i) t += red[i];
        partial[blockIdx.x] = t;
    }
}

// out[0] = sum of partial[0..nb) in a fixed order
__global__ void __launch_bounds__(64) sum_stage2(const double* __restrict__ partial, int nb, double* __restrict__ out)
{
    double s = 0.0;
    for (int i = threadIdx.x; i < nb; i += 64) s += partial[i];
    s = wave_sum(s);
    if (threadIdx.x == 0) out[0] = s;
}

// Global gradient norm from the stage-1 partials (nparts > 0; every block sums
// them in sum_stage2's order, so all blocks, and the two-kernel form, agree bit
// for bit) or from the finished total (nparts == 0).
// The squared gradient norm from the producers' per-workgroup partials, the
// same value in every block (every block sums them in the same order).  All
// 256 threads load: up to 4 partials each, every load issued before the
// first add (indices clamped, masked in the sum), so a block waits for one
// load round trip instead of one per 64 partials; then the four waves' sums
// meet in LDS in wave order.  Called by every thread of a 256-thread block.
__device__ __forceinline__ double grad_total(const double* __restrict__ sumsq, int nparts)
{
    if (nparts <= 0) return sumsq[0];
    __shared__ double part[4];
    constexpr int kPer = 4;
    double t[kPer];
#pragma unroll
    for (int j = 0; j < kPer; ++j) t[j] = sumsq[min(static_cast<int>(threadIdx.x) + 256 * j, nparts - 1)];
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < kPer; ++j) s += static_cast<int>(threadIdx.x) + 256 * j < nparts ? t[j] : 0.0;
    for (int i = static_cast<int>(threadIdx.x) + 256 * kPer; i < nparts; i += 256) s += sumsq[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
    __syncthreads();
    return ((part[0] + part[1]) + part[2]) + part[3];
}

__device__ __forceinline__ float ld_lane(const float4& v, int k) { return k == 0 ? v.x : k == 1 ? v.y : k == 2 ? v.z : v.w; }
__device__ __forceinline__ void st_lane(float4& v, int k, float x)
{
    if (k == 0) v.x = x; else if (k == 1) v.y = x; else if (k == 2) v.z = x; else v.w = x;
}

struct SgdHyper {
    float lr, momentum, wd, grad_scale;
    int nesterov;
};

// optim2.SGD on one element after scale and clip; g receives the gradient used
__device__ __forceinline__ void sgd_elem(float& p, float& g, float& v, const SgdHyper& h, float clipf)
{
    float gk = g * h.grad_scale;
    if (clipf != 1.0f) gk = gk * clipf;
    g = gk;
    if (h.wd != 0.f) gk = gk + h.wd * p;
    if (h.momentum > 0.f) {
        const float vk = h.momentum * v + gk;
        v = vk;
        p = h.nesterov ? p - h.lr * (gk + h.momentum * vk) : p - h.lr * vk;
    } else {
        p = p - h.lr * gk;
    }
}

// One SGD step over n parameters with the LMTrain step logic.  sumsq is the
// sum of squares of the RAW gradients; the norm of the scaled gradients is
// grad_scale * sqrt(sumsq).  g is overwritten with the gradient actually used
// (after scale and clip) so callers can inspect it, as optim2 mutates grads.
// With vec (p, g, v 16-byte aligned) the body runs on float4; a thread's first
// float4 is fetched before the norm is reduced, so the loads overlap it.
typedef float nt_f4 __attribute__((ext_vector_type(4)));
__global__ void __launch_bounds__(256)
sgd_step_kernel(float* __restrict__ p, float* __restrict__ g, float* __restrict__ v, long long n,
                const double* __restrict__ sumsq, int nparts, float lr, float momentum, float wd,
                float grad_scale, float clip_norm, int nesterov, float* __restrict__ gnorm_out,
                int* __restrict__ applied_out, const float* __restrict__ hyper, int vec)
{
    if (hyper) {   // hyper-parameters resident on the device (graph replay)
        lr = hyper[0]; momentum = hyper[1]; wd = hyper[2]; clip_norm = hyper[3];
        nesterov = hyper[4] != 0.f; grad_scale = hyper[9];
    }
    const SgdHyper hy{lr, momentum, wd, grad_scale, nesterov};
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long n4 = vec ? (n >> 2) : 0;
    float4* p4 = reinterpret_cast<float4*>(p);
    float4* g4 = reinterpret_cast<float4*>(g);
    float4* v4 = reinterpret_cast<float4*>(v);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 pv = z4, gv = z4, vv = z4;
    if (t0 < n4) {
        gv = g4[t0];
        pv = p4[t0];
        if (momentum > 0.f) vv = v4[t0];
    }
    const double norm = static_cast<double>(grad_scale) * sqrt(grad_total(sumsq, nparts));
    const bool finite = isfinite(norm);
    if (t0 == 0) {
        if (gnorm_out) gnorm_out[0] = static_cast<float>(norm);
        if (applied_out) applied_out[0] = finite ? 1 : 0;
    }
    if (!finite) return;   // lmtrain.lua:1214-1218: skip the step
    const float clipf = (clip_norm > 0.f && norm > clip_norm) ? static_cast<float>(clip_norm / norm) : 1.0f;
    for (long long i = t0; i < n4; i += stride) {
        if (i != t0) {
            gv = g4[i];
            pv = p4[i];
            if (momentum > 0.f) vv = v4[i];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float pk = ld_lane(pv, k), gk = ld_lane(gv, k), vk = ld_lane(vv, k);
            sgd_elem(pk, gk, vk, hy, clipf);
            st_lane(pv, k, pk); st_lane(gv, k, gk); st_lane(vv, k, vk);
        }
        // streamed out: v is read again by the next step's update, g is
        // overwritten by the next backward, p is read by every XCD
        __builtin_nontemporal_store(nt_f4{gv.x, gv.y, gv.z, gv.w}, reinterpret_cast<nt_f4*>(g4 + i));
        if (momentum > 0.f) __builtin_nontemporal_store(nt_f4{vv.x, vv.y, vv.z, vv.w}, reinterpret_cast<nt_f4*>(v4 + i));
        __builtin_nontemporal_store(nt_f4{pv.x, pv.y, pv.z, pv.w}, reinterpret_cast<nt_f4*>(p4 + i));
    }
    for (long long i = 4 * n4 + t0; i < n; i += stride) {
        float pk = p[i], gk = g[i], vk = momentum > 0.f ? v[i] : 0.f;
        sgd_elem(pk, gk, vk, hy, clipf);
        g[i] = gk;
        if (momentum > 0.f) v[i] = vk;
        p[i] = pk;
    }
}

// One AdamW step (optim2.lua:116-147) inside the same LMTrain step logic as
// sgd_step_kernel (scale, finite check, global-norm clip; g overwritten with
// the gradient used).  The step count t (bias corrections 1 - beta^t) is
// t_in when tcount is NULL; otherwise it lives on the device in two slots:
// the kernel reads tcount[parity] and block 0 writes the advanced count
// (advanced only when the step applies) to tcount[parity ^ 1], so no block
// can read a half-updated counter; the caller alternates parity per call.
// Device hyper-parameters (graph replay): {lr, -, wd, clip, -, beta1, beta2,
// eps, parity, grad_scale}.
__global__ void __launch_bounds__(256)
adamw_step_kernel(float* __restrict__ p, float* __restrict__ g, float* __restrict__ m, float* __restrict__ v,
                  long long n, const double* __restrict__ sumsq, int nparts, float lr, float beta1, float beta2,
                  float eps, float wd, float grad_scale, float clip_norm, int t_in, int* __restrict__ tcount,
                  int parity, float* __restrict__ gnorm_out, int* __restrict__ applied_out,
                  const float* __restrict__ hyper, int vec)
{
    if (hyper) {
        lr = hyper[0]; wd = hyper[2]; clip_norm = hyper[3];
        beta1 = hyper[5]; beta2 = hyper[6]; eps = hyper[7]; parity = hyper[8] != 0.f ? 1 : 0;
        grad_scale = hyper[9];
    }
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    // float4 lanes (vec: every buffer 16-byte aligned); the first float4 of
    // each operand is fetched before the norm is summed, so its loads overlap
    // that reduction
    const long long n4 = vec ? (n >> 2) : 0;
    float4* p4 = reinterpret_cast<float4*>(p);
    float4* g4 = reinterpret_cast<float4*>(g);
    float4* m4 = reinterpret_cast<float4*>(m);
    float4* v4 = reinterpret_cast<float4*>(v);
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 pv = z4, gv = z4, mv = z4, vv = z4;
    if (t0 < n4) {
        gv = g4[t0];
        mv = m4[t0];
        vv = v4[t0];
        pv = p4[t0];
    }
    const double norm = static_cast<double>(grad_scale) * sqrt(grad_total(sumsq, nparts));
    const bool finite = isfinite(norm);
    const int t_old = tcount ? tcount[parity] : t_in - 1;
    const int t = t_old + 1;
    if (t0 == 0) {
        if (gnorm_out) gnorm_out[0] = static_cast<float>(norm);
        if (applied_out) applied_out[0] = finite ? 1 : 0;
        if (tcount) tcount[parity ^ 1] = finite ? t : t_old;
    }
    if (!finite) return;
    const float clipf = (clip_norm > 0.f && norm > clip_norm) ? static_cast<float>(clip_norm / norm) : 1.0f;
    const double bc1 = 1.0 - pow(static_cast<double>(beta1), t);
    const double bc2 = 1.0 - pow(static_cast<double>(beta2), t);
    const float step_size = static_cast<float>(lr / bc1);
    const float inv_bc2 = static_cast<float>(1.0 / bc2);
    const float decay = wd != 0.f ? lr * wd : 0.f;
    const float c1 = 1.0f - beta1, c2 = 1.0f - beta2;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    auto elem = [&](float& pk, float& gk, float& mk, float& vk) {
        gk = gk * grad_scale;
        if (clipf != 1.0f) gk = gk * clipf;
        mk = beta1 * mk + c1 * gk;
        vk = beta2 * vk + c2 * gk * gk;
        const float denom = sqrtf(vk * inv_bc2) + eps;
        if (decay != 0.f) pk = pk - decay * pk;
        pk = pk - step_size * mk / denom;
    };
    for (long long i = t0; i < n4; i += stride) {
        if (i != t0) {
            gv = g4[i];
            mv = m4[i];
            vv = v4[i];
            pv = p4[i];
        }
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            float pk = ld_lane(pv, k), gk = ld_lane(gv, k), mk = ld_lane(mv, k), vk = ld_lane(vv, k);
            elem(pk, gk, mk, vk);
            st_lane(pv, k, pk); st_lane(gv, k, gk); st_lane(mv, k, mk); st_lane(vv, k, vk);
        }
        // streamed out: the moments are read again by the next step's
        // update, the gradient is overwritten by the next backward
        __builtin_nontemporal_store(nt_f4{gv.x, gv.y, gv.z, gv.w}, reinterpret_cast<nt_f4*>(g4 + i));
        __builtin_nontemporal_store(nt_f4{mv.x, mv.y, mv.z, mv.w}, reinterpret_cast<nt_f4*>(m4 + i));
        __builtin_nontemporal_store(nt_f4{vv.x, vv.y, vv.z, vv.w}, reinterpret_cast<nt_f4*>(v4 + i));
        __builtin_nontemporal_store(nt_f4{pv.x, pv.y, pv.z, pv.w}, reinterpret_cast<nt_f4*>(p4 + i));
    }
    for (long long i = 4 * n4 + t0; i < n; i += stride) {
        float pk = p[i], gk = g[i], mk = m[i], vk = v[i];
        elem(pk, gk, mk, vk);
        g[i] = gk;
        m[i] = mk;
        v[i] = vk;
        p[i] = pk;
    }
}

// out[0] = scale * sum(x[0..n)) (float result from a double accumulation; single block)
__global__ void __launch_bounds__(256) sum_f32_kernel(const float* __restrict__ x, int n, float scale, float* __restrict__ out)
{
    __shared__ double red[4];
    double s = 0.0;
    for (int i = threadIdx.x; i < n; i += 256) s += x[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) out[0] = static_cast<float>((red[0] + red[1] + red[2] + red[3]) * scale);
}

}  // namespace

int sumsq_blocks(long long n)
{
    // 16 values per thread: few partials, so the SGD kernel's blocks can each
    // finish the reduction themselves
    long long b = (n + 16LL * kRedThreads - 1) / (16LL * kRedThreads);
    if (b > kRedMaxBlocks) b = kRedMaxBlocks;
    return static_cast<int>(b < 1 ? 1 : b);
}

int sumsq(const float* x, long long n, double* out, double* partial, int partial_len, hipStream_t s)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "sumsq: n < 0");
    if (!out) return fail(LHIP_E_NULL, "sumsq: out is NULL");
    if (n > 0 && !x) return fail(LHIP_E_NULL, "sumsq: x is NULL");
    const int nb = sumsq_blocks(n);
    if (nb > partial_len) return fail(LHIP_E_CAPACITY, "sumsq: workspace %d < %d blocks", partial_len, nb);
    klaunch(sumsq_stage1, nb, kRedThreads, 0, s, x, n, partial, aligned16(x) ? 1 : 0);
    klaunch(sum_stage2, 1, 64, 0, s, partial, nb, out);
    return check_launch("sumsq");
}

int sumsq_partials(const float* x, long long n, double* partial, int partial_len, hipStream_t s)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "sumsq: n < 0");
    if (n > 0 && !x) return fail(LHIP_E_NULL, "sumsq: x is NULL");
    const int nb = sumsq_blocks(n);
    if (nb > partial_len) return fail(LHIP_E_CAPACITY, "sumsq: workspace %d < %d blocks", partial_len, nb);
    klaunch(sumsq_stage1, nb, kRedThreads, 0, s, x, n, partial, aligned16(x) ? 1 : 0);
    return check_launch("sumsq");
}

int sgd_step(float* p, float* g, float* v, long long n, const double* sumsq_dev, float lr, float momentum,
             float wd, float grad_scale, float clip_norm, int nesterov, float* gnorm_out, int* applied_out,
             hipStream_t s, const float* hyper_dev, int nparts)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "sgd_step: n < 0");
    if (!sumsq_dev) return fail(LHIP_E_NULL, "sgd_step: sumsq is NULL");
    if (n > 0 && (!p || !g)) return fail(LHIP_E_NULL, "sgd_step: NULL params/grads");
    if ((momentum > 0.f || hyper_dev) && n > 0 && !v)
        return fail(LHIP_E_NULL, "sgd_step: momentum > 0 needs a velocity buffer");
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    long long blocks = (n + 255) / 256;
    if (blocks > 4LL * cus) blocks = 4LL * cus;
    const int vec = (aligned16(p) && aligned16(g) && (!v || aligned16(v))) ? 1 : 0;
    if (vec) blocks = std::min<long long>((n / 4 + 255) / 256, 4LL * cus);
    if (blocks < 1) blocks = 1;
    klaunch(sgd_step_kernel, static_cast<int>(blocks), 256, 0, s, p, g, v, n, sumsq_dev, nparts, lr, momentum, wd,
                                                           grad_scale, clip_norm, nesterov, gnorm_out, applied_out,
                                                           hyper_dev, vec);
    return check_launch("sgd_step");
}

int adamw_step(float* p, float* g, float* m, float* v, long long n, const double* sumsq_dev, int nparts, float lr,
               float beta1, float beta2, float eps, float wd, float grad_scale, float clip_norm, int t_in,
               int* tcount, int parity, float* gnorm_out, int* applied_out, hipStream_t s, const float* hyper_dev)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "adamw_step: n < 0");
    if (!sumsq_dev) return fail(LHIP_E_NULL, "adamw_step: sumsq is NULL");
    if (n > 0 && (!p || !g || !m || !v)) return fail(LHIP_E_NULL, "adamw_step: NULL params/grads/moments");
    if (!tcount && t_in < 1) return fail(LHIP_E_ARG, "adamw_step: step %d must be >= 1", t_in);
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    long long blocks = (n + 255) / 256;
    if (blocks > 4LL * cus) blocks = 4LL * cus;
    const int vec = (aligned16(p) && aligned16(g) && aligned16(m) && aligned16(v)) ? 1 : 0;
    if (vec) blocks = std::min<long long>((n / 4 + 255) / 256, 4LL * cus);
    if (blocks < 1) blocks = 1;
    klaunch(adamw_step_kernel, static_cast<int>(blocks), 256, 0, s, p, g, m, v, n, sumsq_dev, nparts, lr, beta1, beta2,
                                                             eps, wd, grad_scale, clip_norm, t_in, tcount, parity,
                                                             gnorm_out, applied_out, hyper_dev, vec);
    return check_launch("adamw_step");
}

int sum_f32(const float* x, int n, float scale, float* out, hipStream_t s)
{
    if (n < 0) return fail(LHIP_E_SHAPE, "sum_f32: n < 0");
    if (!out || (n > 0 && !x)) return fail(LHIP_E_NULL, "sum_f32: NULL pointer");
    klaunch(sum_f32_kernel, 1, 256, 0, s, x, n, scale, out);
    return check_launch("sum_f32");
}

}  // namespace lhip

using lhip::st;

extern "C" {

LHIP_API int lhip_sumsq(const float* x, long long n, double* out)
{
    LHIP_REQUIRE_READY();
    double* partial = nullptr;
    const int nb = lhip::sumsq_blocks(n);
    int rc = lhip::workspace(static_cast<size_t>(nb) * sizeof(double), reinterpret_cast<void**>(&partial));
    if (rc != LHIP_OK) return rc;
    return lhip::sumsq(x, n, out, partial, nb, st().stream);
}

LHIP_API int lhip_sgd_step(float* params, float* grads, float* velocity, long long n, const double* grad_sumsq,
                           float lr, float momentum, float weight_decay, float grad_scale, float clip_norm,
                           int nesterov, float* grad_norm_out, int* applied_out)
{
    LHIP_REQUIRE_READY();
    return lhip::sgd_step(params, grads, velocity, n, grad_sumsq, lr, momentum, weight_decay, grad_scale, clip_norm,
                          nesterov, grad_norm_out, applied_out, st().stream, nullptr);
}

LHIP_API int lhip_adamw_step(float* params, float* grads, float* m, float* v, long long n, const double* grad_sumsq,
                             float lr, float beta1, float beta2, float eps, float weight_decay, float grad_scale,
                             float clip_norm, int step, float* grad_norm_out, int* applied_out)
{
    LHIP_REQUIRE_READY();
    if (!(lr >= 0.f) || !(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f) || !(eps >= 0.f) ||
        !(weight_decay >= 0.f) || !(clip_norm >= 0.f))
        return lhip::fail(LHIP_E_ARG, "lhip_adamw_step: lr, eps, weight_decay, clip_norm >= 0 and betas in [0, 1)");
    return lhip::adamw_step(params, grads, m, v, n, grad_sumsq, 0, lr, beta1, beta2, eps, weight_decay, grad_scale,
                            clip_norm, step, nullptr, 0, grad_norm_out, applied_out, st().stream, nullptr);
}

LHIP_API int lhip_sum(const float* x, int n, float scale, float* out)
{
    LHIP_REQUIRE_READY();
    return lhip::sum_f32(x, n, scale, out, st().stream);
}

}  // extern "C"
