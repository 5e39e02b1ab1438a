// lhip_luatl.hip -- the luaTL operation set behind the reference adapter's resident
// API and its Program op list.
//
// The reference adapter (ai/gpu/luatl_adapter.lua:126-187) and luaTL.Program
// (ai/gpu/luaTL_train.lua:365-606) call a fixed set of luaTL operations whose
// semantics live in cuda/luaTL_core.cu and cuda/luaTL_train.cu.  This file
// gives each one a C entry point with the same meaning, built from this
// library's own kernels where one exists (the GEMM family, the row kernels)
// and from small HBM-streaming kernels here otherwise:
//   gemm_ex          strided/batched GEMM with the RMSNorm / activation
//                    prologue, bias, activation and beta epilogue
//                    (luaTL_train.cu:127-234, 391-476)
//   elementwise      the 23 luaTL_ew operators (luaTL_core.cu:49-72, 909-950)
//   rmsnorm_ex       forward with an optional gain, no 1/rms output
//                    (luaTL_core.cu:1092-1114)
//   rmsnorm_bwd_ex   backward from x and eps, dgamma accumulated
//                    (luaTL_train.cu:489-526)
//   softmax_ex       scale, additive bias, group-causal mask with offset
//                    (luaTL_train.cu:545-585), and its backward (:589-619)
//   row_rms, reduce_cols, l2_accum, clip_by_nsq, sum_accum, transpose,
//   bcast_add, adamw_elementwise, swiglu_bwd_ex (luaTL_train.cu:895-979,
//   1031-1050; luaTL_core.cu:1018-1060, 1346-1380; luaTL_train.cu:666-686)
// Every reduction here sums in a fixed order (no atomics), so results are
// deterministic where the reference's atomicAdd forms are not.
#include <algorithm>
#include <cmath>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

constexpr int kThreads = 256;

inline int grid_for(long long units, int threads)
{
    const long long cap = 1LL << 22;
    long long g = (units + threads - 1) / threads;
    if (g > cap) g = cap;
    return static_cast<int>(g < 1 ? 1 : g);
}

// ---------------------------------------------------------------- activations
// Sigmoid by sign, so neither branch overflows.
__device__ __forceinline__ float sigmoidf_(float v)
{
    if (v >= 0.f) return 1.0f / (1.0f + expf(-v));
    const float z = expf(v);
    return z / (1.0f + z);
}

__device__ __forceinline__ float siluf_(float v) { return v * sigmoidf_(v); }

__device__ __forceinline__ float silu_grad_(float v)
{
    const float s = sigmoidf_(v);
    return s * (1.0f + v * (1.0f - s));
}

// GELU in its tanh form (Hendrycks and Gimpel, 2016):
// 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), and that expression's
// derivative -- the form luaTL uses (luaTL_core.cu:370-383).
constexpr float kSqrt2OverPi = 0.7978845608028654f;
constexpr float kGeluCubic = 0.044715f;

__device__ __forceinline__ float geluf_(float x)
{
    const float t = kSqrt2OverPi * (x + kGeluCubic * x * x * x);
    return 0.5f * x * (1.0f + tanhf(t));
}

__device__ __forceinline__ float gelu_grad_(float x)
{
    const float t = kSqrt2OverPi * (x + kGeluCubic * x * x * x);
    const float th = tanhf(t);
    const float dt = kSqrt2OverPi * (1.0f + 3.0f * kGeluCubic * x * x);
    return 0.5f * (1.0f + th) + 0.5f * x * (1.0f - th * th) * dt;
}

// post-GEMM activation (LHIP_ACT_*) and pre-GEMM elementwise map (LHIP_PRE_*)
__device__ __forceinline__ float apply_act(int act, float v)
{
    switch (act) {
    case 1: return fmaxf(v, 0.f);
    case 2: return geluf_(v);
    case 3: return siluf_(v);
    case 4: return tanhf(v);
    case 5: return sigmoidf_(v);
    default: return v;
    }
}

__device__ __forceinline__ float apply_pre(int pre, float v)
{
    switch (pre) {
    case 2: return geluf_(v);
    case 3: return siluf_(v);
    case 4: return fmaxf(v, 0.f);
    default: return v;
    }
}

// ---------------------------------------------------------------- elementwise
// The luaTL_ew operator table (luaTL_core.cu:49-72, 909-934); a missing
// operand reads as 0.
template <int OP>
__device__ __forceinline__ float ew(float a, float b, float alpha, float beta)
{
    if constexpr (OP == 0) return a;
    else if constexpr (OP == 1) return alpha * a + beta * b;
    else if constexpr (OP == 2) return alpha * a - beta * b;
    else if constexpr (OP == 3) return alpha * a * b;
    else if constexpr (OP == 4) return alpha * a / (b + 1e-20f);
    else if constexpr (OP == 5) return alpha * a + beta;
    else if constexpr (OP == 6) return alpha * a + b;
    else if constexpr (OP == 7) return alpha;
    else if constexpr (OP == 8) return fmaxf(a, 0.f);
    else if constexpr (OP == 9) return geluf_(a);
    else if constexpr (OP == 10) return siluf_(a);
    else if constexpr (OP == 11) return tanhf(a);
    else if constexpr (OP == 12) return sigmoidf_(a);
    else if constexpr (OP == 13) return expf(a);
    else if constexpr (OP == 14) return sqrtf(fmaxf(a, 0.f));
    else if constexpr (OP == 15) return 1.0f / sqrtf(fmaxf(a, 1e-20f));
    else if constexpr (OP == 16) return -a;
    else if constexpr (OP == 17) return 1.0f / (a + 1e-20f);
    else if constexpr (OP == 18) return fabsf(a);
    else if constexpr (OP == 19) return fminf(fmaxf(a, alpha), beta);
    else if constexpr (OP == 20) return a > 0.f ? b : 0.f;
    else if constexpr (OP == 21) return b * silu_grad_(a);
    else return b * gelu_grad_(a);
}

template <int OP>
__global__ void __launch_bounds__(kThreads)
ew_kernel(const float* a, const float* b, float* c, long long n, float alpha, float beta, int vec)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const long long t0 = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x;
    long long done = 0;
    if (vec) {
        const long long n4 = n >> 2;
        for (long long i = t0; i < n4; i += stride) {
            float4 av = a ? reinterpret_cast<const float4*>(a)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 bv = b ? reinterpret_cast<const float4*>(b)[i] : make_float4(0.f, 0.f, 0.f, 0.f);
            float4 r;
            r.x = ew<OP>(av.x, bv.x, alpha, beta);
            r.y = ew<OP>(av.y, bv.y, alpha, beta);
            r.z = ew<OP>(av.z, bv.z, alpha, beta);
            r.w = ew<OP>(av.w, bv.w, alpha, beta);
            reinterpret_cast<float4*>(c)[i] = r;
        }
        done = 4 * n4;
    }
    for (long long i = done + t0; i < n; i += stride)
        c[i] = ew<OP>(a ? a[i] : 0.f, b ? b[i] : 0.f, alpha, beta);
}

template <int OP>
void launch_ew(const float* a, const float* b, float* c, long long n, float alpha, float beta, hipStream_t s)
{
    const int vec = (!a || aligned16(a)) && (!b || aligned16(b)) && aligned16(c);
    klaunch(ew_kernel<OP>, grid_for(vec ? (n + 3) / 4 : n, kThreads), kThreads, 0, s, a, b, c, n, alpha, beta, vec);
}

// ------------------------------------------------------------ strided rows
// 1/sqrt(mean_k x[r, k]^2 + eps) of `rows` rows of `cols` elements at
// (row stride rs, column stride cs); one wave per row, summed in lane order.
__global__ void __launch_bounds__(kThreads)
row_rms_kernel(const float* __restrict__ x, float* __restrict__ out, int rows, int cols, long long rs,
               long long cs, float eps, int vec)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const float* xr = x + row * rs;
    float acc = 0.f;
    if (vec) {   // unit column stride, 16-byte aligned rows, cols % 4 == 0
        const float4* x4 = reinterpret_cast<const float4*>(xr);
        for (int i = lane; i < cols / 4; i += 64) {
            const float4 v = x4[i];
            acc = fmaf(v.x, v.x, acc);
            acc = fmaf(v.y, v.y, acc);
            acc = fmaf(v.z, v.z, acc);
            acc = fmaf(v.w, v.w, acc);
        }
    } else {
        for (int i = lane; i < cols; i += 64) {
            const float v = xr[i * cs];
            acc = fmaf(v, v, acc);
        }
    }
    acc = wave_sum(acc);
    if (lane == 0) out[row] = 1.0f / sqrtf(acc / static_cast<float>(cols) + eps);
}

// The luaTL GEMM prologue, materialised: out (rows x K, row-major, per batch
// rows*K apart) = op(A) rows with either x * rowscale[r] * gamma[k] (pre 1,
// rowscale computed from op(A)'s row when NULL) or an elementwise map (pre
// 2-4).  One wave per row.
__global__ void __launch_bounds__(kThreads)
gemm_pre_kernel(const float* __restrict__ A, long long a_rs, long long a_cs, long long a_bs,
                const float* __restrict__ gamma, const float* __restrict__ rowscale, float* __restrict__ out,
                int M, int K, int batch, float eps, int pre)
{
    const int lane = threadIdx.x & 63;
    const long long wrow = static_cast<long long>(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
    if (wrow >= static_cast<long long>(M) * batch) return;
    const int bz = static_cast<int>(wrow / M);
    const int r = static_cast<int>(wrow - static_cast<long long>(bz) * M);
    const float* ar = A + bz * a_bs + r * a_rs;
    float* orow = out + wrow * K;
    float sc = 1.f;
    if (pre == 1) {
        if (rowscale) {
            sc = rowscale[r];
        } else {
            float acc = 0.f;
            for (int k = lane; k < K; k += 64) {
                const float v = ar[k * a_cs];
                acc = fmaf(v, v, acc);
            }
            acc = wave_sum(acc);
            sc = 1.0f / sqrtf(acc / static_cast<float>(K) + eps);
        }
    }
    for (int k = lane; k < K; k += 64) {
        const float v = ar[k * a_cs];
        orow[k] = pre == 1 ? v * sc * (gamma ? gamma[k] : 1.f) : apply_pre(pre, v);
    }
}

// The luaTL GEMM epilogue: C = act(T + bias[col]) + beta * C, T = alpha*op(A)op(B)
// (row-major, rows x N per batch); beta == 0 never reads C.
__global__ void __launch_bounds__(kThreads)
gemm_post_kernel(const float* __restrict__ T, const float* __restrict__ bias, float* C, long long c_rs,
                 long long c_cs, long long c_bs, int M, int N, int batch, float beta, int act)
{
    const long long total = static_cast<long long>(M) * N * batch;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < total; i += stride) {
        const long long mn = static_cast<long long>(M) * N;
        const int bz = static_cast<int>(i / mn);
        const long long rem = i - bz * mn;
        const int r = static_cast<int>(rem / N);
        const int c = static_cast<int>(rem - static_cast<long long>(r) * N);
        float v = T[i];
        if (bias) v += bias[c];
        v = apply_act(act, v);
        float* cp = C + bz * c_bs + r * c_rs + c * c_cs;
        if (beta != 0.f) v += beta * *cp;
        *cp = v;
    }
}

// ------------------------------------------------------------ softmax (luaTL)
// Row `row` keeps columns i <= limit, limit = (group > 0 ? row % group : row)
// + mask_offset when causal, else cols - 1; v = x * scale + bias[i]; masked
// entries are 0 and a row with nothing kept is all 0 (luaTL_train.cu:545-585).
// The general form (additive bias, or an offset that can mask whole rows);
// the common cases go to the register-resident row kernels.
__global__ void __launch_bounds__(kThreads)
softmax_ex_kernel(const float* __restrict__ x, const float* __restrict__ bias, float* __restrict__ y, int rows,
                  int cols, float scale, int causal, int group, int moff)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lrow = group > 0 ? row % group : row;
    const int limit = causal ? lrow + moff : cols - 1;
    const float* xr = x + static_cast<long long>(row) * cols;
    float* yr = y + static_cast<long long>(row) * cols;
    float mx = -INFINITY;
    for (int i = lane; i < cols && i <= limit; i += 64) {
        float v = xr[i] * scale;
        if (bias) v += bias[i];
        mx = fmaxf(mx, v);
    }
    mx = wave_max(mx);
    const float base = mx == -INFINITY ? 0.f : mx;
    float sum = 0.f;
    for (int i = lane; i < cols; i += 64) {
        float e = 0.f;
        if (i <= limit) {
            float v = xr[i] * scale;
            if (bias) v += bias[i];
            e = expf(v - base);
        }
        yr[i] = e;
        sum += e;
    }
    sum = wave_sum(sum);
    const float inv = sum > 0.f ? 1.0f / sum : 0.f;
    for (int i = lane; i < cols; i += 64) yr[i] *= inv;
}

// dx = scale * y * (dy - sum_{i <= limit} dy_i y_i) on the kept columns, 0
// beyond (luaTL_train.cu:589-619), for offsets that mask whole rows.
__global__ void __launch_bounds__(kThreads)
softmax_bwd_ex_kernel(const float* __restrict__ y, const float* __restrict__ dy, float* __restrict__ dx, int rows,
                      int cols, float scale, int causal, int group, int moff)
{
    const int lane = threadIdx.x & 63;
    const int row = blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (row >= rows) return;
    const int lrow = group > 0 ? row % group : row;
    const int limit = causal ? lrow + moff : cols - 1;
    const long long o = static_cast<long long>(row) * cols;
    float dot = 0.f;
    for (int i = lane; i < cols && i <= limit; i += 64) dot += dy[o + i] * y[o + i];
    dot = wave_sum(dot);
    for (int i = lane; i < cols; i += 64) dx[o + i] = i <= limit ? scale * y[o + i] * (dy[o + i] - dot) : 0.f;
}

// ------------------------------------------------------------- reductions
// out[c] = alpha * sum_r x[r*rs + c] + beta * out[c]: 64 columns per block,
// four row phases each summing their rows in order, combined in phase order.
__global__ void __launch_bounds__(kThreads)
reduce_cols_kernel(const float* __restrict__ x, float* out, int rows, int cols, long long rs, float alpha,
                   float beta)
{
    __shared__ float part[4][64];
    const int cl = threadIdx.x & 63, ph = threadIdx.x >> 6;
    const int c = blockIdx.x * 64 + cl;
    float acc = 0.f;
    if (c < cols)
        for (int r = ph; r < rows; r += 4) acc += x[r * rs + c];
    part[ph][cl] = acc;
    __syncthreads();
    if (ph == 0 && c < cols) {
        const float s = ((part[0][cl] + part[1][cl]) + part[2][cl]) + part[3][cl];
        out[c] = beta != 0.f ? alpha * s + beta * out[c] : alpha * s;
    }
}

// *acc += (float) sum of the partials, summed in order in double (one wave)
__global__ void l2_finish_kernel(const double* __restrict__ partial, int np, float* acc)
{
    const int lane = threadIdx.x;
    double s = 0.0;
    for (int i = lane; i < np; i += 64) s += partial[i];
    for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
    if (lane == 0) acc[0] += static_cast<float>(s);
}

// x *= f, f = max_norm / (sqrt(nsq) + 1e-6) when sqrt(nsq) > max_norm > 0
// (luaTL_train.cu:947-965); nothing is written when f == 1.
__global__ void __launch_bounds__(kThreads)
clip_kernel(float* x, long long n, const float* __restrict__ nsq, float max_norm)
{
    const float nrm = sqrtf(fmaxf(nsq[0], 0.f));
    float f = 1.f;
    if (max_norm > 0.f && nrm > max_norm) f = max_norm / (nrm + 1e-6f);
    if (f == 1.f) return;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride) x[i] *= f;
}

// *acc += scale * sum(x): one workgroup, threads summing strided slices in
// order, then the four waves' sums in wave order
__global__ void __launch_bounds__(kThreads)
sum_accum_kernel(const float* __restrict__ x, long long n, float scale, float* acc)
{
    __shared__ float ws[kThreads / 64];
    float s = 0.f;
    for (long long i = threadIdx.x; i < n; i += kThreads) s += x[i];
    s = wave_sum(s);
    if ((threadIdx.x & 63) == 0) ws[threadIdx.x >> 6] = s;
    __syncthreads();
    if (threadIdx.x == 0) acc[0] += scale * (((ws[0] + ws[1]) + ws[2]) + ws[3]);
}

// out (cols x rows) = x (rows x cols)^T through a 64 x 65 LDS tile
__global__ void __launch_bounds__(kThreads)
transpose_kernel(const float* __restrict__ x, float* __restrict__ out, int rows, int cols)
{
    __shared__ float tile[64][65];
    const int c0 = blockIdx.x * 64, r0 = blockIdx.y * 64;
    const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
    for (int j = ty; j < 64; j += 4) {
        const int r = r0 + j, c = c0 + tx;
        tile[j][tx] = (r < rows && c < cols) ? x[static_cast<long long>(r) * cols + c] : 0.f;
    }
    __syncthreads();
    for (int j = ty; j < 64; j += 4) {
        const int c = c0 + j, r = r0 + tx;
        if (c < cols && r < rows) out[static_cast<long long>(c) * rows + r] = tile[tx][j];
    }
}

// out[r, c] = x[r, c] + alpha * v[c] (v NULL reads as 0)
__global__ void __launch_bounds__(kThreads)
bcast_add_kernel(const float* __restrict__ x, const float* __restrict__ v, float* out, int rows, int cols,
                 float alpha)
{
    const long long n = static_cast<long long>(rows) * cols;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const int c = static_cast<int>(i % cols);
        out[i] = x[i] + alpha * (v ? v[c] : 0.f);
    }
}

// luaTL's AdamW (luaTL_core.cu:1346-1380): per-element gradient clamp to
// [-clip, clip] when clip > 0, moments, bias-corrected step with the
// corrections bc1 = 1/(1-beta1^t), bc2 = 1/(1-beta2^t) given, decoupled decay
// applied first; w_mirror (may be NULL) receives a copy of the new weight.
__global__ void __launch_bounds__(kThreads)
adamw_ew_kernel(float* w, const float* __restrict__ g, float* m, float* v, float* w_mirror, long long n, float lr,
                float beta1, float beta2, float eps, float wd, float bc1, float bc2, float clip)
{
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        float gr = g[i];
        if (clip > 0.f) gr = fminf(fmaxf(gr, -clip), clip);
        const float mi = beta1 * m[i] + (1.f - beta1) * gr;
        const float vi = beta2 * v[i] + (1.f - beta2) * gr * gr;
        m[i] = mi;
        v[i] = vi;
        float wi = w[i];
        wi -= lr * wd * wi;
        wi -= lr * (mi * bc1) / (sqrtf(vi * bc2) + eps);
        w[i] = wi;
        if (w_mirror) w_mirror[i] = wi;
    }
}

// SwiGLU backward with either output optional: da = dout*b*silu'(a),
// db = dout*silu(a) (luaTL_train.cu:666-686); the outputs use the leading
// dimensions of their inputs
__global__ void __launch_bounds__(kThreads)
swiglu_bwd_one_kernel(const float* __restrict__ a, int lda, const float* __restrict__ b, int ldb,
                      const float* __restrict__ dout, int ldo, float* da, float* db, int rows, int cols)
{
    const long long n = static_cast<long long>(rows) * cols;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long i = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; i < n; i += stride) {
        const int r = static_cast<int>(i / cols);
        const int c = static_cast<int>(i - static_cast<long long>(r) * cols);
        const float av = a[static_cast<long long>(r) * lda + c];
        const float go = dout[static_cast<long long>(r) * ldo + c];
        if (da) da[static_cast<long long>(r) * lda + c] = go * b[static_cast<long long>(r) * ldb + c] * silu_grad_(av);
        if (db) db[static_cast<long long>(r) * ldb + c] = go * siluf_(av);
    }
}

int waves_grid(long long rows) { return static_cast<int>(std::max<long long>(1, (rows + 3) / 4)); }

// A logical R x S operand at (rs, cs) as a row-major (N-form) or stored-
// transposed (T-form) matrix with a leading dimension; false for strides
// neither form expresses.
bool classify(int R, int S, long long rs, long long cs, int* trans, int* ld)
{
    if ((cs == 1 || S == 1) && (R == 1 || rs >= S)) {
        *trans = 0;
        *ld = static_cast<int>(R == 1 ? S : rs);
        return R == 1 || rs <= 0x7fffffffLL;
    }
    if ((rs == 1 || R == 1) && (S == 1 || cs >= R)) {
        *trans = 1;
        *ld = static_cast<int>(S == 1 ? R : cs);
        return S == 1 || cs <= 0x7fffffffLL;
    }
    return false;
}

}  // namespace

int ones_vector(int n, const float** out)
{
    auto& s = st();
    if (n > kOnesMax) return fail(LHIP_E_CAPACITY, "gain-free row op: %d columns > %d", n, kOnesMax);
    if (!s.ones) return fail(LHIP_E_DEVICE, "gain-free row op: ones vector not initialised");
    *out = s.ones;
    return LHIP_OK;
}

}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

LHIP_API int lhip_elementwise(const float* a, const float* b, float* c, long long n, int op, float alpha, float beta)
{
    LHIP_REQUIRE_READY();
    if (n < 0) return fail(LHIP_E_SHAPE, "lhip_elementwise: n = %lld", n);
    if (op < 0 || op > 22) return fail(LHIP_E_ARG, "lhip_elementwise: unknown operator %d", op);
    if (n == 0) return LHIP_OK;
    if (!c) return fail(LHIP_E_NULL, "lhip_elementwise: c is NULL");
    hipStream_t s = st().stream;
    switch (op) {
#define LHIP_EW_CASE(k) case k: lhip::launch_ew<k>(a, b, c, n, alpha, beta, s); break;
        LHIP_EW_CASE(0) LHIP_EW_CASE(1) LHIP_EW_CASE(2) LHIP_EW_CASE(3) LHIP_EW_CASE(4) LHIP_EW_CASE(5)
        LHIP_EW_CASE(6) LHIP_EW_CASE(7) LHIP_EW_CASE(8) LHIP_EW_CASE(9) LHIP_EW_CASE(10) LHIP_EW_CASE(11)
        LHIP_EW_CASE(12) LHIP_EW_CASE(13) LHIP_EW_CASE(14) LHIP_EW_CASE(15) LHIP_EW_CASE(16) LHIP_EW_CASE(17)
        LHIP_EW_CASE(18) LHIP_EW_CASE(19) LHIP_EW_CASE(20) LHIP_EW_CASE(21) LHIP_EW_CASE(22)
#undef LHIP_EW_CASE
    }
    return lhip::check_launch("lhip_elementwise");
}

LHIP_API int lhip_row_rms(const float* x, float* out, int rows, int cols, long long rs, long long cs, float eps)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "lhip_row_rms: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !out) return fail(LHIP_E_NULL, "lhip_row_rms: NULL pointer");
    const int vec = cs == 1 && rs % 4 == 0 && cols % 4 == 0 && lhip::aligned16(x);
    lhip::klaunch(lhip::row_rms_kernel, lhip::waves_grid(rows), lhip::kThreads, 0, st().stream, x, out, rows, cols, rs, cs, eps,
                                                                                    vec);
    return lhip::check_launch("lhip_row_rms");
}

LHIP_API int lhip_rmsnorm_ex(const float* x, const float* w, float* y, int rows, int cols, float eps)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "lhip_rmsnorm_ex: rows=%d cols=%d", rows, cols);
    if (!w) {
        int rc = lhip::ones_vector(cols, &w);
        if (rc != LHIP_OK) return rc;
    }
    return lhip::rmsnorm_fwd(x, w, y, nullptr, rows, cols, eps, st().stream);
}

LHIP_API int lhip_rmsnorm_bwd_ex(const float* x, const float* w, const float* dy, float* dx, float* dw, int rows,
                                 int cols, float eps)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "lhip_rmsnorm_bwd_ex: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !dy || !dx) return fail(LHIP_E_NULL, "lhip_rmsnorm_bwd_ex: NULL x/dy/dx");
    if (!w) {
        int rc = lhip::ones_vector(cols, &w);
        if (rc != LHIP_OK) return rc;
    }
    const int parts = lhip::rmsnorm_bwd_parts(rows, cols);
    const size_t inv_floats = (static_cast<size_t>(rows) + 63) & ~static_cast<size_t>(63);
    const size_t part_floats = dw ? static_cast<size_t>(parts) * cols : 0;
    float* work = nullptr;
    int rc = lhip::workspace((inv_floats + part_floats) * sizeof(float), reinterpret_cast<void**>(&work));
    if (rc != LHIP_OK) return rc;
    hipStream_t s = st().stream;
    float* inv = work;
    lhip::klaunch(lhip::row_rms_kernel, lhip::waves_grid(rows), lhip::kThreads, 0, s, x, inv, rows, cols, cols, 1, eps,
                                                                          cols % 4 == 0 && lhip::aligned16(x));
    rc = lhip::check_launch("lhip_rmsnorm_bwd_ex: 1/rms");
    if (rc != LHIP_OK) return rc;
    int nparts = 0;
    rc = lhip::rmsnorm_bwd_rows(x, w, inv, dy, dx, nullptr, dw ? work + inv_floats : nullptr, part_floats, rows, cols,
                                &nparts, s);
    if (rc != LHIP_OK || !dw) return rc;
    // dgamma accumulates, as the reference's atomicAdd into it does
    return lhip::rmsnorm_bwd_colsum(work + inv_floats, nparts, dw, cols, 1, s);
}

LHIP_API int lhip_softmax_ex(const float* x, const float* bias, float* y, int rows, int cols, float scale, int causal,
                             int group, int mask_offset)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "lhip_softmax_ex: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!x || !y) return fail(LHIP_E_NULL, "lhip_softmax_ex: NULL x/y");
    // without a bias and with every row keeping at least its first column,
    // the register-resident row kernel has the same semantics
    if (!bias && (!causal || mask_offset >= 0))
        return lhip::softmax_fwd(x, y, rows, cols, scale, causal, mask_offset, group, st().stream);
    lhip::klaunch(lhip::softmax_ex_kernel, lhip::waves_grid(rows), lhip::kThreads, 0, st().stream, x, bias, y, rows, cols, scale,
                                                                                       causal, group, mask_offset);
    return lhip::check_launch("lhip_softmax_ex");
}

LHIP_API int lhip_softmax_bwd_ex(const float* y, const float* dy, float* dx, int rows, int cols, float scale,
                                 int causal, int group, int mask_offset)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols <= 0) return fail(LHIP_E_SHAPE, "lhip_softmax_bwd_ex: rows=%d cols=%d", rows, cols);
    if (rows == 0) return LHIP_OK;
    if (!y || !dy || !dx) return fail(LHIP_E_NULL, "lhip_softmax_bwd_ex: NULL y/dy/dx");
    if (!causal || mask_offset >= 0)
        return lhip::softmax_bwd(y, dy, dx, rows, cols, scale, causal, mask_offset, group, 0, st().stream);
    lhip::klaunch(lhip::softmax_bwd_ex_kernel, lhip::waves_grid(rows), lhip::kThreads, 0, st().stream, 
        y, dy, dx, rows, cols, scale, causal, group, mask_offset);
    return lhip::check_launch("lhip_softmax_bwd_ex");
}

LHIP_API int lhip_swiglu_bwd_ex(const float* a, const float* b, const float* dout, float* da, float* db, int rows,
                                int cols, int lda, int ldb, int ldo)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols < 0) return fail(LHIP_E_SHAPE, "lhip_swiglu_bwd_ex: rows=%d cols=%d", rows, cols);
    if (rows == 0 || cols == 0) return LHIP_OK;
    if (!a || !b || !dout) return fail(LHIP_E_NULL, "lhip_swiglu_bwd_ex: NULL a/b/dout");
    if (lda < cols || ldb < cols || ldo < cols) return fail(LHIP_E_SHAPE, "lhip_swiglu_bwd_ex: leading dimension < cols");
    if (da && db)
        return lhip::swiglu_bwd(a, lda, b, ldb, dout, ldo, da, lda, db, ldb, rows, cols, 0, st().stream);
    if (!da && !db) return LHIP_OK;
    const long long n = static_cast<long long>(rows) * cols;
    lhip::klaunch(lhip::swiglu_bwd_one_kernel, lhip::grid_for(n, lhip::kThreads), lhip::kThreads, 0, st().stream, 
        a, lda, b, ldb, dout, ldo, da, db, rows, cols);
    return lhip::check_launch("lhip_swiglu_bwd_ex");
}

LHIP_API int lhip_reduce_cols(const float* x, float* out, int rows, int cols, long long row_stride, float alpha,
                              float beta)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols < 0 || (rows > 0 && row_stride < cols))
        return fail(LHIP_E_SHAPE, "lhip_reduce_cols: rows=%d cols=%d row_stride=%lld", rows, cols, row_stride);
    if (cols == 0) return LHIP_OK;
    if (!out || (rows > 0 && !x)) return fail(LHIP_E_NULL, "lhip_reduce_cols: NULL pointer");
    lhip::klaunch(lhip::reduce_cols_kernel, lhip::ceil_div(cols, 64), lhip::kThreads, 0, st().stream, x, out, rows, cols,
                                                                                          row_stride, alpha, beta);
    return lhip::check_launch("lhip_reduce_cols");
}

LHIP_API int lhip_l2_accum(const float* x, long long n, float* acc)
{
    LHIP_REQUIRE_READY();
    if (n < 0) return fail(LHIP_E_SHAPE, "lhip_l2_accum: n < 0");
    if (n == 0) return LHIP_OK;
    if (!x || !acc) return fail(LHIP_E_NULL, "lhip_l2_accum: NULL pointer");
    const int nb = lhip::sumsq_blocks(n);
    double* partial = nullptr;
    int rc = lhip::workspace(static_cast<size_t>(nb) * sizeof(double), reinterpret_cast<void**>(&partial));
    if (rc != LHIP_OK) return rc;
    rc = lhip::sumsq_partials(x, n, partial, nb, st().stream);
    if (rc != LHIP_OK) return rc;
    lhip::klaunch(lhip::l2_finish_kernel, 1, 64, 0, st().stream, partial, nb, acc);
    return lhip::check_launch("lhip_l2_accum");
}

LHIP_API int lhip_clip_by_nsq(float* x, long long n, const float* nsq, float max_norm)
{
    LHIP_REQUIRE_READY();
    if (n < 0) return fail(LHIP_E_SHAPE, "lhip_clip_by_nsq: n < 0");
    if (n == 0) return LHIP_OK;
    if (!x || !nsq) return fail(LHIP_E_NULL, "lhip_clip_by_nsq: NULL pointer");
    lhip::klaunch(lhip::clip_kernel, lhip::grid_for(n, lhip::kThreads), lhip::kThreads, 0, st().stream, x, n, nsq, max_norm);
    return lhip::check_launch("lhip_clip_by_nsq");
}

LHIP_API int lhip_sum_accum(const float* x, long long n, float scale, float* acc)
{
    LHIP_REQUIRE_READY();
    if (n < 0) return fail(LHIP_E_SHAPE, "lhip_sum_accum: n < 0");
    if (!acc || (n > 0 && !x)) return fail(LHIP_E_NULL, "lhip_sum_accum: NULL pointer");
    if (n == 0) return LHIP_OK;
    lhip::klaunch(lhip::sum_accum_kernel, 1, lhip::kThreads, 0, st().stream, x, n, scale, acc);
    return lhip::check_launch("lhip_sum_accum");
}

LHIP_API int lhip_transpose(const float* x, float* out, int rows, int cols)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols < 0) return fail(LHIP_E_SHAPE, "lhip_transpose: rows=%d cols=%d", rows, cols);
    if (rows == 0 || cols == 0) return LHIP_OK;
    if (!x || !out) return fail(LHIP_E_NULL, "lhip_transpose: NULL pointer");
    if (x == out) return fail(LHIP_E_ARG, "lhip_transpose: in place is not supported");
    if (lhip::ceil_div(rows, 64) > 65535) return fail(LHIP_E_CAPACITY, "lhip_transpose: rows=%d", rows);
    const dim3 grid(lhip::ceil_div(cols, 64), lhip::ceil_div(rows, 64));
    lhip::klaunch(lhip::transpose_kernel, grid, lhip::kThreads, 0, st().stream, x, out, rows, cols);
    return lhip::check_launch("lhip_transpose");
}

LHIP_API int lhip_bcast_add(const float* x, const float* v, float* out, int rows, int cols, float alpha)
{
    LHIP_REQUIRE_READY();
    if (rows < 0 || cols < 0) return fail(LHIP_E_SHAPE, "lhip_bcast_add: rows=%d cols=%d", rows, cols);
    if (rows == 0 || cols == 0) return LHIP_OK;
    if (!x || !out) return fail(LHIP_E_NULL, "lhip_bcast_add: NULL pointer");
    const long long n = static_cast<long long>(rows) * cols;
    lhip::klaunch(lhip::bcast_add_kernel, lhip::grid_for(n, lhip::kThreads), lhip::kThreads, 0, st().stream, x, v, out, rows, cols,
                                                                                               alpha);
    return lhip::check_launch("lhip_bcast_add");
}

LHIP_API int lhip_adamw_elementwise(float* w, const float* g, float* m, float* v, float* w_mirror, long long n,
                                    int step, float lr, float beta1, float beta2, float eps, float weight_decay,
                                    float clip)
{
    LHIP_REQUIRE_READY();
    if (n < 0) return fail(LHIP_E_SHAPE, "lhip_adamw_elementwise: n < 0");
    if (n == 0) return LHIP_OK;
    if (!w || !g || !m || !v) return fail(LHIP_E_NULL, "lhip_adamw_elementwise: NULL w/g/m/v");
    if (!(beta1 >= 0.f && beta1 < 1.f) || !(beta2 >= 0.f && beta2 < 1.f))
        return fail(LHIP_E_ARG, "lhip_adamw_elementwise: betas must lie in [0, 1)");
    const int t = step < 1 ? 1 : step;
    const float bc1 = 1.0f / (1.0f - powf(beta1, static_cast<float>(t)));
    const float bc2 = 1.0f / (1.0f - powf(beta2, static_cast<float>(t)));
    lhip::klaunch(lhip::adamw_ew_kernel, lhip::grid_for(n, lhip::kThreads), lhip::kThreads, 0, st().stream, 
        w, g, m, v, w_mirror, n, lr, beta1, beta2, eps, weight_decay, bc1, bc2, clip);
    return lhip::check_launch("lhip_adamw_elementwise");
}

LHIP_API int lhip_gemm_ex(const float* A, const float* B, float* C, const float* bias, const float* gamma,
                          const float* rowscale, int M, int N, int K, long long a_rs, long long a_cs, long long b_rs,
                          long long b_cs, long long c_rs, long long c_cs, long long a_bs, long long b_bs,
                          long long c_bs, int batch, float alpha, float beta, float eps, int pre_op, int post_op)
{
    LHIP_REQUIRE_READY();
    if (M <= 0 || N <= 0 || K <= 0) return fail(LHIP_E_SHAPE, "lhip_gemm_ex: M=%d N=%d K=%d", M, N, K);
    if (batch < 1) batch = 1;
    if (batch > 65535) return fail(LHIP_E_CAPACITY, "lhip_gemm_ex: batch %d > 65535", batch);
    if (!A || !B || !C) return fail(LHIP_E_NULL, "lhip_gemm_ex: NULL A/B/C");
    if (pre_op < 0 || pre_op > 4) return fail(LHIP_E_ARG, "lhip_gemm_ex: unknown pre_op %d", pre_op);
    if (post_op < 0 || post_op > 5) return fail(LHIP_E_ARG, "lhip_gemm_ex: unknown post_op %d", post_op);
    if (batch > 1 && (a_bs < 0 || b_bs < 0 || c_bs < 0)) return fail(LHIP_E_SHAPE, "lhip_gemm_ex: negative batch stride");
    hipStream_t s = st().stream;
    const bool pre = pre_op != 0;
    const bool post = bias != nullptr || post_op != 0;
    int ta = 0, lda = K, tb = 0, ldb = N;
    if (!pre && !lhip::classify(M, K, a_rs, a_cs, &ta, &lda))
        return fail(LHIP_E_UNSUPPORTED, "lhip_gemm_ex: A strides (%lld, %lld) are neither row- nor column-major",
                    a_rs, a_cs);
    if (!lhip::classify(K, N, b_rs, b_cs, &tb, &ldb))
        return fail(LHIP_E_UNSUPPORTED, "lhip_gemm_ex: B strides (%lld, %lld) are neither row- nor column-major",
                    b_rs, b_cs);
    int tc = 0, ldc = N;
    if (!post && !lhip::classify(M, N, c_rs, c_cs, &tc, &ldc))
        return fail(LHIP_E_UNSUPPORTED, "lhip_gemm_ex: C strides (%lld, %lld) are neither row- nor column-major",
                    c_rs, c_cs);
    // the product that runs: row-major output, or C^T = op(B)^T op(A)^T when C
    // is stored column-major
    int gm = M, gn = N, gta = ta, gtb = tb;
    const size_t pre_floats = pre ? static_cast<size_t>(M) * K * batch : 0;
    const size_t post_floats = post ? static_cast<size_t>(M) * N * batch : 0;
    const size_t head = ((pre_floats + 63) & ~static_cast<size_t>(63)) + ((post_floats + 63) & ~static_cast<size_t>(63));
    if (!post && tc) { gm = N; gn = M; gta = !tb; gtb = pre ? 1 : !ta; }
    size_t split_need = 0;
    lhip::immediate_plan(gta, gtb, gm, gn, K, batch, &split_need);
    float* work = nullptr;
    if (head + split_need > 0) {
        int rc = lhip::workspace((head + split_need) * sizeof(float), reinterpret_cast<void**>(&work));
        if (rc != LHIP_OK) return rc;
    }
    const float* a_use = A;
    long long sa = a_bs;
    if (pre) {
        float* ap = work;
        lhip::klaunch(lhip::gemm_pre_kernel, lhip::waves_grid(static_cast<long long>(M) * batch), lhip::kThreads, 0, s, 
            A, a_rs, a_cs, a_bs, gamma, rowscale, ap, M, K, batch, eps, pre_op);
        int rc = lhip::check_launch("lhip_gemm_ex: prologue");
        if (rc != LHIP_OK) return rc;
        a_use = ap;
        ta = 0;
        lda = K;
        sa = static_cast<long long>(M) * K;
    }
    lhip::GemmOpts o;
    o.inner = batch;
    if (split_need > 0) {
        o.ws = work + head;
        o.ws_floats = split_need;
    }
    if (post) {
        float* T = work + ((pre_floats + 63) & ~static_cast<size_t>(63));
        int rc = lhip::sgemm_run(ta, tb, M, N, K, alpha, a_use, lda, sa, B, ldb, b_bs, 0.f, T, N,
                                 static_cast<long long>(M) * N, batch, o, s);
        if (rc != LHIP_OK) return rc;
        const long long total = static_cast<long long>(M) * N * batch;
        lhip::klaunch(lhip::gemm_post_kernel, lhip::grid_for(total, lhip::kThreads), lhip::kThreads, 0, s, 
            T, bias, C, c_rs, c_cs, c_bs, M, N, batch, beta, post_op);
        return lhip::check_launch("lhip_gemm_ex: epilogue");
    }
    if (tc) {
        // C^T (N x M, row-major with ldc) = op(B)^T . op(A)^T
        return lhip::sgemm_run(!tb, !ta, N, M, K, alpha, B, ldb, b_bs, a_use, lda, sa, beta, C, ldc, c_bs, batch, o, s);
    }
    return lhip::sgemm_run(ta, tb, M, N, K, alpha, a_use, lda, sa, B, ldb, b_bs, beta, C, ldc, c_bs, batch, o, s);
}

}  // extern "C"
