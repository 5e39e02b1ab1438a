// lhip_lmfuse.hip -- GEMMs of the LMTrain step with their neighbouring row and
// elementwise stages fused in, to cut the launches of a latency-bound step.
//
//   FUSE_NORM         C_y = rmsnorm(X; w) . B_y           (q, k, v projections)
//   FUSE_NORM_SWIGLU  Z = rmsnorm(X; w) . B, U = rmsnorm(X; w) . B2,
//                     A = silu(Z) * U                     (w1, w3 and the gate)
//   FUSE_SWIGLU_BWD   G = X . B^T, then dZ, dU = the SwiGLU backward of
//                     (Z, U) with upstream G               (f = a . w2 backward)
//
// With a gather table the A rows are embedding rows (A row r = table row
// ids[r], transformer.lua:228-231 with Tensor.embed), and the writer also
// stores them (x_0, the residual stream's start).
//
// RMSNorm (ai/core/tensor2.lua:609-634): out(r, k) = x(r, k) * inv(r) * w(k),
// inv(r) = 1 / sqrt(sum_k x(r, k)^2 / K + eps).  inv(r) does not depend on k,
// so it factors out of the product: C(r, n) = inv(r) * sum_k (x(r, k) w(k))
// B(k, n).  Each workgroup sums the squares of the A rows it loads anyway (it
// sees whole rows), applies w on load and inv in the epilogue; the workgroup
// of output column block 0 (batch entry 0) also writes the normalized rows h
// and inv, which the backward needs.  SwiGLU (tensor2.lua:272-303 with
// Tensor.mul :167-183) as in the stand-alone kernels: a = z * sigmoid(z) * u,
// dz = s (1 + z (1 - s)) (u g), du = (z s) g with the stable sigmoid by sign.
//
// Tiling: 16x16 output tiles, four waves each taking the 16-deep K steps
// w, w+4, ... of one pass (K <= 512), v_mfma_f32_16x16x4f32 with lane l
// holding op(A)[row][k0+4q .. +3] and op(B)[k0+4q .. +3][col] (q = l/16) and
// MFMA i multiplying element i; the four partial tiles are summed in LDS in
// wave order.  A is row-major; B is row-major K x N (NN) or, for
// FUSE_SWIGLU_BWD, N x K (NT).
#include <cmath>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kFuseU = 8;   // 16-deep K steps per wave: K <= 4 * 16 * kFuseU

struct FuseArgs {
    int M, N, K;
    const float* A; int lda;
    const float* B; int ldb; long long sB;   // batch entry y uses B + y*sB, C + y*sC
    float* C; int ldc; long long sC;
    int tiles_n;
    const float* nw; float eps; float* h; float* inv;   // norm gain; normalized rows (ld K) and inv out
    const float* B2; float* C2; float* Aout;             // FUSE_NORM_SWIGLU: W3, U, a (ld ldc)
    const float* Z; const float* U; float* dZ; float* dU; // SwiGLU backward epilogue (ld ldc)
    const float* nbx; const float* nbres; const float* nbinv; float* nbout; float* nbpart;  // norm-backward prologue
    int a_parts; long long a_pstride;   // A = sum of a_parts slices (split-K partials), summed in order
    const int* gather; int gather_rows; float* xout;   // gathered A rows (embedding), written to xout
};

__device__ __forceinline__ float sigmoid_sign(float v)
{
    if (v >= 0.f) return 1.0f / (1.0f + expf(-v));
    const float z = expf(v);
    return z / (1.0f + z);
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ void to4(float (&d)[4], float4 v) { d[0] = v.x; d[1] = v.y; d[2] = v.z; d[3] = v.w; }

template <int MODE>
__global__ void __launch_bounds__(256) lm_fused_gemm_kernel(const FuseArgs f)
{
    constexpr bool NORM = (MODE & FB_NORM) != 0;        // A := rmsnorm(A)
    constexpr bool DUAL = (MODE & FB_DUAL) != 0;        // second B, SwiGLU epilogue
    constexpr bool SWB = (MODE & FB_SWIGLU_BWD) != 0;   // SwiGLU-backward epilogue
    constexpr bool TB = (MODE & FB_TB) != 0;            // B is N x K
    constexpr bool NB = (MODE & FB_NORMBWD) != 0;       // A := dres + rmsnorm backward of (x, dy = A)
    constexpr int U = kFuseU;
    __shared__ float red[4][4][64];
    __shared__ float red2[DUAL ? 4 : 1][4][64];
    __shared__ float ssr[4][64];
    __shared__ float row_s[16];
    const int lane = threadIdx.x & 63, lr = lane & 15, q = lane >> 4;
    // wave-uniform (readfirstlane): the K-step bounds below are scalar branches
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, f.tiles_n, tm, tn);
    const int m0 = tm * 16, n0 = tn * 16;
    const int y = blockIdx.y;
    const int K = f.K;
    const float* __restrict__ B = f.B + y * f.sB;
    const int row = m0 + lr, col = n0 + lr;
    const bool rok = row < f.M, cok = col < f.N;
    // Rows past M and columns past N load from row / column 0 (valid
    // addresses): they reach only outputs that are not stored, and their row
    // statistics are masked below (inv, coef and r are 0 for them).
    const int rowc = rok ? row : 0, colc = cok ? col : 0;
    // the A row this lane loads: its own, or the table row its id names
    // (clamped into the table; ids are validated before the step)
    const int arow = f.gather ? min(max(f.gather[rowc], 0), f.gather_rows - 1) : rowc;
    const bool writer = y == 0 && tn == 0;   // writes the row-stage outputs (h/inv or dx/dw partials)

    // Every operand loads unconditionally: a lane past K (the last step, when
    // K % 16 != 0) reads the step start and its A element is zeroed after the
    // loads.  With no select or masked load on a loaded value, all of the
    // pass's loads issue before the first wait.
    float a[U][4], w[U][4], b[U][4], b2[DUAL ? U : 1][4], x[NB ? U : 1][4], rs[NB ? U : 1][4];
    float ss = 0.f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int ks = 16 * wave + 64 * u;          // wave-uniform step start
        if (ks >= K) break;
        const int k = ks + 4 * q;                   // K % 4 == 0: the four k are all in or all out
        const int kc = k < K ? k : ks;
        const long long ro = static_cast<long long>(rowc) * f.lda + kc;
        to4(a[u], ld4(f.A + static_cast<long long>(arow) * f.lda + kc));
        if constexpr (NORM || NB) to4(w[u], ld4(f.nw + kc));
        if constexpr (NB) {
            to4(x[u], ld4(f.nbx + ro));
            if (f.nbres) to4(rs[u], ld4(f.nbres + ro));
            else to4(rs[u], make_float4(0.f, 0.f, 0.f, 0.f));
        }
        if constexpr (TB) {
            to4(b[u], ld4(B + static_cast<long long>(colc) * f.ldb + kc));
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) b[u][i] = B[static_cast<long long>(kc + i) * f.ldb + colc];
        }
        if constexpr (DUAL) {
#pragma unroll
            for (int i = 0; i < 4; ++i) b2[u][i] = f.B2[static_cast<long long>(kc + i) * f.ldb + colc];
        }
    }
    // A = sum of a_parts slices (unreduced split-K of the producer), summed
    // in slice order; each slice's loads cover every step before its adds
    if (f.a_parts > 1) {
        for (int p = 1; p < f.a_parts; ++p) {
            float t[U][4];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int ks = 16 * wave + 64 * u;
                if (ks >= K) break;
                const int k = ks + 4 * q;
                const int kc = k < K ? k : ks;
                to4(t[u], ld4(f.A + p * f.a_pstride + static_cast<long long>(rowc) * f.lda + kc));
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (16 * wave + 64 * u >= K) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) a[u][i] += t[u][i];
            }
        }
    }
    if (K % 16 != 0) {   // the last step is partial: lanes past K contribute zero
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ks = 16 * wave + 64 * u;
            if (ks >= K) break;
            if (ks + 16 > K && ks + 4 * q >= K) {
#pragma unroll
                for (int i = 0; i < 4; ++i) a[u][i] = 0.f;
            }
        }
    }
    // Row statistic over the whole row (lanes l%16 = r of all q groups and
    // waves): sum x^2 (NORM) or sum dy w x (NB).
    if constexpr (NORM || NB) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (16 * wave + 64 * u >= K) break;   // dead steps hold no data
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (NORM) ss += a[u][i] * a[u][i];
                else ss += a[u][i] * w[u][i] * x[u][i];
            }
        }
        ssr[wave][lane] = ss;
        __syncthreads();
        if (threadIdx.x < 16) {
            float s = 0.f;
#pragma unroll
            for (int wv = 0; wv < 4; ++wv)
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) s += ssr[wv][16 * qq + threadIdx.x];
            if constexpr (NORM) {
                const float r = 1.0f / sqrtf(s / static_cast<float>(K) + f.eps);
                row_s[threadIdx.x] = r;
                if (writer && m0 + threadIdx.x < f.M) f.inv[m0 + threadIdx.x] = r;
            } else {
                // coef = dot * r^3 / K (tensor2.lua:641-666)
                const float r = (m0 + threadIdx.x < f.M) ? f.nbinv[m0 + threadIdx.x] : 0.f;
                row_s[threadIdx.x] = s * r * r * r * (1.0f / static_cast<float>(K));
            }
        }
        __syncthreads();
    }
    if constexpr (NB) {
        // dx = dy*w*r - x*coef (+ dres) in place of A; dw partials of this
        // 16-row tile (the 16 rows of one k sit in one DPP row)
        const float r = rok ? f.nbinv[row] : 0.f;
        const float coef = row_s[lr];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (16 * wave + 64 * u >= K) break;
            const int k = 16 * wave + 64 * u + 4 * q;
            float o[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float v = a[u][i] * w[u][i] * r - x[u][i] * coef;
                if (f.nbres) v = v + rs[u][i];
                o[i] = k < K ? v : 0.f;   // lanes past K read real x / dres: keep them out of the product
            }
            if (writer) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float pd = row16_sum(a[u][i] * x[u][i] * r);
                    if (lr == 0 && k < K) f.nbpart[static_cast<long long>(tm) * K + k + i] = pd;
                }
                if (rok && k < K)
                    *reinterpret_cast<float4*>(f.nbout + static_cast<long long>(row) * K + k) =
                        make_float4(o[0], o[1], o[2], o[3]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) a[u][i] = o[i];
        }
    }
    floatx4 acc = {0.f, 0.f, 0.f, 0.f}, acc2 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; ++u) {
        if (16 * wave + 64 * u >= K) break;   // wave-uniform
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float av = NORM ? a[u][i] * w[u][i] : a[u][i];
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[u][i], acc, 0, 0, 0);
            if constexpr (DUAL) acc2 = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b2[u][i], acc2, 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        red[wave][r][lane] = acc[r];
        if constexpr (DUAL) red2[wave][r][lane] = acc2[r];
    }
    if constexpr (NORM) {
        if (writer && rok) {
            const float r = row_s[lr];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (16 * wave + 64 * u >= K) break;
                const int k = 16 * wave + 64 * u + 4 * q;
                if (k < K) {
                    *reinterpret_cast<float4*>(f.h + static_cast<long long>(row) * K + k) =
                        make_float4(a[u][0] * r * w[u][0], a[u][1] * r * w[u][1], a[u][2] * r * w[u][2],
                                    a[u][3] * r * w[u][3]);
                    if (f.xout)
                        *reinterpret_cast<float4*>(f.xout + static_cast<long long>(row) * K + k) =
                            make_float4(a[u][0], a[u][1], a[u][2], a[u][3]);
                }
            }
        }
    }
    __syncthreads();
    // thread (wave, lane) finishes accumulator register `wave` of lane `lane`
    const int orow = m0 + 4 * q + wave, ocol = n0 + lr;
    if (orow >= f.M || ocol >= f.N) return;
    float v = ((red[0][wave][lane] + red[1][wave][lane]) + red[2][wave][lane]) + red[3][wave][lane];
    if (NORM) v *= row_s[4 * q + wave];
    const long long o = static_cast<long long>(orow) * f.ldc + ocol;
    if constexpr (DUAL) {
        float v2 = ((red2[0][wave][lane] + red2[1][wave][lane]) + red2[2][wave][lane]) + red2[3][wave][lane];
        v2 *= row_s[4 * q + wave];
        f.C[o] = v;
        f.C2[o] = v2;
        f.Aout[o] = v * sigmoid_sign(v) * v2;
    } else if constexpr (SWB) {
        const float z = f.Z[o], uu = f.U[o];
        const float s = sigmoid_sign(z);
        f.dU[o] = (z * s) * v;
        f.dZ[o] = (s * (1.0f + z * (1.0f - s))) * (uu * v);
    } else {
        f.C[y * f.sC + o] = v;
    }
}

}  // namespace

bool lm_fuse_ok(int K, int lda, int ldb_nt)
{
    return K > 0 && K <= 64 * kFuseU && K % 4 == 0 && lda % 4 == 0 && ldb_nt % 4 == 0;
}

int lm_fused_gemm(const FuseCall& c, hipStream_t s)
{
    const int mode = c.mode;
    const bool tb = (mode & FB_TB) != 0;
    if (c.M <= 0 || c.N <= 0 || c.batch <= 0)
        return fail(LHIP_E_SHAPE, "lm_fused_gemm: M=%d N=%d batch=%d", c.M, c.N, c.batch);
    if (!lm_fuse_ok(c.K, c.lda, tb ? c.ldb : 4))
        return fail(LHIP_E_UNSUPPORTED, "lm_fused_gemm: K=%d lda=%d ldb=%d outside the fused limits", c.K, c.lda,
                    c.ldb);
    if (!c.A || !c.B || !aligned16(c.A) || (tb && !aligned16(c.B)))
        return fail(LHIP_E_ARG, "lm_fused_gemm: A/B NULL or not 16-byte aligned");
    if ((mode & (FB_NORM | FB_NORMBWD)) && (!c.nw || !aligned16(c.nw)))
        return fail(LHIP_E_ARG, "lm_fused_gemm: norm gain NULL or unaligned");
    if ((mode & FB_NORM) && (!c.h || !c.inv || !aligned16(c.h)))
        return fail(LHIP_E_ARG, "lm_fused_gemm: norm outputs");
    if ((mode & FB_NORMBWD) && (!c.nbx || !c.nbinv || !c.nbout || !c.nbpart || !aligned16(c.nbx) ||
                                !aligned16(c.nbout) || (c.nbres && !aligned16(c.nbres))))
        return fail(LHIP_E_ARG, "lm_fused_gemm: norm-backward operands");
    if ((mode & FB_DUAL) && (!c.C || !c.B2 || !c.C2 || !c.Aout || c.batch != 1))
        return fail(LHIP_E_ARG, "lm_fused_gemm: swiglu operands");
    if ((mode & FB_SWIGLU_BWD) && (!c.Z || !c.U || !c.dZ || !c.dU))
        return fail(LHIP_E_ARG, "lm_fused_gemm: swiglu backward operands");
    if (!(mode & (FB_DUAL | FB_SWIGLU_BWD)) && !c.C) return fail(LHIP_E_NULL, "lm_fused_gemm: C is NULL");
    if (c.gather && (!(mode & FB_NORM) || (mode & FB_NORMBWD) || c.gather_rows <= 0 || c.a_parts > 1 ||
                     (c.xout && !aligned16(c.xout))))
        return fail(LHIP_E_ARG, "lm_fused_gemm: gathered A rows need the norm prologue and a table");
    FuseArgs f{};
    f.M = c.M; f.N = c.N; f.K = c.K;
    f.A = c.A; f.lda = c.lda; f.B = c.B; f.ldb = c.ldb; f.sB = c.sB; f.C = c.C; f.ldc = c.ldc; f.sC = c.sC;
    f.tiles_n = ceil_div(c.N, 16);
    f.nw = c.nw; f.eps = c.eps; f.h = c.h; f.inv = c.inv;
    f.B2 = c.B2; f.C2 = c.C2; f.Aout = c.Aout;
    f.Z = c.Z; f.U = c.U; f.dZ = c.dZ; f.dU = c.dU;
    f.nbx = c.nbx; f.nbres = c.nbres; f.nbinv = c.nbinv; f.nbout = c.nbout; f.nbpart = c.nbpart;
    f.a_parts = c.a_parts > 0 ? c.a_parts : 1; f.a_pstride = c.a_pstride;
    f.gather = c.gather; f.gather_rows = c.gather_rows; f.xout = c.xout;
    const long long nwg = static_cast<long long>(ceil_div(c.M, 16)) * f.tiles_n;
    if (nwg > 0x7fffffffLL || c.batch > 65535) return fail(LHIP_E_CAPACITY, "lm_fused_gemm: grid too large");
    dim3 grid(static_cast<unsigned>(nwg), c.batch);
    switch (mode) {
    case FUSE_NORM: klaunch(lm_fused_gemm_kernel<FUSE_NORM>, grid, 256, 0, s, f); break;
    case FUSE_NORM_SWIGLU: klaunch(lm_fused_gemm_kernel<FUSE_NORM_SWIGLU>, grid, 256, 0, s, f); break;
    case FUSE_SWIGLU_BWD: klaunch(lm_fused_gemm_kernel<FUSE_SWIGLU_BWD>, grid, 256, 0, s, f); break;
    case FUSE_NB_SWIGLU_BWD: klaunch(lm_fused_gemm_kernel<FUSE_NB_SWIGLU_BWD>, grid, 256, 0, s, f); break;
    case FUSE_NB_NT: klaunch(lm_fused_gemm_kernel<FUSE_NB_NT>, grid, 256, 0, s, f); break;
    default: return fail(LHIP_E_ARG, "lm_fused_gemm: mode %d", mode);
    }
    return check_launch("lm_fused_gemm");
}

}  // namespace lhip
