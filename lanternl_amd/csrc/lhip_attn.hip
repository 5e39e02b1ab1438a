// lhip_attn.hip -- fused per-(window, head) attention of the CPU LMTrain path.
//
// Forward (ai/nn/transformer.lua:196-226 for one head of one window):
//   qr, kr = RoPE(q), RoPE(k)        interleaved pairs, angle table of transformer.lua:30-48
//   S = (qr . kr^T) * scale          Tensor.matmul_nt + Tensor.scale
//   P = softmax_rows(S, causal)      tensor2.lua:332-383
//   ctx_h = P . v                    Tensor.matmul, concat_cols
// Backward (tensor2.lua BACKWARD.* in reverse order):
//   dP = dO . v^T, dv = P^T . dO, dS = scale * P o (dP - rowsum(dP o P)),
//   dqr = dS . kr, dkr = dS^T . qr, dq, dk = inverse RoPE of dqr, dkr.
// One workgroup (4 wave64s) per (window, head) keeps q, k, v, S/P and the
// gradients of the head in LDS, so each direction is one launch instead of
// five or six (RoPE, scores GEMM, softmax, PV GEMM / dP and dv GEMMs, softmax
// backward, dq and dk GEMMs, RoPE backward).  Every product runs on
// v_mfma_f32_16x16x4f32: 16x16 output blocks are dealt round-robin to the
// four waves; lane l supplies A[i0 + l%16][k0 + l/16] and B[k0 + l/16][j0 +
// l%16] read from LDS (odd row strides keep those column reads conflict-free)
// and receives D[i0 + 4*(l/16) + r][j0 + l%16] in accumulator r.  Operands
// are zero-padded in LDS to whole 16-blocks so padded lanes contribute 0.
// The inverse RoPE on dqr/dkr pairs columns (2p, 2p+1), which sit in
// neighbouring lanes of the MFMA result: one __shfl_xor(v, 1) brings the
// partner in.
//
// Layouts: qkv[3][N][D] with N = B*T rows (window b's rows b*T .. b*T+T-1) and
// head h in columns h*hd .. h*hd+hd-1; P[B][H][T][T]; rope table cs[T][hd/2]
// of (cos, sin) for positions 0..T-1.
#include <cmath>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kAttnThreads = 256;
constexpr int kMax = 64;          // T and head_dim limits of the fused path
constexpr int kLd = kMax + 1;     // LDS row stride (odd: conflict-free column reads)

struct AttnArgs {
    const float* qkv;     // [3][N][D]
    const float2* cs;     // [T][hd/2]
    float* P;             // [B][H][T][T]
    float* ctx;           // [N][D]        (forward)
    const float* dctx;    // [N][D]        (backward)
    float* dqkv;          // [3][N][D]     (backward)
    int B, H, T, hd, D, N;
    float scale;
    int causal;
};

__device__ __forceinline__ int round16(int x) { return (x + 15) & ~15; }
__device__ __forceinline__ int attn_lim(int i, int T, int causal) { return causal ? (i + 1 < T ? i + 1 : T) : T; }

// Load this head's q and k rotated (forward RoPE) and v into LDS [64][kLd],
// zero outside [T][hd].  Each thread first issues all of its global loads
// (fully unrolled, float2 pairs), then rotates and stores, so the loads of a
// thread are in flight together instead of one round trip per pair.
__device__ __forceinline__ void load_head(const AttnArgs& a, int b, int h, float* qs, float* ks, float* vs)
{
    constexpr int U = kMax * (kMax / 2) / kAttnThreads;   // pair slots per thread
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const long long ND = static_cast<long long>(a.N) * D;
    float2 qv[U], kv[U], vv[U], cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = idx / (kMax / 2), p = idx - t * (kMax / 2);
        qv[u] = kv[u] = vv[u] = cv[u] = make_float2(0.f, 0.f);
        if (t < T && p < pairs) {
            const long long off = static_cast<long long>(b * T + t) * D + h * hd + 2 * p;
            qv[u] = *reinterpret_cast<const float2*>(a.qkv + off);
            kv[u] = *reinterpret_cast<const float2*>(a.qkv + ND + off);
            vv[u] = *reinterpret_cast<const float2*>(a.qkv + 2 * ND + off);
            cv[u] = a.cs[t * pairs + p];
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = idx / (kMax / 2), p = idx - t * (kMax / 2);
        const float2 c = cv[u];
        qs[t * kLd + 2 * p] = qv[u].x * c.x - qv[u].y * c.y;
        qs[t * kLd + 2 * p + 1] = qv[u].x * c.y + qv[u].y * c.x;
        ks[t * kLd + 2 * p] = kv[u].x * c.x - kv[u].y * c.y;
        ks[t * kLd + 2 * p + 1] = kv[u].x * c.y + kv[u].y * c.x;
        vs[t * kLd + 2 * p] = vv[u].x;
        vs[t * kLd + 2 * p + 1] = vv[u].y;
    }
}

// One 16x16 output block of sum_k A(i, k) B(k, j), k < K4 (K4 % 4 == 0, zero padded).
template <class FA, class FB>
__device__ __forceinline__ floatx4 mfma_block(int i0, int j0, int K4, FA fa, FB fb)
{
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K4; k0 += 4)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(fa(i0 + r, k0 + q), fb(k0 + q, j0 + r), acc, 0, 0, 0);
    return acc;
}

__global__ void __launch_bounds__(kAttnThreads) attn_fwd_kernel(const AttnArgs a)
{
    __shared__ float qs[kMax * kLd];
    __shared__ float ks[kMax * kLd];
    __shared__ float vs[kMax * kLd];
    __shared__ float S[kMax * kLd];
    const int b = blockIdx.x / a.H, h = blockIdx.x - b * a.H;
    const int T = a.T, hd = a.hd;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T16 = round16(T), hd16 = round16(hd), hd4 = (hd + 3) & ~3, T4 = (T + 3) & ~3;
    load_head(a, b, h, qs, ks, vs);
    __syncthreads();
    // S = scale * qr . kr^T on the kept prefix, -inf beyond (never read)
    {
        const int nbj = T16 / 16, nblk = nbj * nbj;
        for (int blk = wave; blk < nblk; blk += 4) {
            const int i0 = (blk / nbj) * 16, j0 = (blk % nbj) * 16;
            const floatx4 acc = mfma_block(i0, j0, hd4, [&](int i, int k) { return qs[i * kLd + k]; },
                                           [&](int k, int j) { return ks[j * kLd + k]; });
            const int j = j0 + (lane & 15);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int i = i0 + 4 * (lane >> 4) + r;
                S[i * kLd + j] = acc[r] * a.scale;
            }
        }
    }
    __syncthreads();
    // row softmax: one wave per row, one lane per column (T <= 64)
    float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
    for (int i = wave; i < T; i += 4) {
        const int lim = attn_lim(i, T, a.causal);
        const float v = lane < lim ? S[i * kLd + lane] : -INFINITY;
        float mx = wave_max(v);
        if (mx == -INFINITY || mx != mx) mx = 0.f;
        const float e = lane < lim ? expf(v - mx) : 0.f;
        float sum = wave_sum(e);
        if (!(sum > 0.f)) sum = 1.f;
        const float p = e * (1.0f / sum);
        S[i * kLd + lane] = p;                // zero beyond the kept prefix (and past T)
        if (lane < T) Pg[i * T + lane] = p;
    }
    for (int i = T + wave; i < T4; i += 4) S[i * kLd + lane] = 0.f;
    __syncthreads();
    // ctx_h = P . v
    {
        const int nbi = T16 / 16, nbj = hd16 / 16, nblk = nbi * nbj;
        for (int blk = wave; blk < nblk; blk += 4) {
            const int i0 = (blk / nbj) * 16, j0 = (blk % nbj) * 16;
            const floatx4 acc = mfma_block(i0, j0, T4, [&](int i, int k) { return S[i * kLd + k]; },
                                           [&](int k, int j) { return vs[k * kLd + j]; });
            const int d = j0 + (lane & 15);
            if (d < hd) {
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int i = i0 + 4 * (lane >> 4) + r;
                    if (i < T) a.ctx[static_cast<long long>(b * T + i) * a.D + h * hd + d] = acc[r];
                }
            }
        }
    }
}

__global__ void __launch_bounds__(kAttnThreads) attn_bwd_kernel(const AttnArgs a)
{
    __shared__ float qs[kMax * kLd];
    __shared__ float ks[kMax * kLd];
    __shared__ float vs[kMax * kLd];
    __shared__ float dO[kMax * kLd];
    __shared__ float Ps[kMax * kLd];
    __shared__ float dS[kMax * kLd];
    const int b = blockIdx.x / a.H, h = blockIdx.x - b * a.H;
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int T16 = round16(T), hd16 = round16(hd), hd4 = (hd + 3) & ~3, T4 = (T + 3) & ~3;
    const long long ND = static_cast<long long>(a.N) * D;
    load_head(a, b, h, qs, ks, vs);
    const float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
    {
        // all of this thread's P and dO loads first, then the LDS stores
        constexpr int U = kMax * kMax / kAttnThreads;
        float pv[U], ov[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / kMax, j = idx - i * kMax;
            pv[u] = (i < T && j < T) ? Pg[i * T + j] : 0.f;
            ov[u] = (i < T && j < hd) ? a.dctx[static_cast<long long>(b * T + i) * D + h * hd + j] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / kMax, j = idx - i * kMax;
            Ps[i * kLd + j] = pv[u];
            dO[i * kLd + j] = ov[u];
        }
    }
    __syncthreads();
    // dP = dO . v^T (T x T, into dS); dv = P^T . dO (T x hd, to global)
    {
        const int nbt = T16 / 16, nbd = hd16 / 16;
        const int n1 = nbt * nbt, n2 = nbt * nbd;
        for (int blk = wave; blk < n1 + n2; blk += 4) {
            if (blk < n1) {
                const int i0 = (blk / nbt) * 16, j0 = (blk % nbt) * 16;
                const floatx4 acc = mfma_block(i0, j0, hd4, [&](int i, int k) { return dO[i * kLd + k]; },
                                               [&](int k, int j) { return vs[j * kLd + k]; });
                const int j = j0 + (lane & 15);
#pragma unroll
                for (int r = 0; r < 4; ++r) dS[(i0 + 4 * (lane >> 4) + r) * kLd + j] = acc[r];
            } else {
                const int bb = blk - n1;
                const int i0 = (bb / nbd) * 16, j0 = (bb % nbd) * 16;   // i: key row j, j: d
                const floatx4 acc = mfma_block(i0, j0, T4, [&](int i, int k) { return Ps[k * kLd + i]; },
                                               [&](int k, int j) { return dO[k * kLd + j]; });
                const int d = j0 + (lane & 15);
                if (d < hd) {
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int t = i0 + 4 * (lane >> 4) + r;
                        if (t < T) a.dqkv[2 * ND + static_cast<long long>(b * T + t) * D + h * hd + d] = acc[r];
                    }
                }
            }
        }
    }
    __syncthreads();
    // dS = scale * P o (dP - sum_{j<lim} dP P); zero beyond the kept prefix and past T
    for (int i = wave; i < kMax; i += 4) {
        if (i < T) {
            const int lim = attn_lim(i, T, a.causal);
            const float p = lane < lim ? Ps[i * kLd + lane] : 0.f;
            const float g = lane < lim ? dS[i * kLd + lane] : 0.f;
            const float dot = wave_sum(g * p);
            dS[i * kLd + lane] = lane < lim ? a.scale * (p * (g - dot)) : 0.f;
        } else {
            dS[i * kLd + lane] = 0.f;
        }
    }
    __syncthreads();
    // dqr = dS . kr, dkr = dS^T . qr, then the inverse rotation of each pair
    {
        const int nbt = T16 / 16, nbd = hd16 / 16, n = nbt * nbd;
        for (int blk = wave; blk < 2 * n; blk += 4) {
            const bool isq = blk < n;
            const int bb = isq ? blk : blk - n;
            const int i0 = (bb / nbd) * 16, j0 = (bb % nbd) * 16;
            floatx4 acc;
            if (isq)
                acc = mfma_block(i0, j0, T4, [&](int i, int k) { return dS[i * kLd + k]; },
                                 [&](int k, int j) { return ks[k * kLd + j]; });
            else
                acc = mfma_block(i0, j0, T4, [&](int i, int k) { return dS[k * kLd + i]; },
                                 [&](int k, int j) { return qs[k * kLd + j]; });
            const int d = j0 + (lane & 15);
            const bool odd = d & 1;
            float* dst = a.dqkv + (isq ? 0 : ND);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int t = i0 + 4 * (lane >> 4) + r;
                const float mine = acc[r];
                const float other = __shfl_xor(mine, 1, 64);   // column d ^ 1 of the same row
                if (t < T && d < hd) {
                    const float2 c = a.cs[t * pairs + (d >> 1)];
                    const float g0 = odd ? other : mine, g1 = odd ? mine : other;
                    dst[static_cast<long long>(b * T + t) * D + h * hd + d] =
                        odd ? (-g0 * c.y + g1 * c.x) : (g0 * c.x + g1 * c.y);
                }
            }
        }
    }
}

}  // namespace

bool attn_fused_ok(int T, int hd) { return T >= 1 && T <= kMax && hd >= 2 && hd <= kMax && hd % 2 == 0; }

int attn_fwd(const float* qkv, const float2* cs, float* P, float* ctx, int B, int H, int T, int hd, float scale,
             int causal, hipStream_t s)
{
    if (!attn_fused_ok(T, hd)) return fail(LHIP_E_UNSUPPORTED, "attn_fwd: T=%d hd=%d outside the fused limits", T, hd);
    if (!qkv || !cs || !P || !ctx) return fail(LHIP_E_NULL, "attn_fwd: NULL argument");
    AttnArgs a{};
    a.qkv = qkv; a.cs = cs; a.P = P; a.ctx = ctx;
    a.B = B; a.H = H; a.T = T; a.hd = hd; a.D = H * hd; a.N = B * T;
    a.scale = scale; a.causal = causal;
    attn_fwd_kernel<<<B * H, kAttnThreads, 0, s>>>(a);
    return check_launch("attn_fwd");
}

int attn_bwd(const float* qkv, const float2* cs, const float* P, const float* dctx, float* dqkv, int B, int H, int T,
             int hd, float scale, int causal, hipStream_t s)
{
    if (!attn_fused_ok(T, hd)) return fail(LHIP_E_UNSUPPORTED, "attn_bwd: T=%d hd=%d outside the fused limits", T, hd);
    if (!qkv || !cs || !P || !dctx || !dqkv) return fail(LHIP_E_NULL, "attn_bwd: NULL argument");
    AttnArgs a{};
    a.qkv = qkv; a.cs = cs; a.P = const_cast<float*>(P); a.dctx = dctx; a.dqkv = dqkv;
    a.B = B; a.H = H; a.T = T; a.hd = hd; a.D = H * hd; a.N = B * T;
    a.scale = scale; a.causal = causal;
    attn_bwd_kernel<<<B * H, kAttnThreads, 0, s>>>(a);
    return check_launch("attn_bwd");
}

}  // namespace lhip
