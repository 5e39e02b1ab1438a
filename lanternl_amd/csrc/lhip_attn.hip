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
// One workgroup (4 wave64s) per (window, head) keeps q, k, v, P and the
// gradients of the head in LDS, so each direction is one launch instead of
// five or six (RoPE, scores GEMM, softmax, PV GEMM / dP and dv GEMMs, softmax
// backward, dq and dk GEMMs, RoPE backward).  Wave w owns the 16 query rows
// 16w .. 16w+15 (and, backward, the 16 key rows of the same block), so row
// work needs no workgroup barrier.  Every product runs on
// v_mfma_f32_16x16x4f32: lane l supplies A[i0 + l%16][k0 + l/16] and
// B[k0 + l/16][j0 + l%16] from LDS copies stored k-contiguous (row stride
// 68 = 4 mod 64 banks, so these reads are conflict-free) and receives
// D[i0 + 4*(l/16) + e][j0 + l%16] in accumulator e.  A row of a 16x16 block
// therefore lies in one 16-lane DPP row: the softmax and its backward reduce
// the accumulators in place with DPP (no LDS round trip).  Causal blocks above
// the diagonal are skipped.  Operands are zero-padded in LDS to whole
// 16-blocks so padded lanes contribute 0.  The inverse RoPE on dqr/dkr pairs
// columns (2p, 2p+1), which sit in neighbouring lanes of the MFMA result: one
// DPP quad permute brings the partner in.
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

constexpr int kAttnThreads = 256;  // four waves; wave w owns query (and key) rows 16w .. 16w+15
constexpr int kMax = 64;           // T and head_dim limits of the fused path
constexpr int kLd = kMax + 4;      // LDS row stride: 68 = 4 (mod 64 banks), so the operand
                                   // reads X[(base + l%16) * kLd + k0 + l/16] hit 64 banks

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
    int vec;              // T, hd, D % 4 == 0 and 16-byte aligned bases: float4 loads
};

__device__ __forceinline__ int round16(int x) { return (x + 15) & ~15; }
__device__ __forceinline__ int attn_lim(int i, int T, int causal) { return causal ? (i + 1 < T ? i + 1 : T) : T; }

// 16x16 block sum_{k0 <= k < k1} A(i0 + l%16, k) B(k, j0 + l%16) for NB blocks
// side by side (independent accumulator chains); lane l reads
// A(i0 + l%16, k0 + l/16) = a[(i0 + l%16) * kLd + k] and the B element
// b_j[(j0 + l%16) * kLd + k] of block j (both operands stored k-contiguous).
// (Reading every step's operands before the first MFMA was measured slower:
// 10.8 -> 13.3 us for the C2 backward.)
template <int NB>
__device__ __forceinline__ void mfma_rows(floatx4 (&acc)[NB], const float* a, int i0, const float* b, int j0,
                                          int jstep, int nb, int k0, int k1)
{
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
#pragma unroll
    for (int j = 0; j < NB; ++j) acc[j] = floatx4{0.f, 0.f, 0.f, 0.f};
    for (int k = k0; k < k1; k += 4) {
        const float av = a[(i0 + r) * kLd + k + q];
#pragma unroll
        for (int j = 0; j < NB; ++j)
            if (j < nb) acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(av, b[(j0 + j * jstep + r) * kLd + k + q], acc[j], 0, 0, 0);
    }
}

// Load this head's q and k rotated by the forward RoPE and v into LDS, zero on
// [T16, hd16) padding: row-major (rm, [t][d]) and/or transposed (tr, [d][t])
// copies as the caller asks (NULL = not wanted).  Each thread issues all of
// its global loads before any LDS store.
__device__ __forceinline__ void load_qkv(const AttnArgs& a, int b, int h, float* q_rm, float* q_tr, float* k_rm,
                                         float* k_tr, float* v_rm, float* v_tr)
{
    constexpr int U = kMax * (kMax / 2) / kAttnThreads;   // pair slots per thread
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int T16 = round16(T), p16 = round16(hd) >> 1;
    const long long ND = static_cast<long long>(a.N) * D;
    float2 qv[U], kv[U], vv[U], cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = idx / p16, p = idx - t * p16;
        qv[u] = kv[u] = vv[u] = make_float2(0.f, 0.f);
        cv[u] = make_float2(1.f, 0.f);
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
        const int t = idx / p16, p = idx - t * p16;
        if (t < T16) {
            const float2 c = cv[u];
            const int d = 2 * p;
            const float q0 = qv[u].x * c.x - qv[u].y * c.y, q1 = qv[u].x * c.y + qv[u].y * c.x;
            const float k0 = kv[u].x * c.x - kv[u].y * c.y, k1 = kv[u].x * c.y + kv[u].y * c.x;
            if (q_rm) { q_rm[t * kLd + d] = q0; q_rm[t * kLd + d + 1] = q1; }
            if (q_tr) { q_tr[d * kLd + t] = q0; q_tr[(d + 1) * kLd + t] = q1; }
            if (k_rm) { k_rm[t * kLd + d] = k0; k_rm[t * kLd + d + 1] = k1; }
            if (k_tr) { k_tr[d * kLd + t] = k0; k_tr[(d + 1) * kLd + t] = k1; }
            if (v_rm) { v_rm[t * kLd + d] = vv[u].x; v_rm[t * kLd + d + 1] = vv[u].y; }
            if (v_tr) { v_tr[d * kLd + t] = vv[u].x; v_tr[(d + 1) * kLd + t] = vv[u].y; }
        }
    }
}

// float4 form of load_qkv (AttnArgs::vec): a unit is (row t, 4-column group
// g); its q, k, v and (cos, sin) pairs are one float4 load each, row-major
// copies are float4 LDS stores.
__device__ __forceinline__ void load_qkv4(const AttnArgs& a, int b, int h, float* q_rm, float* q_tr, float* k_rm,
                                          float* k_tr, float* v_rm, float* v_tr)
{
    constexpr int U = kMax * (kMax / 4) / kAttnThreads;   // units per thread
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int T16 = round16(T), g16 = round16(hd) >> 2, gq = hd >> 2;
    const long long ND = static_cast<long long>(a.N) * D;
    float4 qv[U], kv[U], vv[U], cv[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = idx / g16, g = idx - t * g16;
        qv[u] = kv[u] = vv[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        cv[u] = make_float4(1.f, 0.f, 1.f, 0.f);
        if (t < T && g < gq) {
            const long long off = static_cast<long long>(b * T + t) * D + h * hd + 4 * g;
            qv[u] = *reinterpret_cast<const float4*>(a.qkv + off);
            kv[u] = *reinterpret_cast<const float4*>(a.qkv + ND + off);
            vv[u] = *reinterpret_cast<const float4*>(a.qkv + 2 * ND + off);
            cv[u] = *reinterpret_cast<const float4*>(a.cs + t * pairs + 2 * g);
        }
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = idx / g16, g = idx - t * g16;
        if (t < T16 && g < g16) {
            const float4 c = cv[u], x = qv[u], y = kv[u], v = vv[u];
            const float4 qr = make_float4(x.x * c.x - x.y * c.y, x.x * c.y + x.y * c.x,
                                          x.z * c.z - x.w * c.w, x.z * c.w + x.w * c.z);
            const float4 kr = make_float4(y.x * c.x - y.y * c.y, y.x * c.y + y.y * c.x,
                                          y.z * c.z - y.w * c.w, y.z * c.w + y.w * c.z);
            const int d = 4 * g;
            if (q_rm) *reinterpret_cast<float4*>(q_rm + t * kLd + d) = qr;
            if (k_rm) *reinterpret_cast<float4*>(k_rm + t * kLd + d) = kr;
            if (v_rm) *reinterpret_cast<float4*>(v_rm + t * kLd + d) = v;
            if (q_tr) { q_tr[d * kLd + t] = qr.x; q_tr[(d + 1) * kLd + t] = qr.y; q_tr[(d + 2) * kLd + t] = qr.z; q_tr[(d + 3) * kLd + t] = qr.w; }
            if (k_tr) { k_tr[d * kLd + t] = kr.x; k_tr[(d + 1) * kLd + t] = kr.y; k_tr[(d + 2) * kLd + t] = kr.z; k_tr[(d + 3) * kLd + t] = kr.w; }
            if (v_tr) { v_tr[d * kLd + t] = v.x; v_tr[(d + 1) * kLd + t] = v.y; v_tr[(d + 2) * kLd + t] = v.z; v_tr[(d + 3) * kLd + t] = v.w; }
        }
    }
}

// Forward.  Wave w: S = scale * qr kr^T for its 16 query rows against the key
// blocks it can see (all, or blocks 0..w when causal), the row softmax in the
// MFMA accumulators (each row's 16 columns of a block sit in one 16-lane DPP
// row), P to global and to LDS, then ctx = P v.
__global__ void __launch_bounds__(kAttnThreads) attn_fwd_kernel(const AttnArgs a)
{
    __shared__ float qs[kMax * kLd];   // [t][d] rotated q
    __shared__ float ks[kMax * kLd];   // [t][d] rotated k
    __shared__ float vT[kMax * kLd];   // [d][t]
    __shared__ float Ps[kMax * kLd];   // [i][j]
    const int b = blockIdx.x / a.H, h = blockIdx.x - b * a.H;
    const int T = a.T, hd = a.hd;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, q = lane >> 4;
    const int nbt = round16(T) >> 4, nbd = round16(hd) >> 4, hd4 = (hd + 3) & ~3, T4 = (T + 3) & ~3;
    if (a.vec) load_qkv4(a, b, h, qs, nullptr, ks, nullptr, nullptr, vT);
    else load_qkv(a, b, h, qs, nullptr, ks, nullptr, nullptr, vT);
    __syncthreads();
    const int i0 = 16 * wave;
    const bool active = i0 < T;
    const int nj = a.causal ? min(wave + 1, nbt) : nbt;   // key blocks this wave sees
    float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
    if (active) {
        // S(i, j) = sum_d q(i, d) k(j, d)
        floatx4 S[4];
        mfma_rows<4>(S, qs, i0, ks, 0, 16, nj, 0, hd4);
        float mx[4], sum[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 4 * q + e, lim = attn_lim(i, T, a.causal);
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float v = (j < nj && 16 * j + r < lim) ? S[j][e] * a.scale : -INFINITY;
                S[j][e] = v;
                m = fmaxf(m, v);
            }
            m = row16_max(m);
            mx[e] = (m == -INFINITY || m != m) ? 0.f : m;
            float sm = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float ev = (j < nj && 16 * j + r < lim) ? expf(S[j][e] - mx[e]) : 0.f;
                S[j][e] = ev;
                sm += ev;
            }
            sm = row16_sum(sm);
            sum[e] = sm > 0.f ? 1.0f / sm : 1.0f;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 4 * q + e;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int c = 16 * j + r;
                const float p = S[j][e] * sum[e];
                if (j < nj) Ps[i * kLd + c] = p;
                if (i < T && c < T && j < nbt) Pg[i * T + c] = j < nj ? p : 0.f;
            }
        }
    }
    __syncthreads();
    if (active) {
        // ctx(i, d) = sum_j P(i, j) v(j, d), j below the causal edge of this block
        const int kend = min(T4, 16 * nj);
        floatx4 O[4];
        mfma_rows<4>(O, Ps, i0, vT, 0, 16, nbd, 0, kend);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 16 * db + r;
            if (db < nbd && d < hd) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = i0 + 4 * q + e;
                    if (i < T) a.ctx[static_cast<long long>(b * T + i) * a.D + h * hd + d] = O[db][e];
                }
            }
        }
    }
}

// Inverse RoPE of a 16x16 result block in MFMA layout (rows t0 + 4q + e,
// columns d0 + l%16) and its store: the pair partner of column d is column
// d ^ 1, held by lane l ^ 1 (DPP quad_perm [1,0,3,2]).
__device__ __forceinline__ void store_unrotated(const AttnArgs& a, float* dst, const floatx4& acc, int b, int h,
                                                int t0, int d0)
{
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const int d = d0 + r, pairs = a.hd >> 1;
    const bool odd = d & 1;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const float mine = acc[e];
        const float other = dpp_f<0xB1>(mine);
        const int t = t0 + 4 * q + e;
        if (t < a.T && d < a.hd) {
            const float2 c = a.cs[t * pairs + (d >> 1)];
            const float g0 = odd ? other : mine, g1 = odd ? mine : other;
            dst[static_cast<long long>(b * a.T + t) * a.D + h * a.hd + d] =
                odd ? (-g0 * c.y + g1 * c.x) : (g0 * c.x + g1 * c.y);
        }
    }
}

// Backward.  Wave w owns query rows 16w.. (dP, dS, dq) and key rows 16w..
// (dv, dk).  Phase 1: dP = dO v^T and dS = scale P o (dP - rowsum(dP o P)) in
// the accumulators (P read from global in the same layout), dS to LDS in both
// orientations, dv = P^T dO.  Phase 2 (after a barrier, all of dS present):
// dq = dS kr, dk = dS^T qr, each through the inverse RoPE.
__global__ void __launch_bounds__(kAttnThreads) attn_bwd_kernel(const AttnArgs a)
{
    __shared__ float qT[kMax * kLd];    // [d][t] rotated q
    __shared__ float kT[kMax * kLd];    // [d][t] rotated k
    __shared__ float vs[kMax * kLd];    // [t][d]
    __shared__ float dOs[kMax * kLd];   // [t][d]
    __shared__ float dOT[kMax * kLd];   // [d][t]
    __shared__ float PT[kMax * kLd];    // [j][i]
    __shared__ float dSs[kMax * kLd];   // [i][j]
    __shared__ float dST[kMax * kLd];   // [j][i]
    const int b = blockIdx.x / a.H, h = blockIdx.x - b * a.H;
    const int T = a.T, hd = a.hd, D = a.D;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, r = lane & 15, q = lane >> 4;
    const int T16 = round16(T), hd16 = round16(hd);
    const int nbt = T16 >> 4, nbd = hd16 >> 4, hd4 = (hd + 3) & ~3, T4 = (T + 3) & ~3;
    const long long ND = static_cast<long long>(a.N) * D;
    const int i0 = 16 * wave;
    const bool active = i0 < T;
    const int nj = a.causal ? min(wave + 1, nbt) : nbt;
    const float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
    if (a.vec) {
        load_qkv4(a, b, h, nullptr, qT, nullptr, kT, vs, nullptr);
        // P^T and dO, dO^T from float4 loads: a P unit is (row i, 4-column
        // group c), a dO unit (row i, 4-column group g); zero padded to T16 / hd16
        constexpr int UP = kMax * (kMax / 4) / kAttnThreads;
        const int c16 = T16 >> 2, g16 = hd16 >> 2;
        float4 pv[UP], ov[UP];
#pragma unroll
        for (int u = 0; u < UP; ++u) {
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / c16, c = idx - i * c16;
            const int oi = idx / g16, og = idx - oi * g16;
            pv[u] = (i < T && 4 * c < T) ? *reinterpret_cast<const float4*>(Pg + i * T + 4 * c)
                                         : make_float4(0.f, 0.f, 0.f, 0.f);
            ov[u] = (oi < T && 4 * og < hd)
                        ? *reinterpret_cast<const float4*>(a.dctx + static_cast<long long>(b * T + oi) * D + h * hd + 4 * og)
                        : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int u = 0; u < UP; ++u) {
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / c16, c = idx - i * c16;
            const int oi = idx / g16, og = idx - oi * g16;
            if (i < T16) {
                const int j = 4 * c;
                PT[j * kLd + i] = pv[u].x; PT[(j + 1) * kLd + i] = pv[u].y;
                PT[(j + 2) * kLd + i] = pv[u].z; PT[(j + 3) * kLd + i] = pv[u].w;
            }
            if (oi < T16) {
                const int d = 4 * og;
                *reinterpret_cast<float4*>(dOs + oi * kLd + d) = ov[u];
                dOT[d * kLd + oi] = ov[u].x; dOT[(d + 1) * kLd + oi] = ov[u].y;
                dOT[(d + 2) * kLd + oi] = ov[u].z; dOT[(d + 3) * kLd + oi] = ov[u].w;
            }
        }
    } else {
        load_qkv(a, b, h, nullptr, qT, nullptr, kT, vs, nullptr);
        // P^T, dO and dO^T over [T16) x [T16) / [T16) x [hd16), zero padded
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
            if (i < T16 && j < T16) PT[j * kLd + i] = pv[u];
            if (i < T16 && j < hd16) { dOs[i * kLd + j] = ov[u]; dOT[j * kLd + i] = ov[u]; }
        }
    }
    __syncthreads();
    // this wave's P rows in accumulator layout (P^T is zero padded past T)
    float Pd[4][4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 4 * q + e, c = 16 * j + r;
            Pd[j][e] = (active && j < nj) ? PT[c * kLd + i] : 0.f;
        }
    if (active) {
        // dP(i, j) = sum_d dO(i, d) v(j, d)
        floatx4 G[4];
        mfma_rows<4>(G, dOs, i0, vs, 0, 16, nj, 0, hd4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float dot = 0.f;
#pragma unroll
            for (int j = 0; j < 4; ++j) dot += (j < nj) ? G[j][e] * Pd[j][e] : 0.f;
            dot = row16_sum(dot);
            const int i = i0 + 4 * q + e;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                if (j < nj) {
                    const float ds = a.scale * (Pd[j][e] * (G[j][e] - dot));
                    dSs[i * kLd + 16 * j + r] = ds;
                    dST[(16 * j + r) * kLd + i] = ds;
                }
            }
        }
        // dv(j, d) = sum_i P(i, j) dO(i, d) over query rows i >= 16w (causal) for keys j in block w
        const int kbeg = a.causal ? i0 : 0;
        floatx4 V[4];
        mfma_rows<4>(V, PT, i0, dOT, 0, 16, nbd, kbeg, T4);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int d = 16 * db + r;
            if (db < nbd && d < hd) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int t = i0 + 4 * q + e;
                    if (t < T) a.dqkv[2 * ND + static_cast<long long>(b * T + t) * D + h * hd + d] = V[db][e];
                }
            }
        }
    }
    __syncthreads();
    if (active) {
        // dqr(i, d) = sum_j dS(i, j) kr(j, d) ; dkr(j, d) = sum_i dS(i, j) qr(i, d)
        const int kend = min(T4, 16 * nj);
        const int kbeg = a.causal ? i0 : 0;
        floatx4 Q[4], K[4];
        mfma_rows<4>(Q, dSs, i0, kT, 0, 16, nbd, 0, kend);
        mfma_rows<4>(K, dST, i0, qT, 0, 16, nbd, kbeg, T4);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            if (db < nbd) {
                store_unrotated(a, a.dqkv, Q[db], b, h, i0, 16 * db);
                store_unrotated(a, a.dqkv + ND, K[db], b, h, i0, 16 * db);
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
    a.vec = (hd % 4 == 0 && aligned16(qkv) && aligned16(cs)) ? 1 : 0;
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
    a.vec = (hd % 4 == 0 && T % 4 == 0 && aligned16(qkv) && aligned16(cs) && aligned16(P) && aligned16(dctx)) ? 1 : 0;
    attn_bwd_kernel<<<B * H, kAttnThreads, 0, s>>>(a);
    return check_launch("attn_bwd");
}

}  // namespace lhip
