// lhip_attn.hip -- fused attention of the CPU LMTrain path.
//
// Forward (ai/nn/transformer.lua:196-226 for one head of one window):
//   qr, kr = RoPE(q), RoPE(k)        interleaved pairs, angle table of transformer.lua:30-48
//   S = (qr . kr^T) * scale          Tensor.matmul_nt + Tensor.scale
//   P = softmax_rows(S, causal)      tensor2.lua:332-383
//   ctx_h = P . v                    Tensor.matmul, concat_cols
// Backward (tensor2.lua BACKWARD.* in reverse order):
//   dP = dO . v^T, dv = P^T . dO, dS = scale * P o (dP - rowsum(dP o P)),
//   dqr = dS . kr, dkr = dS^T . qr, dq, dk = inverse RoPE of dqr, dkr.
// Each direction is one launch instead of five or six (RoPE, scores GEMM,
// softmax, PV GEMM / dP and dv GEMMs, softmax backward, dq and dk GEMMs, RoPE
// backward).  The forward runs one wave per (window, head, 16-row query
// block) with no LDS when the float4 forms apply (attn_fwd_wave_kernel);
// otherwise, and in the backward, a (window, head) is split over one
// workgroup (4 wave64s) per 16-row block, so a C2 layer runs 256 workgroups
// (one per CU) instead of 64:
// the step is latency-bound and a wave's VALU work is what it waits on, so the
// work is spread over CUs, one 16x16 block per wave.  The backward uses
// rowsum(dP o P) = rowsum(dO o O) (O = ctx), which makes each dS block
// computable from its own dO, v and P blocks, so no workgroup needs another's
// results.  Every product runs on v_mfma_f32_16x16x4f32 (lane l supplies
// A[l%16][k0 + l/16] and B[k0 + l/16][l%16] and receives C[4*(l/16) + e][l%16]
// in element e) from LDS copies stored k-contiguous (row stride 68 = 4 mod 64
// banks, so the reads are conflict-free); a row of a 16x16 block therefore
// lies in one 16-lane DPP row and the softmax reduces it in place with DPP.
// Operands are zero-padded in LDS to whole 16-blocks so padded lanes
// contribute 0.  Partial sums over blocks go through LDS and are added in a
// fixed (wave) order, so results are deterministic.
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
constexpr int kBl = 20;            // row stride of a wave's own 16x16 LDS block: writes from the
                                   // accumulator layout ([4(l/16) + e][l%16]) hit 64 banks

struct AttnArgs {
    const float* qkv;     // [3][N][D]
    const float2* cs;     // [T][hd/2]
    float* P;             // [B][H][T][T]
    float* ctx;           // [N][D]        (forward output; backward input O)
    const float* dctx;    // [N][D]        (backward)
    float* dqkv;          // [3][N][D]     (backward)
    int B, H, T, hd, D, N;
    float scale;
    int causal;
    int vec;              // T, hd, D % 4 == 0 and 16-byte aligned bases: float4 loads
    const int* wlen;      // [B] keys of each window (NULL: T); keys past it are masked
};

__device__ __forceinline__ int round16(int x) { return (x + 15) & ~15; }
// keys visible to query row i: those below kl (the window's length, or T),
// and at most i when causal; a row with none gets a zero P row
__device__ __forceinline__ int attn_lim(int i, int kl, int causal) { return causal ? (i + 1 < kl ? i + 1 : kl) : kl; }

// One 16x16 block C(i, j) = sum_{0 <= k < K4} A(i, k) B(k, j) (K4 % 4 == 0,
// wave-uniform): lane l supplies A(l%16, k + l/16) = a[(l%16) * ars +
// (k + l/16) * aks] and B(k + l/16, l%16) = b[(l%16) * brs + (k + l/16) * bks]
// and receives C(4 (l/16) + e, l%16) in element e.  K is walked in chunks of
// four 4-deep steps whose LDS reads (steps past K4 clamped to the last one)
// issue before their MFMAs.
__device__ __forceinline__ floatx4 mfma_block(const float* a, int ars, int aks, const float* b, int brs, int bks,
                                              int K4)
{
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    K4 = __builtin_amdgcn_readfirstlane(K4);
    floatx4 acc = {0.f, 0.f, 0.f, 0.f};
    const float* ar = a + r * ars + q * aks;
    const float* br = b + r * brs + q * bks;
    for (int k = 0; k < K4; k += 16) {
        float av[4], bv[4];
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            const int kk = min(k + 4 * st, K4 - 4);
            av[st] = ar[kk * aks];
            bv[st] = br[kk * bks];
        }
#pragma unroll
        for (int st = 0; st < 4; ++st) {
            if (k + 4 * st >= K4) break;
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(av[st], bv[st], acc, 0, 0, 0);
        }
    }
    return acc;
}

// Orders a wave's LDS writes before its own later LDS reads of other lanes'
// values (the LDS serves one wave's requests in order; the fences keep the
// compiler from moving the reads above the writes).
__device__ __forceinline__ void wave_lds_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// This thread's units of q, k, v and their (cos, sin) pairs, in registers.  A
// unit is (row t, column group g) of W columns; fetch issues the global loads
// (zeros outside [T) x [hd)), put rotates q and k by the forward RoPE and
// writes row-major (rm, [t][d]) and/or transposed (tr, [d][t]) LDS copies as
// the caller asks (NULL = not wanted), zero on the [T16, hd16) padding.  A
// caller issues every global load it needs before its first put.
// idx / gw for idx < 4096 and 1 <= gw <= 64 as a multiply-shift: with
// m = ceil(2^18 / gw) the error idx * (m - 2^18/gw) / 2^18 stays below
// 1/64 <= 1/gw, so the quotient's floor is exact.
__device__ __forceinline__ int div_magic(int gw) { return ((1 << 18) + gw - 1) / gw; }
__device__ __forceinline__ int div_by(int idx, int magic) { return (idx * magic) >> 18; }

template <typename V, int W>
struct QkvUnits {
    static constexpr int U = kMax * (kMax / W) / kAttnThreads;   // unit slots per thread
    V q[U], k[U], v[U], c[U];
};
using Qkv4 = QkvUnits<float4, 4>;   // AttnArgs::vec: head_dim % 4 == 0, 16-byte aligned
using Qkv2 = QkvUnits<float2, 2>;

__device__ __forceinline__ void qkv_fetch(const AttnArgs& a, int b, int h, Qkv4& x)
{
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int g16 = round16(hd) >> 2, gq = hd >> 2, units = round16(T) * g16, mg = div_magic(g16);
    const long long ND = static_cast<long long>(a.N) * D;
#pragma unroll
    for (int u = 0; u < Qkv4::U; ++u) {
        if (kAttnThreads * u >= units) break;   // uniform: no thread has this slot
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = div_by(idx, mg), g = idx - t * g16;
        x.q[u] = x.k[u] = x.v[u] = make_float4(0.f, 0.f, 0.f, 0.f);
        x.c[u] = make_float4(1.f, 0.f, 1.f, 0.f);
        if (t < T && g < gq) {
            const long long off = static_cast<long long>(b * T + t) * D + h * hd + 4 * g;
            x.q[u] = *reinterpret_cast<const float4*>(a.qkv + off);
            x.k[u] = *reinterpret_cast<const float4*>(a.qkv + ND + off);
            x.v[u] = *reinterpret_cast<const float4*>(a.qkv + 2 * ND + off);
            x.c[u] = *reinterpret_cast<const float4*>(a.cs + t * pairs + 2 * g);
        }
    }
}

__device__ __forceinline__ void qkv_put(const AttnArgs& a, const Qkv4& x, float* q_rm, float* q_tr, float* k_rm,
                                        float* k_tr, float* v_rm, float* v_tr)
{
    const int T16 = round16(a.T), g16 = round16(a.hd) >> 2, units = T16 * g16, mg = div_magic(g16);
#pragma unroll
    for (int u = 0; u < Qkv4::U; ++u) {
        if (kAttnThreads * u >= units) break;
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = div_by(idx, mg), g = idx - t * g16;
        if (idx < units) {
            const float4 c = x.c[u], y = x.q[u], z = x.k[u], v = x.v[u];
            const float4 qr = make_float4(y.x * c.x - y.y * c.y, y.x * c.y + y.y * c.x,
                                          y.z * c.z - y.w * c.w, y.z * c.w + y.w * c.z);
            const float4 kr = make_float4(z.x * c.x - z.y * c.y, z.x * c.y + z.y * c.x,
                                          z.z * c.z - z.w * c.w, z.z * c.w + z.w * c.z);
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

__device__ __forceinline__ void qkv_fetch(const AttnArgs& a, int b, int h, Qkv2& x)
{
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int p16 = round16(hd) >> 1, units = round16(T) * p16, mg = div_magic(p16);
    const long long ND = static_cast<long long>(a.N) * D;
#pragma unroll
    for (int u = 0; u < Qkv2::U; ++u) {
        if (kAttnThreads * u >= units) break;
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = div_by(idx, mg), p = idx - t * p16;
        x.q[u] = x.k[u] = x.v[u] = make_float2(0.f, 0.f);
        x.c[u] = make_float2(1.f, 0.f);
        if (t < T && p < pairs) {
            const long long off = static_cast<long long>(b * T + t) * D + h * hd + 2 * p;
            x.q[u] = *reinterpret_cast<const float2*>(a.qkv + off);
            x.k[u] = *reinterpret_cast<const float2*>(a.qkv + ND + off);
            x.v[u] = *reinterpret_cast<const float2*>(a.qkv + 2 * ND + off);
            x.c[u] = a.cs[t * pairs + p];
        }
    }
}

__device__ __forceinline__ void qkv_put(const AttnArgs& a, const Qkv2& x, float* q_rm, float* q_tr, float* k_rm,
                                        float* k_tr, float* v_rm, float* v_tr)
{
    const int T16 = round16(a.T), p16 = round16(a.hd) >> 1, units = T16 * p16, mg = div_magic(p16);
#pragma unroll
    for (int u = 0; u < Qkv2::U; ++u) {
        if (kAttnThreads * u >= units) break;
        const int idx = threadIdx.x + kAttnThreads * u;
        const int t = div_by(idx, mg), p = idx - t * p16;
        if (idx < units) {
            const float2 c = x.c[u], v = x.v[u];
            const int d = 2 * p;
            const float q0 = x.q[u].x * c.x - x.q[u].y * c.y, q1 = x.q[u].x * c.y + x.q[u].y * c.x;
            const float k0 = x.k[u].x * c.x - x.k[u].y * c.y, k1 = x.k[u].x * c.y + x.k[u].y * c.x;
            if (q_rm) { q_rm[t * kLd + d] = q0; q_rm[t * kLd + d + 1] = q1; }
            if (q_tr) { q_tr[d * kLd + t] = q0; q_tr[(d + 1) * kLd + t] = q1; }
            if (k_rm) { k_rm[t * kLd + d] = k0; k_rm[t * kLd + d + 1] = k1; }
            if (k_tr) { k_tr[d * kLd + t] = k0; k_tr[(d + 1) * kLd + t] = k1; }
            if (v_rm) { v_rm[t * kLd + d] = v.x; v_rm[t * kLd + d + 1] = v.y; }
            if (v_tr) { v_tr[d * kLd + t] = v.x; v_tr[(d + 1) * kLd + t] = v.y; }
        }
    }
}

// Forward.  Workgroup (window b, head h, query block c); wave w takes key
// block w when it is visible (w < nj: every block, or blocks 0..c when
// causal).  S = scale * qr kr^T for the 16x16 block; the row maxima, then the
// row sums of exp, are exchanged through LDS and combined in wave order; P goes
// to global and, through a per-wave LDS block, into the wave's share
// P(c, w) v(w) of ctx; the shares are summed in wave order by the store.
__global__ void __launch_bounds__(kAttnThreads) attn_fwd_kernel(const AttnArgs a)
{
    __shared__ float qs[kMax * kLd];                    // [t][d] rotated q
    __shared__ float ks[kMax * kLd];                    // [t][d] rotated k
    __shared__ float vT[kMax * kLd];                    // [d][t]
    __shared__ float Pw[4][16 * kBl];                   // per wave: P(c, w) [i][j]
    __shared__ __align__(16) float part[4][16 * kLd];   // per wave: ctx share [i][d]
    __shared__ float rmax[4][16], rsum[4][16];
    const int T = a.T, hd = a.hd;
    const int nbt = round16(T) >> 4, nbd = round16(hd) >> 4, hd4 = (hd + 3) & ~3;
    const int pid = xcd_pid(blockIdx.x, gridDim.x);   // window-major, XCD-contiguous (as the GEMMs' rows)
    const int c = pid % nbt, bh = pid / nbt, b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
    const int i0 = 16 * c;
    const int nj = a.causal ? c + 1 : nbt;
    const bool act = wave < nj;
    const int col = 16 * wave + r;
    const int kl = a.wlen ? min(T, a.wlen[b]) : T;
    if (a.vec) {
        Qkv4 x;
        qkv_fetch(a, b, h, x);
        qkv_put(a, x, qs, nullptr, ks, nullptr, nullptr, vT);
    } else {
        Qkv2 x;
        qkv_fetch(a, b, h, x);
        qkv_put(a, x, qs, nullptr, ks, nullptr, nullptr, vT);
    }
    __syncthreads();
    float v[4] = {0.f, 0.f, 0.f, 0.f}, p[4] = {0.f, 0.f, 0.f, 0.f};
    if (act) {
        const floatx4 S = mfma_block(qs + i0 * kLd, kLd, 1, ks + 16 * wave * kLd, kLd, 1, hd4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[e] = col < attn_lim(i0 + 4 * q + e, kl, a.causal) ? S[e] * a.scale : -INFINITY;
            const float m = row16_max(v[e]);
            if (r == 0) rmax[wave][4 * q + e] = m;
        }
    }
    __syncthreads();
    if (act) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float m = -INFINITY;
            for (int w = 0; w < nj; ++w) m = fmaxf(m, rmax[w][4 * q + e]);
            const float mx = (m == -INFINITY || m != m) ? 0.f : m;
            p[e] = col < attn_lim(i0 + 4 * q + e, kl, a.causal) ? expf(v[e] - mx) : 0.f;
            const float s = row16_sum(p[e]);
            if (r == 0) rsum[wave][4 * q + e] = s;
        }
    }
    __syncthreads();
    if (act) {
        float* pw = Pw[wave];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            float s = 0.f;
            for (int w = 0; w < nj; ++w) s += rsum[w][4 * q + e];
            p[e] *= s > 0.f ? 1.0f / s : 1.0f;
            pw[(4 * q + e) * kBl + r] = p[e];
        }
        wave_lds_sync();
        for (int db = 0; db < nbd; ++db) {
            const floatx4 O = mfma_block(pw, kBl, 1, vT + 16 * db * kLd + 16 * wave, kLd, 1, 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) part[wave][(4 * q + e) * kLd + 16 * db + r] = O[e];
        }
    }
    __syncthreads();
    // P rows i0 .. i0+15 (zeros above the causal edge), stored after the last
    // barrier: a barrier waits for the wave's outstanding global stores
    if (wave < nbt) {
        float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int i = i0 + 4 * q + e;
            if (i < T && col < T) Pg[i * T + col] = p[e];
        }
    }
    // ctx rows i0 .. i0+15: thread (i, g) sums the shares of columns 4g .. 4g+3
    const int i = threadIdx.x >> 4, d = 4 * (threadIdx.x & 15), row = i0 + i;
    if (row < T && d < hd) {
        float4 o = *reinterpret_cast<const float4*>(&part[0][i * kLd + d]);
        for (int w = 1; w < nj; ++w) {
            const float4 t = *reinterpret_cast<const float4*>(&part[w][i * kLd + d]);
            o.x += t.x; o.y += t.y; o.z += t.z; o.w += t.w;
        }
        float* dst = a.ctx + static_cast<long long>(b * T + row) * a.D + h * hd + d;
        if (a.vec) {
            *reinterpret_cast<float4*>(dst) = o;
        } else {
            dst[0] = o.x; dst[1] = o.y;             // hd even: d + 1 < hd
            if (d + 2 < hd) { dst[2] = o.z; dst[3] = o.w; }
        }
    }
}

// Forward on one wave per (window b, head h, query block c), with no LDS and
// no barrier.  The wave forms S^T = kr . qr^T block by block (keys as rows:
// lane (r, q) supplies kr(j0 + r, k) and qr(i0 + r, k) for k = 16u + 4q + e
// with MFMA e of a step taking element e of each float4, and receives
// S(i0 + r, j0 + 4q + e) in element e), so a query row's scores sit in the 4
// lanes r, r+16, r+32, r+48: its max and sum of exp are an in-lane reduction
// over blocks and elements, then two lane exchanges.  The same registers are
// then the A operand of P . v (k = key j0 + 4q + e), with v(j0 + 4q + e,
// 16db + r) loaded per lane as B, and P goes to global as float4 rows.  All
// global loads (q, k, v, the (cos, sin) pairs) issue before the first use,
// at clamped addresses.  Requires hd % 4 == 0, T % 4 == 0 and 16-byte aligned
// qkv, cs, P and ctx.
constexpr int kWaveJobs = 1;   // waves (jobs) per workgroup
template <int U>   // float4 groups of 16 head dims: hd <= 16 U
__global__ void __launch_bounds__(64 * kWaveJobs) attn_fwd_wave_kernel(const AttnArgs a)
{
    const int T = a.T, hd = a.hd, D = a.D, pairs = hd >> 1;
    const int nbt = (T + 15) >> 4;
    // window-major jobs, XCD-contiguous: window b's jobs share the XCD of its rows in the GEMMs
    const int job = xcd_pid(blockIdx.x, gridDim.x) * kWaveJobs + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (job >= a.B * a.H * nbt) return;
    const int c = job % nbt, bh = job / nbt, b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const int i0 = 16 * c;
    const int nj = a.causal ? c + 1 : nbt;
    const int kl = a.wlen ? min(T, a.wlen[b]) : T;
    const long long ND = static_cast<long long>(a.N) * D;
    const float* __restrict__ base = a.qkv + static_cast<long long>(b * T) * D + h * hd;
    // query row i0 + r and key rows j0 + r: U float4 of dims 16u + 4q .. +3
    const int qi = min(i0 + r, T - 1);
    float4 qv[U], qc[U], kv[4][U], kc[4][U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int g = 4 * u + q;                       // float4 index within the head
        const int gc = 4 * g < hd ? g : 0;             // past hd: loaded from column 0, zeroed below
        qv[u] = *reinterpret_cast<const float4*>(base + static_cast<long long>(qi) * D + 4 * gc);
        qc[u] = *reinterpret_cast<const float4*>(a.cs + qi * pairs + 2 * gc);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            const int kj = min(16 * jb + r, T - 1);
            kv[jb][u] = *reinterpret_cast<const float4*>(base + ND + static_cast<long long>(kj) * D + 4 * gc);
            kc[jb][u] = *reinterpret_cast<const float4*>(a.cs + kj * pairs + 2 * gc);
        }
    }
    // v(j0 + 4q + e, 16 db + r) for the output's 16-column blocks db
    float vv[4][U][4];
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int db = 0; db < U; ++db)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int j = min(16 * jb + 4 * q + e, T - 1), d = 16 * db + r;
                vv[jb][db][e] = base[2 * ND + static_cast<long long>(j) * D + (d < hd ? d : 0)];
            }
    auto rot = [](float4 x, float4 c) {
        return make_float4(x.x * c.x - x.y * c.y, x.x * c.y + x.y * c.x, x.z * c.z - x.w * c.w, x.z * c.w + x.w * c.z);
    };
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const bool in = 4 * (4 * u + q) < hd;
        qv[u] = in ? rot(qv[u], qc[u]) : make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) kv[jb][u] = in ? rot(kv[jb][u], kc[jb][u]) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    // scores of query row i0 + r against keys j0 + 4q + e, masked
    const int lim = attn_lim(i0 + r, kl, a.causal);
    float sv[4][4];
    float mx = -INFINITY;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
        floatx4 acc = {0.f, 0.f, 0.f, 0.f};
        if (jb < nj) {   // wave-uniform
#pragma unroll
            for (int u = 0; u < U; ++u) {
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[jb][u].x, qv[u].x, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[jb][u].y, qv[u].y, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[jb][u].z, qv[u].z, acc, 0, 0, 0);
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(kv[jb][u].w, qv[u].w, acc, 0, 0, 0);
            }
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * jb + 4 * q + e;
            sv[jb][e] = (jb < nj && j < lim) ? acc[e] * a.scale : -INFINITY;
            mx = fmaxf(mx, sv[jb][e]);
        }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m0 = (mx == -INFINITY || mx != mx) ? 0.f : mx;
    float sum = 0.f;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int j = 16 * jb + 4 * q + e;
            sv[jb][e] = (jb < nj && j < lim) ? expf(sv[jb][e] - m0) : 0.f;
            sum += sv[jb][e];
        }
    sum += __shfl_xor(sum, 16);
    sum += __shfl_xor(sum, 32);
    const float is = sum > 0.f ? 1.0f / sum : 1.0f;
    // P rows i0 .. i0+15 (zeros past the causal edge), float4 per lane and block
    const int row = i0 + r;
    float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T + static_cast<long long>(row) * T;
#pragma unroll
    for (int jb = 0; jb < 4; ++jb) {
#pragma unroll
        for (int e = 0; e < 4; ++e) sv[jb][e] *= is;
        const int j = 16 * jb + 4 * q;
        if (jb < nbt && row < T && j < T)
            *reinterpret_cast<float4*>(Pg + j) = make_float4(sv[jb][0], sv[jb][1], sv[jb][2], sv[jb][3]);
    }
    // ctx(i0 + 4q + e, 16 db + r) = sum_j P(i0 + 4q + e, j) v(j, 16 db + r): A = P with
    // rows r (query) and k = key, B = v
#pragma unroll
    for (int db = 0; db < U; ++db) {
        if (16 * db >= hd) continue;   // uniform (no break: the loops must unroll fully)
        floatx4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
            if (jb >= nj) continue;   // uniform
#pragma unroll
            for (int e = 0; e < 4; ++e) o = __builtin_amdgcn_mfma_f32_16x16x4f32(sv[jb][e], vv[jb][db][e], o, 0, 0, 0);
        }
        const int d = 16 * db + r;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int orow = i0 + 4 * q + e;
            if (orow < T && d < hd) a.ctx[static_cast<long long>(b * T + orow) * D + h * hd + d] = o[e];
        }
    }
}

// Backward.  Workgroup (window b, head h, block c).  With D_i = rowsum(dO o O)
// (O the forward's ctx; it equals rowsum(dP o P)), a block
// dS(i, j) = scale * P(i, j) o (dP(i, j) - D_i) needs only dP(i, j) =
// dO(i) v(j)^T and P(i, j), so the workgroup's two jobs use no other
// workgroup's results:
//   A (key block c): wave w takes query block w (w >= c when causal) and
//     forms its shares P(w, c)^T dO(w) of dv(c) and dS(w, c)^T qr(w) of dk(c);
//   B (query block c): wave w takes key block w (w <= c when causal) and
//     forms its share dS(c, w) kr(w) of dq(c).
// P and dS pass through per-wave LDS blocks into the operand layouts; the
// shares are summed in wave order by the store, which applies the inverse
// RoPE to dq and dk.
__global__ void __launch_bounds__(kAttnThreads) attn_bwd_kernel(const AttnArgs a)
{
    __shared__ float qT[kMax * kLd];                       // [d][t] rotated q
    __shared__ float kT[kMax * kLd];                       // [d][t] rotated k
    __shared__ float vs[kMax * kLd];                       // [t][d]
    __shared__ float dOs[kMax * kLd];                      // [t][d]
    __shared__ float dOT[kMax * kLd];                      // [d][t]
    __shared__ float sA[4][2][16 * kBl];                   // per wave: P(w, c), dS(w, c) [i][j]
    __shared__ float sB[4][16 * kBl];                      // per wave: dS(c, w) [i][j]
    __shared__ __align__(16) float part[3][4][16 * kLd];   // per wave: dv, dk, dq shares [row][d]
    __shared__ float Ds[kMax];
    const int T = a.T, hd = a.hd, D = a.D;
    const int T16 = round16(T), hd16 = round16(hd);
    const int nbt = T16 >> 4, nbd = hd16 >> 4, hd4 = (hd + 3) & ~3, pairs = hd >> 1;
    const int pid = xcd_pid(blockIdx.x, gridDim.x);   // window-major, XCD-contiguous (as the GEMMs' rows)
    const int c = pid % nbt, bh = pid / nbt, b = bh / a.H, h = bh - b * a.H;
    const int lane = threadIdx.x & 63, r = lane & 15, q = lane >> 4;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);   // wave-uniform: scalar branches
    const long long ND = static_cast<long long>(a.N) * D;
    const float* Pg = a.P + (static_cast<long long>(b) * a.H + h) * T * T;
    const bool actA = wave < nbt && (!a.causal || wave >= c);
    const bool actB = wave < nbt && (!a.causal || wave <= c);

    // Global loads first, all issued before the first wait (clamped addresses,
    // out-of-range values replaced after the loads):
    // P(w, c) and P(c, w) in the accumulator layout (lane (r, q), element e:
    // row 4q + e, column r of the block)
    float PA[4], PB[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int ia = 16 * wave + 4 * q + e, ja = 16 * c + r;
        const int ib = 16 * c + 4 * q + e, jb = 16 * wave + r;
        PA[e] = Pg[min(ia, T - 1) * T + min(ja, T - 1)];
        PB[e] = Pg[min(ib, T - 1) * T + min(jb, T - 1)];
        PA[e] = (actA && ia < T && ja < T) ? PA[e] : 0.f;
        PB[e] = (actB && ib < T && jb < T) ? PB[e] : 0.f;
    }
    // O and dO of row 16w + r for D: with float4 loads (vec) lane (r, q) takes
    // columns 4q + 16s .. +3, otherwise columns q + 4s
    const int trow = 16 * wave + r;
    const long long ro = static_cast<long long>(b * T + min(trow, T - 1)) * D + h * hd;
    float4 ov[kMax / 16], gv[kMax / 16];
    float os[kMax / 4], gs[kMax / 4];
    if (a.vec) {
#pragma unroll
        for (int s = 0; s < kMax / 16; ++s) {
            if (16 * s >= hd) break;                   // uniform
            const int d = min(4 * q + 16 * s, hd - 4);
            ov[s] = *reinterpret_cast<const float4*>(a.ctx + ro + d);
            gv[s] = *reinterpret_cast<const float4*>(a.dctx + ro + d);
        }
    } else {
#pragma unroll
        for (int s = 0; s < kMax / 4; ++s) {
            if (4 * s >= hd4) break;
            const int d = min(q + 4 * s, hd - 1);
            os[s] = a.ctx[ro + d];
            gs[s] = a.dctx[ro + d];
        }
    }
    // (cos, sin) of the store position (row 16c + t/16, pairs 2g, 2g + 1)
    const int si = threadIdx.x >> 4, sd = 4 * (threadIdx.x & 15), srow = 16 * c + si;
    const int spos = min(srow, T - 1), sp = min(sd >> 1, pairs - 1), sp1 = min((sd >> 1) + 1, pairs - 1);
    const float2 cs0 = a.cs[spos * pairs + sp], cs1 = a.cs[spos * pairs + sp1];
    if (a.vec) {
        Qkv4 x;
        qkv_fetch(a, b, h, x);
        // dO and dO^T (unit: row i, 4-column group g), zero padded to T16 x hd16
        constexpr int UO = kMax * (kMax / 4) / kAttnThreads;
        const int g16 = hd16 >> 2, units = T16 * g16, mg = div_magic(g16);
        float4 ovv[UO];
#pragma unroll
        for (int u = 0; u < UO; ++u) {
            if (kAttnThreads * u >= units) break;
            const int idx = threadIdx.x + kAttnThreads * u;
            const int oi = div_by(idx, mg), og = idx - oi * g16;
            ovv[u] = (oi < T && 4 * og < hd)
                         ? *reinterpret_cast<const float4*>(a.dctx + static_cast<long long>(b * T + oi) * D + h * hd + 4 * og)
                         : make_float4(0.f, 0.f, 0.f, 0.f);
        }
        qkv_put(a, x, nullptr, qT, nullptr, kT, vs, nullptr);
#pragma unroll
        for (int u = 0; u < UO; ++u) {
            if (kAttnThreads * u >= units) break;
            const int idx = threadIdx.x + kAttnThreads * u;
            const int oi = div_by(idx, mg), og = idx - oi * g16;
            if (idx < units) {
                const int d = 4 * og;
                *reinterpret_cast<float4*>(dOs + oi * kLd + d) = ovv[u];
                dOT[d * kLd + oi] = ovv[u].x; dOT[(d + 1) * kLd + oi] = ovv[u].y;
                dOT[(d + 2) * kLd + oi] = ovv[u].z; dOT[(d + 3) * kLd + oi] = ovv[u].w;
            }
        }
    } else {
        Qkv2 x;
        qkv_fetch(a, b, h, x);
        // dO and dO^T over [T16) x [hd16), zero padded
        constexpr int UO = kMax * kMax / kAttnThreads;
        float ovs[UO];
#pragma unroll
        for (int u = 0; u < UO; ++u) {
            if (kAttnThreads * u >= T16 * kMax) break;
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / kMax, j = idx - i * kMax;
            ovs[u] = (i < T && j < hd) ? a.dctx[static_cast<long long>(b * T + i) * D + h * hd + j] : 0.f;
        }
        qkv_put(a, x, nullptr, qT, nullptr, kT, vs, nullptr);
#pragma unroll
        for (int u = 0; u < UO; ++u) {
            if (kAttnThreads * u >= T16 * kMax) break;
            const int idx = threadIdx.x + kAttnThreads * u;
            const int i = idx / kMax, j = idx - i * kMax;
            if (i < T16 && j < hd16) { dOs[i * kLd + j] = ovs[u]; dOT[j * kLd + i] = ovs[u]; }
        }
    }
    // D for row 16w + r: lane (r, q) sums its columns, then the four q lanes
    float dsum = 0.f;
    if (a.vec) {
#pragma unroll
        for (int s = 0; s < kMax / 16; ++s) {
            if (16 * s >= hd) break;
            if (4 * q + 16 * s < hd)
                dsum += ov[s].x * gv[s].x + ov[s].y * gv[s].y + ov[s].z * gv[s].z + ov[s].w * gv[s].w;
        }
    } else {
#pragma unroll
        for (int s = 0; s < kMax / 4; ++s) {
            if (4 * s >= hd4) break;
            if (q + 4 * s < hd) dsum += os[s] * gs[s];
        }
    }
    dsum += __shfl_xor(dsum, 16);
    dsum += __shfl_xor(dsum, 32);
    if (q == 0 && wave < nbt) Ds[trow] = trow < T ? dsum : 0.f;
    __syncthreads();

    if (actA) {
        // dP(w, c) = dO(w) v(c)^T; dS(w, c); shares of dv(c) and dk(c)
        const floatx4 G = mfma_block(dOs + 16 * wave * kLd, kLd, 1, vs + 16 * c * kLd, kLd, 1, hd4);
        float* pa = sA[wave][0];
        float* da = sA[wave][1];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            pa[(4 * q + e) * kBl + r] = PA[e];
            da[(4 * q + e) * kBl + r] = a.scale * (PA[e] * (G[e] - Ds[16 * wave + 4 * q + e]));
        }
        wave_lds_sync();
        for (int db = 0; db < nbd; ++db) {
            const floatx4 V = mfma_block(pa, 1, kBl, dOT + 16 * db * kLd + 16 * wave, kLd, 1, 16);
            const floatx4 K = mfma_block(da, 1, kBl, qT + 16 * db * kLd + 16 * wave, kLd, 1, 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                part[0][wave][(4 * q + e) * kLd + 16 * db + r] = V[e];
                part[1][wave][(4 * q + e) * kLd + 16 * db + r] = K[e];
            }
        }
    }
    if (actB) {
        // dP(c, w) = dO(c) v(w)^T; dS(c, w); share of dq(c)
        const floatx4 G = mfma_block(dOs + 16 * c * kLd, kLd, 1, vs + 16 * wave * kLd, kLd, 1, hd4);
        float* sb = sB[wave];
#pragma unroll
        for (int e = 0; e < 4; ++e)
            sb[(4 * q + e) * kBl + r] = a.scale * (PB[e] * (G[e] - Ds[16 * c + 4 * q + e]));
        wave_lds_sync();
        for (int db = 0; db < nbd; ++db) {
            const floatx4 Q = mfma_block(sb, kBl, 1, kT + 16 * db * kLd + 16 * wave, kLd, 1, 16);
#pragma unroll
            for (int e = 0; e < 4; ++e) part[2][wave][(4 * q + e) * kLd + 16 * db + r] = Q[e];
        }
    }
    __syncthreads();
    // rows 16c .. 16c+15 of dv, dk and dq: thread (i, g) sums the shares of
    // columns 4g .. 4g+3 in wave order; dk and dq through the inverse RoPE of
    // the pairs (4g, 4g+1) and (4g+2, 4g+3)
    if (srow < T && sd < hd) {
        const int a0 = a.causal ? c : 0, b1 = a.causal ? c + 1 : nbt;
        float4 sv = make_float4(0.f, 0.f, 0.f, 0.f), sk = sv, sq = sv;
        for (int w = a0; w < nbt; ++w) {
            const float4 tv = *reinterpret_cast<const float4*>(&part[0][w][si * kLd + sd]);
            const float4 tk = *reinterpret_cast<const float4*>(&part[1][w][si * kLd + sd]);
            sv.x += tv.x; sv.y += tv.y; sv.z += tv.z; sv.w += tv.w;
            sk.x += tk.x; sk.y += tk.y; sk.z += tk.z; sk.w += tk.w;
        }
        for (int w = 0; w < b1; ++w) {
            const float4 tq = *reinterpret_cast<const float4*>(&part[2][w][si * kLd + sd]);
            sq.x += tq.x; sq.y += tq.y; sq.z += tq.z; sq.w += tq.w;
        }
        const float4 dk = make_float4(sk.x * cs0.x + sk.y * cs0.y, -sk.x * cs0.y + sk.y * cs0.x,
                                      sk.z * cs1.x + sk.w * cs1.y, -sk.z * cs1.y + sk.w * cs1.x);
        const float4 dq = make_float4(sq.x * cs0.x + sq.y * cs0.y, -sq.x * cs0.y + sq.y * cs0.x,
                                      sq.z * cs1.x + sq.w * cs1.y, -sq.z * cs1.y + sq.w * cs1.x);
        float* o = a.dqkv + static_cast<long long>(b * T + srow) * D + h * hd + sd;
        if (a.vec) {
            *reinterpret_cast<float4*>(o) = dq;
            *reinterpret_cast<float4*>(o + ND) = dk;
            *reinterpret_cast<float4*>(o + 2 * ND) = sv;
        } else {
            o[0] = dq.x; o[1] = dq.y; o[ND] = dk.x; o[ND + 1] = dk.y; o[2 * ND] = sv.x; o[2 * ND + 1] = sv.y;
            if (sd + 2 < hd) {
                o[2] = dq.z; o[3] = dq.w; o[ND + 2] = dk.z; o[ND + 3] = dk.w; o[2 * ND + 2] = sv.z; o[2 * ND + 3] = sv.w;
            }
        }
    }
}

}  // namespace

bool attn_fused_ok(int T, int hd) { return T >= 1 && T <= kMax && hd >= 2 && hd <= kMax && hd % 2 == 0; }

int attn_fwd(const float* qkv, const float2* cs, float* P, float* ctx, int B, int H, int T, int hd, float scale,
             int causal, hipStream_t s, const int* wlen)
{
    if (!attn_fused_ok(T, hd)) return fail(LHIP_E_UNSUPPORTED, "attn_fwd: T=%d hd=%d outside the fused limits", T, hd);
    if (!qkv || !cs || !P || !ctx) return fail(LHIP_E_NULL, "attn_fwd: NULL argument");
    AttnArgs a{};
    a.qkv = qkv; a.cs = cs; a.P = P; a.ctx = ctx;
    a.B = B; a.H = H; a.T = T; a.hd = hd; a.D = H * hd; a.N = B * T;
    a.scale = scale; a.causal = causal; a.wlen = wlen;
    a.vec = (hd % 4 == 0 && aligned16(qkv) && aligned16(cs)) ? 1 : 0;
    a.vec = a.vec && aligned16(ctx);
    const int jobs = B * H * ((T + 15) / 16);
    if (a.vec && T % 4 == 0 && aligned16(P)) {   // one wave per (window, head, query block)
        const unsigned grid = static_cast<unsigned>((jobs + kWaveJobs - 1) / kWaveJobs);
        if (hd <= 16) klaunch(attn_fwd_wave_kernel<1>, grid, 64 * kWaveJobs, 0, s, a);
        else if (hd <= 32) klaunch(attn_fwd_wave_kernel<2>, grid, 64 * kWaveJobs, 0, s, a);
        else if (hd <= 48) klaunch(attn_fwd_wave_kernel<3>, grid, 64 * kWaveJobs, 0, s, a);
        else klaunch(attn_fwd_wave_kernel<4>, grid, 64 * kWaveJobs, 0, s, a);
        return check_launch("attn_fwd");
    }
    klaunch(attn_fwd_kernel, jobs, kAttnThreads, 0, s, a);
    return check_launch("attn_fwd");
}

int attn_bwd(const float* qkv, const float2* cs, const float* P, const float* ctx, const float* dctx, float* dqkv, int B,
             int H, int T, int hd, float scale, int causal, hipStream_t s)
{
    if (!attn_fused_ok(T, hd)) return fail(LHIP_E_UNSUPPORTED, "attn_bwd: T=%d hd=%d outside the fused limits", T, hd);
    if (!qkv || !cs || !P || !ctx || !dctx || !dqkv) return fail(LHIP_E_NULL, "attn_bwd: NULL argument");
    AttnArgs a{};
    a.qkv = qkv; a.cs = cs; a.P = const_cast<float*>(P); a.ctx = const_cast<float*>(ctx); a.dctx = dctx; a.dqkv = dqkv;
    a.B = B; a.H = H; a.T = T; a.hd = hd; a.D = H * hd; a.N = B * T;
    a.scale = scale; a.causal = causal;
    // the float4 path also reads ctx (the forward's O, for rowsum(dO*O))
    a.vec = (hd % 4 == 0 && aligned16(qkv) && aligned16(cs) && aligned16(ctx) && aligned16(dctx) &&
             aligned16(dqkv)) ? 1 : 0;
    klaunch(attn_bwd_kernel, B * H * ((T + 15) / 16), kAttnThreads, 0, s, a);
    return check_launch("attn_bwd");
}

}  // namespace lhip
