// lhip_gemm.hip -- fp32 GEMM family on CDNA4 matrix cores (v_mfma_f32_32x32x2f32).
//
// C = alpha * op(A) * op(B) + beta * C, row-major, op = identity or transpose.
// Serves the three products of the reference's strided luaTL_gemm_ex
// (cuda/luaTL_train.cu:1075-1094 -> luaTL_gemm_ex_launch 391-476): A.B for the
// forward, A.B^T (matmul_dx) and A^T.B (matmul_dw) for the backward
// (ai/gpu/luaTL_train.lua:154-182), and the host-table products of
// ai/core/matrix.lua (multiply :541, matmul_nt :597, matmul_tn :627).
//
// Design (gfx950):
//   * a workgroup of 4 wave64s computes a BM x BN tile; each wave owns a
//     (BM/2) x (BN/2) sub-tile made of 32x32 MFMA blocks whose accumulators
//     stay in registers for the whole K loop;
//   * both operands are staged in LDS K-major (As[k][m], Bs[k][n]) so that one
//     MFMA operand fetch is a single ds_read_b32 in which lanes 0-31 read 32
//     consecutive floats of row k and lanes 32-63 those of row k+1 -- exactly
//     the A (32x2) / B (2x32) fragment layout of v_mfma_f32_32x32x2f32;
//   * global->LDS loads are 128-bit and coalesced along the contiguous
//     dimension of each operand; a transposed operand is transposed on the
//     LDS write (4 ds_write_b32 per float4), never by a separate pass; the
//     transposing stores use an odd LDS row stride so that the 32 lanes of a
//     half-wave hit 32 distinct banks;
//   * two LDS buffers: the next K tile is fetched into registers while the
//     current one feeds the MFMAs, one barrier per K tile;
//   * workgroup ids are remapped so that consecutive tiles of a row band land
//     on the same XCD (blocks are dispatched round-robin over the 8 XCDs, each
//     with its own L2), then grouped GROUP_M bands at a time for L2 reuse.
// Edge tiles (any M, N, K) use bounds-checked scalar loads with zero fill and
// checked stores; unaligned operands (ld % 4 != 0 or a base not 16-byte
// aligned) always take the scalar path.
#include <algorithm>
#include <type_traits>

#include "lhip_internal.h"
#include "lhip_reduce.h"

namespace lhip {
namespace {

typedef float floatx16 __attribute__((ext_vector_type(16)));
typedef float floatx4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;  // 4 wave64s
constexpr int kSmallU = 8;     // K steps whose loads the small kernel issues together

// Loads a ROWS x COLS tile of a row-major matrix into registers, float4 per
// thread per pass, consecutive threads walking the contiguous dimension.
template <int ROWS, int COLS>
struct TileRegs {
    static constexpr int CQ = COLS / 4;            // float4s per tile row
    static constexpr int RPP = kThreads / CQ;      // tile rows per pass
    static constexpr int PASSES = ROWS / RPP;
    static_assert(COLS % 4 == 0 && kThreads % CQ == 0 && ROWS % RPP == 0, "tile/thread mismatch");
    float4 v[PASSES];

    __device__ __forceinline__ void load(const float* __restrict__ g, int ld, int r0, int c0,
                                         int rmax, int cmax, bool vec, int tid)
    {
        const int cq = tid % CQ;
        const int rr = tid / CQ;
        const int gc = c0 + 4 * cq;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int gr = r0 + rr + p * RPP;
            const float* src = g + static_cast<long long>(gr) * ld + gc;
            if (vec && gr < rmax && gc + 3 < cmax) {
                v[p] = *reinterpret_cast<const float4*>(src);
            } else {
                const bool rok = gr < rmax;
                v[p].x = (rok && gc + 0 < cmax) ? src[0] : 0.f;
                v[p].y = (rok && gc + 1 < cmax) ? src[1] : 0.f;
                v[p].z = (rok && gc + 2 < cmax) ? src[2] : 0.f;
                v[p].w = (rok && gc + 3 < cmax) ? src[3] : 0.f;
            }
        }
    }

    // Every element in bounds and the stored rows 16-byte aligned: one
    // unconditional float4 load per pass (no branch for a wait to be
    // conservative about).
    // Rows past rmax and columns past cmax (cmax % 4 == 0) are clamped into
    // the operand: they only reach outputs that are not stored.
    __device__ __forceinline__ void load_full(const float* __restrict__ g, int ld, int r0, int c0, int rmax, int cmax,
                                              int tid)
    {
        const int cq = tid % CQ;
        const int rr = tid / CQ;
        const int c = min(c0 + 4 * cq, cmax - 4);
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int r = min(r0 + rr + p * RPP, rmax - 1);
            const float4 t = *reinterpret_cast<const float4*>(g + static_cast<long long>(r) * ld + c);
            v[p].x = t.x; v[p].y = t.y; v[p].z = t.z; v[p].w = t.w;   // per component: stays in VGPRs
        }
    }

    // Store as lds[row][col] (tile orientation kept; LD % 4 == 0).
    template <int LD>
    __device__ __forceinline__ void store_direct(float* lds, int tid) const
    {
        const int cq = tid % CQ;
        const int rr = tid / CQ;
#pragma unroll
        for (int p = 0; p < PASSES; ++p)
            *reinterpret_cast<float4*>(lds + (rr + p * RPP) * LD + 4 * cq) = v[p];
    }

    // Store transposed as lds[col][row].
    template <int LD>
    __device__ __forceinline__ void store_transposed(float* lds, int tid) const
    {
        const int cq = tid % CQ;
        const int rr = tid / CQ;
#pragma unroll
        for (int p = 0; p < PASSES; ++p) {
            const int r = rr + p * RPP;
            lds[(4 * cq + 0) * LD + r] = v[p].x;
            lds[(4 * cq + 1) * LD + r] = v[p].y;
            lds[(4 * cq + 2) * LD + r] = v[p].z;
            lds[(4 * cq + 3) * LD + r] = v[p].w;
        }
    }
};

// Map the linear workgroup id to a (tile_m, tile_n) pair: XCD-contiguous
// chunks, then GROUP_M-row-band grouped raster inside the chunk order.
__device__ __forceinline__ void tile_coords(int pid, int nwg, int tiles_m, int tiles_n, int& tm, int& tn)
{
    constexpr int kXcds = 8;
    constexpr int kGroupM = 8;
    if ((nwg % kXcds) == 0) pid = (pid % kXcds) * (nwg / kXcds) + pid / kXcds;
    const int per_group = kGroupM * tiles_n;
    const int group = pid / per_group;
    const int first_m = group * kGroupM;
    const int gsz = min(tiles_m - first_m, kGroupM);
    const int in_group = pid - group * per_group;
    tm = first_m + in_group % gsz;
    tn = in_group / gsz;
}

// Kernel arguments (one struct: the launch passes it by value).
struct GemmArgs {
    int M, N, K;
    float alpha, beta;
    const float* A; int lda; long long sA, sA2;
    const float* B; int ldb; long long sB, sB2;
    float* C; int ldc; long long sC, sC2;
    const float* R; int ldr;          // the beta term reads R (R == C unless a residual is given)
    int tiles_m, tiles_n, vecA, vecB, inner;
    int splits, kchunk;               // split-K: blockIdx.z = slice, K range [z*kchunk, (z+1)*kchunk)
    float* ws;                        // split-K partials [split][batch][M][N]
    int Kb;                           // batch-reduce: K = kblocks * Kb, block j reads A + j*sAk, B + j*sBk
    long long sAk, sBk;
    int skip_reduce;                  // split-K slices stay in ws for the caller to sum
    size_t ws_floats_avail;           // floats available at ws (skinny path's split plan)
};

// C = alpha * sum_s ws[s] + beta * R, the slices summed in order (deterministic).
__global__ void __launch_bounds__(256)
splitk_reduce(const GemmArgs g, int batch)
{
    const long long mn = static_cast<long long>(g.M) * g.N;
    const long long total = mn * batch;
    const long long pstride = mn * batch;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    for (long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; idx < total; idx += stride) {
        const long long z = idx / mn, rc = idx - z * mn;
        const int row = static_cast<int>(rc / g.N), col = static_cast<int>(rc - static_cast<long long>(row) * g.N);
        float sum = 0.f;
        const float* src = g.ws + idx;
        for (int p = 0; p < g.splits; ++p) sum += src[p * pstride];
        const long long coff = (z / g.inner) * g.sC2 + (z % g.inner) * g.sC;
        float* dst = g.C + coff + static_cast<long long>(row) * g.ldc + col;
        const float v = g.alpha * sum;
        if (g.beta != 0.f) {
            const float* r = g.R ? g.R + coff + static_cast<long long>(row) * g.ldr + col : dst;
            *dst = v + g.beta * (*r);
        } else {
            *dst = v;
        }
    }
}

// Float4 form of splitk_reduce for batch 1 (N % 4 == 0, ldc % 4 == 0 and
// 16-byte aligned C, R): four columns per thread, the slices' loads issued
// eight at a time, summed in slice order.
__global__ void __launch_bounds__(256)
splitk_reduce4(const GemmArgs g)
{
    const long long mn4 = static_cast<long long>(g.M) * g.N / 4;
    const long long stride = static_cast<long long>(gridDim.x) * blockDim.x;
    const int n4 = g.N / 4;
    for (long long idx = blockIdx.x * static_cast<long long>(blockDim.x) + threadIdx.x; idx < mn4; idx += stride) {
        const int row = static_cast<int>(idx / n4), col = 4 * static_cast<int>(idx - static_cast<long long>(row) * n4);
        const float4* src = reinterpret_cast<const float4*>(g.ws) + idx;
        float4 sum = make_float4(0.f, 0.f, 0.f, 0.f);
        int p = 0;
        for (; p + 8 <= g.splits; p += 8) {
            float4 t[8];
#pragma unroll
            for (int u = 0; u < 8; ++u) t[u] = src[(p + u) * mn4];
#pragma unroll
            for (int u = 0; u < 8; ++u) { sum.x += t[u].x; sum.y += t[u].y; sum.z += t[u].z; sum.w += t[u].w; }
        }
        for (; p < g.splits; ++p) {
            const float4 t = src[p * mn4];
            sum.x += t.x; sum.y += t.y; sum.z += t.z; sum.w += t.w;
        }
        float4* dst = reinterpret_cast<float4*>(g.C + static_cast<long long>(row) * g.ldc + col);
        float4 v = make_float4(g.alpha * sum.x, g.alpha * sum.y, g.alpha * sum.z, g.alpha * sum.w);
        if (g.beta != 0.f) {
            const float4 r = g.R ? *reinterpret_cast<const float4*>(g.R + static_cast<long long>(row) * g.ldr + col) : *dst;
            v.x += g.beta * r.x; v.y += g.beta * r.y; v.z += g.beta * r.z; v.w += g.beta * r.w;
        }
        *dst = v;
    }
}

template <int BM, int BN, int BK, bool TA, bool TB>
__global__ void __launch_bounds__(kThreads)
sgemm_mfma_kernel(const GemmArgs g)
{
    constexpr int WM = BM / 2, WN = BN / 2;        // 2x2 waves
    constexpr int FM = WM / 32, FN = WN / 32;      // 32x32 MFMA blocks per wave
    static_assert(FM >= 1 && FN >= 1 && BK % 2 == 0, "bad tile");
    // K-major LDS tiles.  Transposing stores want an odd row stride; direct
    // float4 stores want a multiple of 4.
    constexpr int LDA = TA ? BM + 4 : BM + 1;
    constexpr int LDB = TB ? BN + 1 : BN + 4;
    __shared__ float As[2][BK * LDA];
    __shared__ float Bs[2][BK * LDB];

    const int M = g.M, N = g.N;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 31;   // row (A) / column (B) inside a 32-wide fragment
    const int lk = lane >> 5;   // which of the two k of an MFMA step

    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    // two-level batch: z = outer * inner + inner_index (e.g. window x head)
    const long long zo = blockIdx.y / g.inner, zi = blockIdx.y % g.inner;
    const float* __restrict__ A = g.A + zo * g.sA2 + zi * g.sA;
    const float* __restrict__ B = g.B + zo * g.sB2 + zi * g.sB;
    const long long coff = zo * g.sC2 + zi * g.sC;

    const int wm = (wave >> 1) * WM;
    const int wn = (wave & 1) * WN;

    // op(A) tile is BM x BK: rows m, cols k.  Stored (!TA) M x K -> tile (m, k);
    // stored (TA) K x M -> tile (k, m).
    TileRegs<TA ? BK : BM, TA ? BM : BK> ra;
    // op(B) tile is BK x BN.  Stored (!TB) K x N -> tile (k, n); (TB) N x K -> tile (n, k).
    TileRegs<TB ? BN : BK, TB ? BK : BN> rb;

    // split-K: this workgroup reduces k in [kbeg, kend) (kchunk = K when unsplit)
    const int kbeg = blockIdx.z * g.kchunk;
    const int kend = min(g.K, kbeg + g.kchunk);
    auto gload = [&](int k0) {
        if (TA) ra.load(A, g.lda, k0, m0, kend, M, g.vecA, tid);
        else    ra.load(A, g.lda, m0, k0, M, kend, g.vecA, tid);
        if (TB) rb.load(B, g.ldb, n0, k0, N, kend, g.vecB, tid);
        else    rb.load(B, g.ldb, k0, n0, kend, N, g.vecB, tid);
    };
    auto lstore = [&](int buf) {
        if (TA) ra.template store_direct<LDA>(As[buf], tid);
        else    ra.template store_transposed<LDA>(As[buf], tid);
        if (TB) rb.template store_transposed<LDB>(Bs[buf], tid);
        else    rb.template store_direct<LDB>(Bs[buf], tid);
    };

    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    if (nk > 0) {
        gload(kbeg);
        lstore(0);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload(kbeg + (kt + 1) * BK);
        const float* as = As[cur];
        const float* bs = Bs[cur];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = as[(kk + lk) * LDA + wm + 32 * i + lr];
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = bs[(kk + lk) * LDB + wn + 32 * j + lr];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
        if (more) lstore(cur ^ 1);
        __syncthreads();
    }

    // Accumulator layout of a 32x32 block: element r of lane l sits at
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    if (g.splits > 1) {
        // split-K partial of this slice: dense [split][batch][M][N], summed in
        // slice order by splitk_reduce (a second launch: a device-scope fence
        // inside this kernel would have to write back the per-XCD L2)
        float* wz = g.ws + (static_cast<long long>(blockIdx.z) * gridDim.y + blockIdx.y) *
                               (static_cast<long long>(M) * N);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = n0 + wn + 32 * j + lr;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
                    if (row < M) wz[static_cast<long long>(row) * N + col] = acc[i][j][r];
                }
            }
        return;
    }
    float* __restrict__ C = g.C + coff;
    const float* R = g.R ? g.R + coff : C;
    const int ldr = g.R ? g.ldr : g.ldc;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn + 32 * j + lr;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (row < M) {
                    const float v = g.alpha * acc[i][j][r];
                    C[static_cast<long long>(row) * g.ldc + col] =
                        (g.beta != 0.f) ? v + g.beta * R[static_cast<long long>(row) * ldr + col] : v;
                }
            }
        }
}

// sgemm_mfma_kernel with KS wave sets per workgroup (KS * 256 threads): set
// s takes the K chunks s, s+KS, ... with its own double-buffered LDS, so each
// SIMD holds KS waves and each set's chain of dependent chunk loads is KS
// times shorter; the sets' partial tiles meet in LDS (fixed order).  For long
// K on one or two 64x64 tiles per CU (1024^3: 29.1, 28.9-29.1 and 27.6-27.7 us
// on one, four and two wave sets; split-K slices take four).  PF = 2: two
// register sets per wave set, so chunk kt + 2 KS is in flight while chunk kt
// runs and chunk kt + KS goes to LDS.
template <int BM, int BN, int BK, bool TA, bool TB, int KS, int PF = 1, bool FULL = false>
__global__ void __launch_bounds__(kThreads * KS)
sgemm_mfma_ks_kernel(const GemmArgs g)
{
    constexpr int WM = BM / 2, WN = BN / 2;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int LDA = TA ? BM + 4 : BM + 1;
    constexpr int LDB = TB ? BN + 1 : BN + 4;
    __shared__ float As[KS][2][BK * LDA];
    __shared__ float Bs[KS][2][BK * LDB];
    const int M = g.M, N = g.N;
    const int tid = threadIdx.x;
    const int grp = __builtin_amdgcn_readfirstlane(tid >> 8), gt = tid & 255;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int lr = lane & 31, lk = lane >> 5;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const long long zo = blockIdx.y / g.inner, zi = blockIdx.y % g.inner;
    const float* __restrict__ A = g.A + zo * g.sA2 + zi * g.sA;
    const float* __restrict__ B = g.B + zo * g.sB2 + zi * g.sB;
    const long long coff = zo * g.sC2 + zi * g.sC;
    const int wm = (wave >> 1) * WM, wn = (wave & 1) * WN;
    TileRegs<TA ? BK : BM, TA ? BM : BK> ra, ra2;
    TileRegs<TB ? BN : BK, TB ? BK : BN> rb, rb2;
    const int kbeg = blockIdx.z * g.kchunk;
    const int kend = min(g.K, kbeg + g.kchunk);
    auto gload_to = [&](auto& xa, auto& xb, int k0) {
        if constexpr (FULL) {
            // K is whole chunks; M and N are clamped (M % 4 == 0 when A is
            // stored K-major, N % 4 == 0 when B is)
            if (TA) xa.load_full(A, g.lda, k0, m0, kend, M, gt);
            else    xa.load_full(A, g.lda, m0, k0, M, kend, gt);
            if (TB) xb.load_full(B, g.ldb, n0, k0, N, kend, gt);
            else    xb.load_full(B, g.ldb, k0, n0, kend, N, gt);
        } else {
            if (TA) xa.load(A, g.lda, k0, m0, kend, M, g.vecA, gt);
            else    xa.load(A, g.lda, m0, k0, M, kend, g.vecA, gt);
            if (TB) xb.load(B, g.ldb, n0, k0, N, kend, g.vecB, gt);
            else    xb.load(B, g.ldb, k0, n0, kend, N, g.vecB, gt);
        }
    };
    auto lstore_from = [&](const auto& xa, const auto& xb, int buf) {
        if (TA) xa.template store_direct<LDA>(As[grp][buf], gt);
        else    xa.template store_transposed<LDA>(As[grp][buf], gt);
        if (TB) xb.template store_transposed<LDB>(Bs[grp][buf], gt);
        else    xb.template store_direct<LDB>(Bs[grp][buf], gt);
    };
    auto gload = [&](int k0) { gload_to(ra, rb, k0); };
    auto lstore = [&](int buf) { lstore_from(ra, rb, buf); };
    floatx16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int iters = (nk + KS - 1) / KS;
    auto mma = [&](int cur) {
        const float* as = As[grp][cur];
        const float* bs = Bs[grp][cur];
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float a[FM], b[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) a[i] = as[(kk + lk) * LDA + wm + 32 * i + lr];
#pragma unroll
            for (int j = 0; j < FN; ++j) b[j] = bs[(kk + lk) * LDB + wn + 32 * j + lr];
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(a[i], b[j], acc[i][j], 0, 0, 0);
        }
    };
    // FULL: every chunk load is unconditional (past the last chunk a set
    // reloads the last one, which it never stores), so the wait before an LDS
    // store counts only the loads of the chunk being stored; a set with no
    // chunk stores and reads only its own LDS, and adds a zero tile
    if (FULL) gload(kbeg + min(grp, nk - 1) * BK);
    else if (grp < nk) gload(kbeg + grp * BK);
    else { ra = decltype(ra){}; rb = decltype(rb){}; }
    if constexpr (PF == 2) {
        // two register sets: chunk kt + 2 KS is loaded while chunk kt runs its
        // MFMAs and chunk kt + KS (loaded one iteration earlier) goes to LDS
        if (FULL) gload_to(ra2, rb2, kbeg + min(grp + KS, nk - 1) * BK);
        else if (grp + KS < nk) gload_to(ra2, rb2, kbeg + (grp + KS) * BK);
        lstore(0);
        __syncthreads();
        // the register sets are picked at compile time (a run-time choice
        // between them would put both in scratch memory)
        auto body = [&](int it, auto setc) {
            constexpr int L = decltype(setc)::value;   // the set loaded; the other is stored
            auto& la = L == 0 ? ra : ra2;
            auto& lb = L == 0 ? rb : rb2;
            const auto& sa = L == 0 ? ra2 : ra;
            const auto& sb = L == 0 ? rb2 : rb;
            const int cur = it & 1;
            const int kt = it * KS + grp;
            if (FULL) gload_to(la, lb, kbeg + min(kt + 2 * KS, nk - 1) * BK);
            else if (kt + 2 * KS < nk) gload_to(la, lb, kbeg + (kt + 2 * KS) * BK);
            if (kt < nk) mma(cur);
            if (kt + KS < nk) lstore_from(sa, sb, cur ^ 1);
            __syncthreads();
        };
        // FULL: no branch around the second body (past the last iteration it
        // only reloads the last chunk; its MFMAs and LDS store are skipped),
        // so every path through the loop has the same loads in flight and each
        // LDS store waits for its own chunk alone; behind the branch the
        // compiler made the stores wait for the next chunk's loads as well
        // (tied head 512x2000x128 NT 7.04 -> 6.88 us, 512x2048x1024 27.05 ->
        // 26.71; a third register set, chunks three ahead, was 8-15% slower)
        for (int it = 0; it < iters; it += 2) {
            body(it, std::integral_constant<int, 0>{});
            if (FULL || it + 1 < iters) body(it + 1, std::integral_constant<int, 1>{});
        }
    } else {
        lstore(0);
        __syncthreads();
        for (int it = 0; it < iters; ++it) {
            const int cur = it & 1;
            const int kt = it * KS + grp;
            const bool more = it + 1 < iters;
            const bool next_in = kt + KS < nk;
            if (FULL) gload(kbeg + min(kt + KS, nk - 1) * BK);
            else if (more && next_in) gload(kbeg + (kt + KS) * BK);
            if (kt < nk) mma(cur);
            if (more && next_in) lstore(cur ^ 1);
            __syncthreads();
        }
    }
    constexpr int SZ = 4 * FM * FN * 1024;   // one set's partial tiles (floats)
    static_assert(KS == 1 || (KS - 1) * SZ <= KS * 2 * BK * LDA, "reduction area");
    float* red = &As[0][0][0];   // sets 1..KS-1 leave their partial tiles here
    if (grp > 0) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    red[(grp - 1) * SZ + ((wave * FM + i) * FN + j) * 1024 + r * 64 + lane] = acc[i][j][r];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int t = 1; t < KS; ++t)   // in set order
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] += red[(t - 1) * SZ + ((wave * FM + i) * FN + j) * 1024 + r * 64 + lane];
    // Accumulator layout of a 32x32 block: element r of lane l sits at
    // row 8*(r/4) + 4*(l/32) + r%4, column l%32.
    if (g.splits > 1) {   // split-K partial of this slice, summed by splitk_reduce
        float* wz = g.ws + (static_cast<long long>(blockIdx.z) * gridDim.y + blockIdx.y) *
                               (static_cast<long long>(M) * N);
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = n0 + wn + 32 * j + lr;
                if (col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
                    if (row < M) wz[static_cast<long long>(row) * N + col] = acc[i][j][r];
                }
            }
        return;
    }
    float* __restrict__ C = g.C + coff;
    const float* R = g.R ? g.R + coff : C;
    const int ldr = g.R ? g.ldr : g.ldc;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn + 32 * j + lr;
            if (col >= N) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * lk + (r & 3);
                if (row < M) {   // streamed out, not left dirty in L2 for the kernel's end
                    const float v = g.alpha * acc[i][j][r];
                    __builtin_nontemporal_store(
                        (g.beta != 0.f) ? v + g.beta * R[static_cast<long long>(row) * ldr + col] : v,
                        &C[static_cast<long long>(row) * g.ldc + col]);
                }
            }
        }
}

// ---------------------------------------------------------------------------
// Large problems (at least one 256x256 tile per CU): 256x256 output tiles,
// four waves of 128x128 (16 v_mfma_f32_32x32x2f32 accumulators each, 256
// AGPRs, one wave per SIMD), 32-deep K tiles double-buffered in LDS (128 KB).
//
// Both LDS tiles are k-contiguous: As[m][k], Bs[n][k], 32 floats (8 quads of
// 4 k) per row, quad q of row r stored at quad position q ^ swz(r) with
// swz(r) = (r ^ (r >> 3)) & 7.  For an 8-deep K step at k0, lane l (row or
// column r = l%32 of a 32-block, half h = l/32) fetches op(A)[r][k0+4h ..
// k0+4h+3] and op(B)[k0+4h .. +3][c] with one ds_read_b128 each; MFMA t of
// the step multiplies element t of both, so its two k slots are k0+t and
// k0+4+t and the four MFMAs cover k0 .. k0+7 once.  A wave thus reads 8 b128
// per 64 MFMAs.  The swizzle maps any 8 rows 8m .. 8m+7 (one 8-lane phase of
// those reads) and any 8 rows 32m + 4j + c, j = 0..7 (a phase of the
// transposed writes below) to 8 distinct quad positions: both are free of
// bank conflicts.
//
// Global -> LDS, float4 loads along the stored contiguous dimension:
//  - operand stored k-contiguous (A when !TA, B when TB): 8 lanes read one
//    row's 32 k, written as they are (ds_write_b128);
//  - operand stored K-major (A when TA, B when !TB): a lane reads a 4 k x 4
//    column block (4 float4 from 4 k-rows, 64 lanes = 1 KB of a row per
//    instruction) and writes it transposed: column c's 4 k as one b128.
__device__ __forceinline__ float f4get(const float4& v, int t)
{
    return t == 0 ? v.x : t == 1 ? v.y : t == 2 ? v.z : v.w;   // t is a compile-time constant after unrolling
}

constexpr int kBig = 256;
constexpr int kBigK = 32;
constexpr int kLd256 = kBigK;        // floats per LDS row (quad-swizzled, no padding)
constexpr int kBigQ = kBigK / 4;     // k quads per row of a tile
constexpr int kBigLds = kBig * kLd256;

__device__ __forceinline__ int big_swz(int row) { return (row ^ (row >> 3)) & 7; }

template <bool KMAJOR, bool FULL, int ROWS = kBig>
struct BigTileRegs {
    // ROWS rows (m or n) x kBigK k of one operand: NS float4 per thread
    static constexpr int NS = ROWS * kBigK / 4 / kThreads;
    static constexpr int CQ = ROWS / 4;              // KMAJOR: column quads of a k row
    static constexpr int KQS = kThreads / CQ;        // KMAJOR: k quads per slot block
    static_assert(NS % 4 == 0 && kThreads % CQ == 0, "tile rows");
    float4 v[NS];

    // stored: element (row, k) at X[row * ld + k] (!KMAJOR) or X[k * ld + row] (KMAJOR).
    // Slot s (0 .. NS-1) is one float4 load:
    // !KMAJOR: row tid/8 + 32s, k quad tid%8;
    // KMAJOR: k row 4kq + s%4 of block (columns 4(tid%CQ) .. +3, k quad kq = tid/CQ + KQS(s/4)).
    // The slots are loaded and stored one at a time so that the main loop can
    // spread them between MFMA groups; a KMAJOR store slot needs the four
    // load slots of its block.
    __device__ __forceinline__ void load_slot(int s, const float* __restrict__ X, int ld, int r0, int k0, int rmax,
                                              int kmax, bool vec, int tid)
    {
        int gr, gk;
        const float* src;
        if (!KMAJOR) {
            gr = r0 + tid / kBigQ + (kThreads / kBigQ) * s;
            gk = k0 + 4 * (tid % kBigQ);
            src = X + static_cast<long long>(gr) * ld + gk;
        } else {
            gr = r0 + 4 * (tid % CQ);
            gk = k0 + 4 * (tid / CQ + KQS * (s >> 2)) + (s & 3);
            src = X + static_cast<long long>(gk) * ld + gr;
        }
        // the 4 contiguous elements: (row gr, k gk..gk+3) or (k gk, columns gr..gr+3)
        const int lim = KMAJOR ? rmax - gr : kmax - gk;
        const bool lineok = KMAJOR ? gk < kmax : gr < rmax;
        if (FULL || (vec && lineok && lim >= 4)) {
            const float4 t = *reinterpret_cast<const float4*>(src);
            v[s].x = t.x; v[s].y = t.y; v[s].z = t.z; v[s].w = t.w;   // per component: stays in VGPRs
        } else {
            v[s].x = (lineok && lim > 0) ? src[0] : 0.f;
            v[s].y = (lineok && lim > 1) ? src[1] : 0.f;
            v[s].z = (lineok && lim > 2) ? src[2] : 0.f;
            v[s].w = (lineok && lim > 3) ? src[3] : 0.f;
        }
    }

    __device__ __forceinline__ void store_slot(int s, float* lds, int tid) const
    {
        if (!KMAJOR) {
            const int row = tid / kBigQ + (kThreads / kBigQ) * s;
            *reinterpret_cast<float4*>(lds + row * kLd256 + 4 * ((tid % kBigQ) ^ big_swz(row))) = v[s];
        } else {
            // column 4(tid%CQ) + s%4 of block s/4: its four k from the block's four loads
            const int b = s >> 2, c = s & 3;
            const int row = 4 * (tid % CQ) + c;
            const int kq = tid / CQ + KQS * b;
            const float4 t = make_float4(f4get(v[4 * b + 0], c), f4get(v[4 * b + 1], c), f4get(v[4 * b + 2], c),
                                         f4get(v[4 * b + 3], c));
            *reinterpret_cast<float4*>(lds + row * kLd256 + 4 * (kq ^ big_swz(row))) = t;
        }
    }
};

// FULL: M and N multiples of TILE, K of kBigK, k-contiguous operands 16-byte
// aligned -- every tile load is in bounds and unconditional.  TILE = 128 is
// the same kernel on 128x128 tiles (four waves of 64x64, 4 accumulators each,
// 64 KB of LDS: two workgroups per CU), for problems with fewer 256x256 tiles
// than CUs but many 128x128 ones.
template <bool TA, bool TB, bool FULL, int TILE = kBig>
__global__ void __launch_bounds__(kThreads)
sgemm_256_kernel(const GemmArgs g)
{
    constexpr int F = TILE / 64;   // 32x32 blocks per wave and dimension
    constexpr int LDS = TILE * kLd256;
    __shared__ float As[2][LDS];
    __shared__ float Bs[2][LDS];
    const int M = g.M, N = g.N;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 31;
    const int h = lane >> 5;
    int tm, tn;
    tile_coords(blockIdx.x, gridDim.x, g.tiles_m, g.tiles_n, tm, tn);
    const int m0 = tm * TILE, n0 = tn * TILE;
    const long long zo = blockIdx.y / g.inner, zi = blockIdx.y % g.inner;
    // split-K: this workgroup takes k in [kbeg, kbeg + K); the operands are
    // offset to the slice start (k runs along a stored row of A when !TA and
    // of B when TB, down the stored columns otherwise)
    const int kbeg = blockIdx.z * g.kchunk;
    const int K = min(g.K, kbeg + g.kchunk) - kbeg;
    const float* __restrict__ A = g.A + zo * g.sA2 + zi * g.sA + (TA ? static_cast<long long>(kbeg) * g.lda : kbeg);
    const float* __restrict__ B = g.B + zo * g.sB2 + zi * g.sB + (TB ? kbeg : static_cast<long long>(kbeg) * g.ldb);
    const long long coff = zo * g.sC2 + zi * g.sC;
    const int wm = (wave >> 1) * (TILE / 2), wn = (wave & 1) * (TILE / 2);

    BigTileRegs<TA, FULL, TILE> ra;    // op(A): row m; stored M x K (!TA) or K x M (TA)
    BigTileRegs<!TB, FULL, TILE> rb;   // op(B): row n; stored N x K (TB) or K x N (!TB)
    constexpr int NS = BigTileRegs<TA, FULL, TILE>::NS;
    auto gload = [&](int s, int k0) {
        ra.load_slot(s, A, g.lda, m0, k0, M, K, g.vecA, tid);
        rb.load_slot(s, B, g.ldb, n0, k0, N, K, g.vecB, tid);
    };
    auto lstore = [&](int s, int buf) {
        ra.store_slot(s, As[buf], tid);
        rb.store_slot(s, Bs[buf], tid);
    };

    floatx16 acc[F][F];
#pragma unroll
    for (int i = 0; i < F; ++i)
#pragma unroll
        for (int j = 0; j < F; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;

    // Fragments of one 8-deep step: a[i] = op(A) rows wm+32i+lr, b[j] = op(B)
    // columns wn+32j+lr, k = k0+4h .. k0+4h+3 each.
    // Quad k0/4 + h of row wm + 32i + lr sits at position (k0/4 + h) ^ swz, with
    // swz = (lr ^ (lr >> 3) ^ 4(i & 1)) & 7 (wm, wn are multiples of 64);
    // k0/4 is even, so the position is (k0/4) ^ g with g = h ^ swz.
    struct Frag { float4 a[F], b[F]; };
    const int g_even = (h ^ lr ^ (lr >> 3)) & 7;
    auto read_frag = [&](Frag& f, int buf, int k0) {
        const float* as = As[buf] + (wm + lr) * kLd256;
        const float* bs = Bs[buf] + (wn + lr) * kLd256;
#pragma unroll
        for (int i = 0; i < F; ++i)
            f.a[i] = *reinterpret_cast<const float4*>(as + 32 * i * kLd256 + 4 * ((k0 / 4) ^ g_even ^ (4 * (i & 1))));
#pragma unroll
        for (int j = 0; j < F; ++j)
            f.b[j] = *reinterpret_cast<const float4*>(bs + 32 * j * kLd256 + 4 * ((k0 / 4) ^ g_even ^ (4 * (j & 1))));
    };
    auto mma_t = [&](const Frag& f, int t) {
#pragma unroll
        for (int i = 0; i < F; ++i)
#pragma unroll
            for (int j = 0; j < F; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x2f32(f4get(f.a[i], t), f4get(f.b[j], t), acc[i][j],
                                                                0, 0, 0);
    };

    // Software pipeline over the four 8-deep steps of a K tile:
    //   steps 0-2: read the next step's fragments, then four groups of F*F
    //     MFMAs; after each group, steps 0-1 issue one slot of the next tile's
    //     global loads (8 slots; with TILE = 128, 4 slots in step 0), step 2
    //     writes two slots (one) to the other LDS buffer (so the loads have
    //     had two steps to land);
    //   barrier; read the next tile's step-0 fragments; step 3's MFMAs.
    // Spreading the loads and LDS writes keeps the MFMA pipe fed (a CU's
    // address path takes 64 B/clk: a whole tile's 64 KB issued at once stalls
    // the waves for ~1K cycles).  All reads of an LDS buffer are issued before
    // the barrier that precedes its next write.
    constexpr int kSteps = kBigK / 8;
    static_assert(kSteps == 4 && kBigQ == 8 && (NS == 8 || NS == 4), "the load/store schedule assumes 32-deep K tiles");
    const int nk = (K + kBigK - 1) / kBigK;
    Frag f[2];
    if (nk > 0) {
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) gload(sl, 0);
#pragma unroll
        for (int sl = 0; sl < NS; ++sl) lstore(sl, 0);
        __syncthreads();
        read_frag(f[0], 0, 0);
    }
    // The loads, stores and reads of the next tile are unconditional (no
    // branches for the waitcnt placement to be conservative about): on the
    // last tile they repeat the current tile's loads into the idle buffer.
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const int kn = (kt + 1 < nk ? kt + 1 : kt) * kBigK;
#pragma unroll
        for (int st = 0; st + 1 < kSteps; ++st) {
            read_frag(f[(st + 1) & 1], cur, 8 * (st + 1));
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                __builtin_amdgcn_sched_barrier(0);
                mma_t(f[st & 1], t);
                __builtin_amdgcn_sched_barrier(0);
                if (NS == 8) {
                    if (st < 2) {
                        gload(4 * st + t, kn);
                    } else {
                        lstore(2 * t, cur ^ 1);
                        lstore(2 * t + 1, cur ^ 1);
                    }
                } else {
                    if (st == 0) gload(t, kn);
                    else if (st == 2) lstore(t, cur ^ 1);
                }
            }
        }
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        read_frag(f[0], cur ^ 1, 0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            __builtin_amdgcn_sched_barrier(0);
            mma_t(f[1], t);
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    if (g.splits > 1) {
        // raw slice sums, [slice][batch][M][N]; the ordered reduce applies
        // alpha, beta and R
        float* __restrict__ wz =
            g.ws + (static_cast<long long>(blockIdx.z) * gridDim.y + blockIdx.y) * (static_cast<long long>(M) * N);
#pragma unroll
        for (int i = 0; i < F; ++i)
#pragma unroll
            for (int j = 0; j < F; ++j) {
                const int col = n0 + wn + 32 * j + lr;
                if (!FULL && col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (FULL || row < M) wz[static_cast<long long>(row) * N + col] = acc[i][j][r];
                }
            }
        return;
    }
    float* __restrict__ C = g.C + coff;
    const float* R = g.R ? g.R + coff : C;
    const int ldr = g.R ? g.ldr : g.ldc;
    // The beta test sits outside the unrolled stores (one branch, not 256).
    auto epilogue = [&](auto use_rc) {
        constexpr bool USE_R = decltype(use_rc)::value;
#pragma unroll
        for (int i = 0; i < F; ++i)
#pragma unroll
            for (int j = 0; j < F; ++j) {
                const int col = n0 + wn + 32 * j + lr;
                if (!FULL && col >= N) continue;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = m0 + wm + 32 * i + 8 * (r >> 2) + 4 * h + (r & 3);
                    if (FULL || row < M) {
                        float v = g.alpha * acc[i][j][r];
                        if (USE_R) v += g.beta * R[static_cast<long long>(row) * ldr + col];
                        C[static_cast<long long>(row) * g.ldc + col] = v;
                    }
                }
            }
    };
    if (g.beta != 0.f) epilogue(std::true_type{});
    else epilogue(std::false_type{});
}

int launch_reduce(const GemmArgs& g, int batch, hipStream_t stream);

template <int TILE>
int launch_big(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    g.tiles_m = ceil_div(g.M, TILE);
    g.tiles_n = ceil_div(g.N, TILE);
    const long long nwg = static_cast<long long>(g.tiles_m) * g.tiles_n;
    if (nwg > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm: %lld workgroups exceed the grid limit", nwg);
    if (g.splits <= 1 || !g.ws) { g.splits = 1; g.kchunk = g.K; g.ws = nullptr; }
    dim3 grid(static_cast<unsigned>(nwg), batch, g.splits), block(kThreads, 1, 1);
    // FULL: every tile and every K slice whole (slices start at multiples of
    // kchunk, itself a multiple of the 32-deep K tile)
    const bool full = g.M % TILE == 0 && g.N % TILE == 0 && g.K % kBigK == 0 && g.kchunk % kBigK == 0 &&
                      (ta || g.vecA) && (!tb || g.vecB);
    auto go = [&](auto fullc) {
        constexpr bool F = decltype(fullc)::value;
        if (!ta && !tb) klaunch(sgemm_256_kernel<false, false, F, TILE>, grid, block, 0, stream, g);
        else if (ta && !tb) klaunch(sgemm_256_kernel<true, false, F, TILE>, grid, block, 0, stream, g);
        else if (!ta && tb) klaunch(sgemm_256_kernel<false, true, F, TILE>, grid, block, 0, stream, g);
        else klaunch(sgemm_256_kernel<true, true, F, TILE>, grid, block, 0, stream, g);
    };
    if (full) go(std::true_type{});
    else go(std::false_type{});
    const int rc = check_launch("sgemm (256): kernel launch");
    if (rc != LHIP_OK || g.splits <= 1) return rc;
    return launch_reduce(g, batch, stream);
}

int launch_256(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    return launch_big<kBig>(ta, tb, g, batch, stream);
}

// ---------------------------------------------------------------------------
// Small problems (fewer 64x64 output tiles than CUs, e.g. every GEMM of the
// C2 LMTrain step): one workgroup per 32x32 output tile, and the NW waves of
// the workgroup (4, or 8 once K >= 256) split K among themselves -- wave w
// takes the 8-deep K steps w, w+NW, w+2NW, ... -- each accumulating the whole
// 32x32 tile, so one tile's K loop runs on all four SIMDs of its CU.  The
// partial tiles are summed in LDS in wave order (deterministic).  Operands are loaded straight from
// global memory into MFMA fragments: for an 8-deep K step, lane l (row or
// column l%32, half h = l/32) holds op(A)[row][k0+4h .. k0+4h+3] and
// op(B)[k0+4h .. k0+4h+3][col]; MFMA i of the step multiplies element i of
// both, so the two halves of one v_mfma_f32_32x32x2f32 cover k0+i and
// k0+4+i and the four MFMAs cover k0 .. k0+7 exactly once.  The contiguous
// operand dimension is read as float4 when aligned, otherwise element-wise.
//
// With BR (batch-reduce, non-transposed A only) the K range is kblocks blocks
// of Kb (Kb % 4 == 0): logical k lies in block j = k / Kb, whose operands start
// at A + j*sAk and B + j*sBk, so C = alpha * sum_j A_j . op(B_j) + beta * R in
// one launch.  A lane's four k never straddle a block.
template <bool TA, bool TB, bool BR, int NW>
__global__ void __launch_bounds__(64 * NW)
sgemm_small_kernel(const GemmArgs g)
{
    __shared__ float red[NW][16][64];
    const int M = g.M, N = g.N;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int lr = lane & 31;
    const int h = lane >> 5;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, g.tiles_n, tm, tn);
    const int m0 = tm * 32, n0 = tn * 32;
    const long long zo = blockIdx.y / g.inner, zi = blockIdx.y % g.inner;
    const float* __restrict__ A = g.A + zo * g.sA2 + zi * g.sA;
    const float* __restrict__ B = g.B + zo * g.sB2 + zi * g.sB;
    const long long coff = zo * g.sC2 + zi * g.sC;
    const int kbeg = blockIdx.z * g.kchunk;
    const int kend = min(g.K, kbeg + g.kchunk);
    const int row = m0 + lr;      // this lane's A row
    const int col = n0 + lr;      // this lane's B column
    const bool rok = row < M, cok = col < N;

    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    // Each pass issues the loads of kSmallU K steps before any of their MFMAs,
    // so that many loads are in flight per wave (these launches have few
    // workgroups: latency, not bandwidth, bounds them).
    constexpr int U = kSmallU;
    for (int kp = kbeg + 8 * wave; kp < kend; kp += 8 * NW * U) {
        float a[U][4], b[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kl = kp + 8 * NW * u + 4 * h;   // first of this lane's four k (logical)
            const bool kfull = kl + 3 < kend;
            const int kend_l = kend - kl;         // valid k from kl on: i < kend_l
            int kb = kl;
            const float* __restrict__ Ab = A;
            const float* __restrict__ Bb = B;
            if (BR) {
                const int j = kl / g.Kb;
                kb = kl - j * g.Kb;
                Ab = A + j * g.sAk;
                Bb = B + j * g.sBk;
            }
            if (!TA) {
                const float* src = Ab + static_cast<long long>(row) * g.lda + kb;
                if (g.vecA && rok && kfull) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) a[u][i] = (rok && i < kend_l) ? src[i] : 0.f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    a[u][i] = (rok && i < kend_l) ? Ab[static_cast<long long>(kb + i) * g.lda + row] : 0.f;
            }
            if (!TB) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    b[u][i] = (cok && i < kend_l) ? Bb[static_cast<long long>(kb + i) * g.ldb + col] : 0.f;
            } else {
                const float* src = Bb + static_cast<long long>(col) * g.ldb + kb;
                if (g.vecB && cok && kfull) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    b[u][0] = v.x; b[u][1] = v.y; b[u][2] = v.z; b[u][3] = v.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) b[u][i] = (cok && i < kend_l) ? src[i] : 0.f;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int i = 0; i < 4; ++i)
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u][i], b[u][i], acc, 0, 0, 0);
    }

    // sum the waves' tiles in wave order; thread (wave w, lane l) finishes
    // accumulator registers (16/NW)w .. (16/NW)(w+1)-1 of lane l
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    const int ocol = n0 + (lane & 31);
    const int lk = lane >> 5;
    float* wz = nullptr;
    if (g.splits > 1)
        wz = g.ws + (static_cast<long long>(blockIdx.z) * gridDim.y + blockIdx.y) * (static_cast<long long>(M) * N);
    float* __restrict__ C = g.C + coff;
    const float* R = g.R ? g.R + coff : C;
    const int ldr = g.R ? g.ldr : g.ldc;
    constexpr int RPW = 16 / NW;
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int r = RPW * wave + q;
        float v = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[w][r][lane];
        const int orow = m0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (orow >= M || ocol >= N) continue;
        if (wz) {
            wz[static_cast<long long>(orow) * N + ocol] = v;
        } else {
            const float o = g.alpha * v;
            C[static_cast<long long>(orow) * g.ldc + ocol] =
                (g.beta != 0.f) ? o + g.beta * R[static_cast<long long>(orow) * ldr + ocol] : o;
        }
    }
}

// ---------------------------------------------------------------------------
// Skinny products (M <= 64 rows of C, B stored K x N): the work is one
// streaming pass over B, HBM-bound.  With one or two rows of C this VALU form
// streams B (2 to 4 FMAs per float4 of B); three to 64 rows take the MFMA
// form below, since at 16 rows the 64 FMAs per float4 outrun the VALU (packed
// fp32 is not used).  Each wave covers 256 columns with one float4 per lane.  The workgroup walks its K slice in chunks of kSkinnyKC
// rows: the chunk of A is staged in LDS as [k][m] (zero past M and past the
// slice), then wave w streams rows [w*KC/4, (w+1)*KC/4) of the chunk, U rows of
// B in flight, reading the M values of A of a row as broadcast LDS reads.
// Waves 1..3 hand their sums to wave 0 through LDS, added in wave order.  A K
// split over blockIdx.y writes [split][M][N] partials that splitk_reduce adds
// in split order.
constexpr int kSkinnyMax = 64;
constexpr int kSkinnyCols = 256;    // columns per workgroup (64 lanes x float4)
constexpr int kSkinnyKC = 256;      // K rows of A staged per chunk

template <int MS, bool TA, bool VEC>
__global__ void __launch_bounds__(256)
sgemm_skinny_kernel(const GemmArgs g)
{
    constexpr int U = MS >= 8 ? 4 : 8;
    constexpr int KC = kSkinnyKC;
    static_assert(KC % (4 * U) == 0, "a chunk must split into whole U-row steps per wave");
    constexpr int kRed = 3 * MS * 64;                    // float4s: waves 1..3 x MS rows x 64 lanes
    constexpr int kTab = KC * MS / 4;                    // float4s: A chunk [KC][MS]
    __shared__ float4 smem[kRed > kTab ? kRed : kTab];
    float* atab = reinterpret_cast<float*>(smem);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int M = g.M, N = g.N;
    const int n0 = blockIdx.x * kSkinnyCols + 4 * lane;
    const int k0 = blockIdx.y * g.kchunk;
    const int k1 = min(g.K, k0 + g.kchunk);
    const bool colfull = VEC && n0 + 3 < N;
    float4 acc[MS];
#pragma unroll
    for (int m = 0; m < MS; ++m) acc[m] = make_float4(0.f, 0.f, 0.f, 0.f);
    for (int kc0 = k0; kc0 < k1; kc0 += KC) {
        const int nk = min(KC, k1 - kc0);
        for (int i = tid; i < KC * MS; i += 256) {
            const int c = TA ? i / MS : i % KC;
            const int m = TA ? i % MS : i / KC;
            float v = 0.f;
            if (c < nk && m < M)
                v = TA ? g.A[static_cast<long long>(kc0 + c) * g.lda + m]
                       : g.A[static_cast<long long>(m) * g.lda + kc0 + c];
            atab[c * MS + m] = v;
        }
        __syncthreads();
        const int rpw = (nk + 4 * U - 1) / (4 * U) * U;   // rows per wave in this chunk
        const int rb = wv * rpw;
        const int re = min(rb + rpw, nk);
        for (int r = rb; r < re; r += U) {
            float4 b[U];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                b[u] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (r + u < re) {
                    const float* src = g.B + static_cast<long long>(kc0 + r + u) * g.ldb + n0;
                    if (colfull) {
                        const floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(src));
                        b[u] = make_float4(v.x, v.y, v.z, v.w);
                    } else {
                        b[u].x = n0 + 0 < N ? src[0] : 0.f;
                        b[u].y = n0 + 1 < N ? src[1] : 0.f;
                        b[u].z = n0 + 2 < N ? src[2] : 0.f;
                        b[u].w = n0 + 3 < N ? src[3] : 0.f;
                    }
                }
            }
            // rows past the slice hold zeros in both atab and b
#pragma unroll
            for (int u = 0; u < U; ++u) {
                float a[MS];
                const float* arow = atab + (r + u) * MS;
                if constexpr (MS >= 4) {
#pragma unroll
                    for (int q = 0; q < MS / 4; ++q) {
                        const float4 t = reinterpret_cast<const float4*>(arow)[q];
                        a[4 * q] = t.x; a[4 * q + 1] = t.y; a[4 * q + 2] = t.z; a[4 * q + 3] = t.w;
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < MS; ++m) a[m] = arow[m];
                }
#pragma unroll
                for (int m = 0; m < MS; ++m) {
                    acc[m].x += a[m] * b[u].x;
                    acc[m].y += a[m] * b[u].y;
                    acc[m].z += a[m] * b[u].z;
                    acc[m].w += a[m] * b[u].w;
                }
            }
        }
        __syncthreads();   // atab is rewritten by the next chunk (and reused below)
    }
    if (wv > 0) {
#pragma unroll
        for (int m = 0; m < MS; ++m) smem[((wv - 1) * MS + m) * 64 + lane] = acc[m];
    }
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int m = 0; m < MS; ++m) {
#pragma unroll
        for (int w = 0; w < 3; ++w) {
            const float4 t = smem[(w * MS + m) * 64 + lane];
            acc[m].x += t.x; acc[m].y += t.y; acc[m].z += t.z; acc[m].w += t.w;
        }
    }
    const bool split = g.splits > 1;
    float* base = split ? g.ws + static_cast<long long>(blockIdx.y) * M * N : g.C;
    const int ld = split ? N : g.ldc;
    const bool vst = colfull && (split ? (N % 4 == 0) : (g.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(g.C) & 15u) == 0));
#pragma unroll
    for (int m = 0; m < MS; ++m) {
        if (m < M) {
            float v[4] = {acc[m].x, acc[m].y, acc[m].z, acc[m].w};
            float* dst = base + static_cast<long long>(m) * ld + n0;
            if (!split) {
                const float* rr = g.R ? g.R + static_cast<long long>(m) * g.ldr + n0 : dst;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + e < N) v[e] = g.alpha * v[e] + (g.beta != 0.f ? g.beta * rr[e] : 0.f);
            }
            if (vst) {
                *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    if (n0 + e < N) dst[e] = v[e];
            }
        }
    }
}

// Skinny products with 3..64 rows of C on the matrix cores.  The VALU form
// above would spend up to 64 FMAs per float4 of B, more than the VALU issues at
// HBM rate; v_mfma_f32_16x16x4f32 covers 16 rows at once, and MG groups of 16
// rows (MG = ceil(M / 16)) reuse each float4 of B for 4 * MG MFMAs.  Each wave
// covers 64 columns: lane (q = l/16, p = l%16) loads the float4
// B[k][c0+4p .. c0+4p+3] of row k = k0 + 4s + q of step s (four 256-byte row
// segments per step), and MFMA e (e = 0..3) multiplies element e of it, so MFMA
// e computes the columns c0 + 4p + e with A[16g + p][k] as its A operand (zero
// past M).  Accumulator register r of MFMA e then holds C[16g + 4q + r][c0 + 4p
// + e]: each lane owns 4x4 blocks, stored as float4 rows.  Splits as in the
// VALU form.
constexpr int kSkinnyMfmaCols = 64;

// A is staged in LDS per chunk of KC K rows (loading it per step, MG scalar
// loads a lane per 4-row step each touching 16 rows, outweighed the stream of
// B at 64 rows and measured 6% slower at 16).  Eight
// waves (two per SIMD) take the 4-row steps w, w + 8, ... of a chunk.  A chunk
// is loaded as float4 along k (thread (m, k4): A[m][kc + 4k4 .. +3]) and written
// k-major As[k][m] with row stride 80 (16k + m spreads a wave's writes and the
// operand reads As[(4s + q) * 80 + 16g + p] over all 64 banks).  The next
// chunk's A and B are loaded into a second register set before the current
// chunk's MFMAs.  The waves' sums meet in two fixed rounds (waves 4..7 into
// 0..3, then 1..3 into 0).
constexpr int kSkinnyKCA = 128;
constexpr int kSkinnyLdsA = 80;
constexpr int kSkinnyLdsWaves = 8;

template <bool TA, bool VEC, int MG>
__global__ void __launch_bounds__(64 * kSkinnyLdsWaves)
sgemm_skinny_mfma_lds_kernel(const GemmArgs g)
{
    constexpr int NW = kSkinnyLdsWaves;
    constexpr int NT = 64 * NW;
    constexpr int KC = kSkinnyKCA;
    constexpr int U = KC / (4 * NW);                    // 4-row steps per wave per chunk
    constexpr int UA = 16 * MG * (KC / 4) / NT;         // A float4 units per thread per chunk
    static_assert(UA >= 1 && 16 * MG * (KC / 4) % NT == 0, "A chunk units must split evenly");
    // one LDS region for the A chunks and, after the last chunk, the waves' sums
    constexpr int kAs = KC * kSkinnyLdsA;               // floats
    constexpr int kRed = 4 * 4 * MG * 64 * 4;           // floats: 4 waves' partial tiles
    __shared__ floatx4 lds[(kAs > kRed ? kAs : kRed) / 4];
    float* As = reinterpret_cast<float*>(lds);
    floatx4 (*red)[4 * MG][64] = reinterpret_cast<floatx4 (*)[4 * MG][64]>(lds);
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int p = lane & 15, q = lane >> 4;
    const int M = g.M, N = g.N;
    const int col = blockIdx.x * kSkinnyMfmaCols + 4 * p;
    const int k0 = blockIdx.y * g.kchunk;
    const int k1 = min(g.K, k0 + g.kchunk);
    const bool colfull = VEC && col + 3 < N;
    floatx4 acc[MG][4];
#pragma unroll
    for (int gi = 0; gi < MG; ++gi)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[gi][e] = floatx4{0.f, 0.f, 0.f, 0.f};

    struct Chunk { float4 b[U]; float a[UA][4]; };
    auto load = [&](Chunk& c, int kc) {
        const int kn = min(KC, k1 - kc);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kl = 4 * (wv + NW * u) + q;
            c.b[u] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (kl < kn) {
                const float* src = g.B + static_cast<long long>(kc + kl) * g.ldb + col;
                if (colfull) {
                    const floatx4 v = __builtin_nontemporal_load(reinterpret_cast<const floatx4*>(src));
                    c.b[u] = make_float4(v.x, v.y, v.z, v.w);
                } else {
                    c.b[u].x = col + 0 < N ? src[0] : 0.f;
                    c.b[u].y = col + 1 < N ? src[1] : 0.f;
                    c.b[u].z = col + 2 < N ? src[2] : 0.f;
                    c.b[u].w = col + 3 < N ? src[3] : 0.f;
                }
            }
        }
#pragma unroll
        for (int j = 0; j < UA; ++j) {
            const int idx = threadIdx.x + NT * j;
            const int m = idx % (16 * MG), k4 = idx / (16 * MG);
            if (!TA && g.vecA && m < M && 4 * k4 + 3 < kn) {   // kc is a multiple of 4
                const float4 v = *reinterpret_cast<const float4*>(g.A + static_cast<long long>(m) * g.lda + kc + 4 * k4);
                c.a[j][0] = v.x; c.a[j][1] = v.y; c.a[j][2] = v.z; c.a[j][3] = v.w;
                continue;
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int kl = 4 * k4 + e;
                c.a[j][e] = (m < M && kl < kn)
                                ? (TA ? g.A[static_cast<long long>(kc + kl) * g.lda + m]
                                      : g.A[static_cast<long long>(m) * g.lda + kc + kl])
                                : 0.f;
            }
        }
    };
    auto consume = [&](const Chunk& c, int kc) {
        const int kn = min(KC, k1 - kc);
        __syncthreads();   // the previous chunk's operand reads are done
#pragma unroll
        for (int j = 0; j < UA; ++j) {
            const int idx = threadIdx.x + NT * j;
            const int m = idx % (16 * MG), k4 = idx / (16 * MG);
#pragma unroll
            for (int e = 0; e < 4; ++e) As[(4 * k4 + e) * kSkinnyLdsA + m] = c.a[j][e];
        }
        __syncthreads();
        return kn;
    };
    auto mma = [&](const Chunk& c, int kn) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int st = wv + NW * u;
            if (4 * st >= kn) break;                     // uniform
            const float* ar = As + (4 * st + q) * kSkinnyLdsA + p;
#pragma unroll
            for (int gi = 0; gi < MG; ++gi) {
                const float a = ar[16 * gi];
                acc[gi][0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, c.b[u].x, acc[gi][0], 0, 0, 0);
                acc[gi][1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, c.b[u].y, acc[gi][1], 0, 0, 0);
                acc[gi][2] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, c.b[u].z, acc[gi][2], 0, 0, 0);
                acc[gi][3] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, c.b[u].w, acc[gi][3], 0, 0, 0);
            }
        }
    };
    // two register sets: chunk c + 1 is loaded while chunk c runs its MFMAs
    if (k0 < k1) {
        Chunk c0, c1;
        load(c0, k0);
        for (int kc = k0; kc < k1; kc += 2 * KC) {
            int kn = consume(c0, kc);
            if (kc + KC < k1) load(c1, kc + KC);
            mma(c0, kn);
            if (kc + KC >= k1) break;
            kn = consume(c1, kc + KC);
            if (kc + 2 * KC < k1) load(c0, kc + 2 * KC);
            mma(c1, kn);
        }
    }
    __syncthreads();   // the last chunk's operand reads are done: the region becomes the hand-off
    if (wv >= 4) {
#pragma unroll
        for (int gi = 0; gi < MG; ++gi)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wv - 4][4 * gi + e][lane] = acc[gi][e];
    }
    __syncthreads();
    if (wv < 4) {
#pragma unroll
        for (int gi = 0; gi < MG; ++gi)
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[gi][e] += red[wv][4 * gi + e][lane];
    }
    __syncthreads();
    if (wv >= 1 && wv < 4) {
#pragma unroll
        for (int gi = 0; gi < MG; ++gi)
#pragma unroll
            for (int e = 0; e < 4; ++e) red[wv - 1][4 * gi + e][lane] = acc[gi][e];
    }
    __syncthreads();
    if (wv != 0) return;
#pragma unroll
    for (int gi = 0; gi < MG; ++gi)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
#pragma unroll
            for (int w = 0; w < 3; ++w) acc[gi][e] += red[w][4 * gi + e][lane];
        }
    const bool split = g.splits > 1;
    float* base = split ? g.ws + static_cast<long long>(blockIdx.y) * M * N : g.C;
    const int ld = split ? N : g.ldc;
    const bool vst = colfull && (split ? (N % 4 == 0) : (g.ldc % 4 == 0 && (reinterpret_cast<uintptr_t>(g.C) & 15u) == 0));
#pragma unroll
    for (int gr = 0; gr < 4 * MG; ++gr) {
        const int gi = gr >> 2, r = gr & 3;
        const int row = 16 * gi + 4 * q + r;
        if (row >= M) continue;
        float v[4] = {acc[gi][0][r], acc[gi][1][r], acc[gi][2][r], acc[gi][3][r]};
        float* dst = base + static_cast<long long>(row) * ld + col;
        if (!split) {
            const float* rr = g.R ? g.R + static_cast<long long>(row) * g.ldr + col : dst;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < N) v[e] = g.alpha * v[e] + (g.beta != 0.f ? g.beta * rr[e] : 0.f);
        }
        if (vst) {
            *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < N) dst[e] = v[e];
        }
    }
}

// ---------------------------------------------------------------------------
// Tiny problems (fewer 32x32 output tiles than CUs, e.g. the 512x128 outputs
// of the C2 step): one workgroup per 16x16 output tile, four times as many
// workgroups as the 32x32 kernel, so the fp32 MFMA work (64 cycles per
// 32x32x2 or 32 per 16x16x4 instruction and SIMD) spreads over more CUs.
// Same scheme as the small kernel with v_mfma_f32_16x16x4f32: for a 16-deep
// K step at k0, lane l (row or column l%16, group q = l/16) holds
// op(A)[row][k0+4q .. k0+4q+3] and op(B)[k0+4q .. k0+4q+3][col]; MFMA i of the
// step multiplies element i of both, so its four k slots (one per lane group)
// are k0+4q+i and the four MFMAs cover k0 .. k0+15 exactly once.  The NW
// waves (4, or 8 for one-pass slices deeper than 256) take the 16-deep steps
// w, w+NW, ...; their tiles are summed in LDS in wave order.  Steps wholly
// past the end of K issue no MFMA.  BR as above.
template <bool TA, bool TB, bool BR, bool PIPE, int NW = 4>
__global__ void __launch_bounds__(64 * NW)
sgemm_tiny_kernel(const GemmArgs g)
{
    __shared__ float red[NW][4][64];
    const int M = g.M, N = g.N;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave-uniform (readfirstlane): the K-step bounds below become scalar
    // branches, so a pass's loads issue back to back with no exec-mask joins
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lr = lane & 15;
    const int q = lane >> 4;
    int tm, tn;
    xcd_tile(blockIdx.x, gridDim.x, g.tiles_n, tm, tn);
    const int m0 = tm * 16, n0 = tn * 16;
    const long long zo = blockIdx.y / g.inner, zi = blockIdx.y % g.inner;
    const float* __restrict__ A = g.A + zo * g.sA2 + zi * g.sA;
    const float* __restrict__ B = g.B + zo * g.sB2 + zi * g.sB;
    const long long coff = zo * g.sC2 + zi * g.sC;
    const int kbeg = blockIdx.z * g.kchunk;
    const int kend = min(g.K, kbeg + g.kchunk);
    const int row = m0 + lr;
    const int col = n0 + lr;
    const bool rok = row < M, cok = col < N;
    // rows / columns past the edge load from row / column 0 (a valid address)
    const int rowc = rok ? row : 0, colc = cok ? col : 0;

    floatx4 acc;
#pragma unroll
    for (int r = 0; r < 4; ++r) acc[r] = 0.f;

    // A pass covers the wave's next U 16-deep steps; with more than one pass
    // the next pass's loads are issued before this pass's MFMAs (two register
    // sets), so the passes' load latencies overlap.
    constexpr int U = kSmallU;
    auto load_pass = [&](int kp, float (&a)[U][4], float (&b)[U][4]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ks = kp + 16 * NW * u;                 // wave-uniform step start
            const bool live = ks < kend;                // uniform
            // Without a second pass to overlap, steps past the end are skipped
            // by a scalar branch.  A pipelined pass keeps a fixed load count
            // (the wait before the previous pass's MFMAs counts them): its dead
            // steps load from kbeg and are zeroed.
            if (!PIPE && !live) break;
            const int kl = live ? ks + 4 * q : kbeg;
            const bool sfull = live && ks + 16 <= kend; // uniform: every lane's four k are in range
            const int kend_l = live ? kend - kl : 0;
            int kb = kl;
            const float* __restrict__ Ab = A;
            const float* __restrict__ Bb = B;
            if (BR) {
                // block of this k: with Kb % 16 == 0 a 16-deep step lies in one
                // block, so the index is the wave-uniform step start's
                const int j = (g.Kb % 16 == 0 && live) ? ks / g.Kb : kl / g.Kb;
                kb = kl - j * g.Kb;
                Ab = A + j * g.sAk;
                Bb = B + j * g.sBk;
            }
            // Rows of A past M and columns of B past N only reach outputs that
            // are not stored, so they load from row / column 0 unmasked; only
            // k past the end (the last step) must contribute zeros.
            if (!TA) {
                const float* src = Ab + static_cast<long long>(rowc) * g.lda + kb;
                if (sfull && g.vecA) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
                } else if (sfull) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) a[u][i] = src[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v = src[i < kend_l ? i : 0];
                        a[u][i] = i < kend_l ? v : 0.f;
                    }
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool ok = sfull || i < kend_l;
                    const float v = Ab[static_cast<long long>(ok ? kb + i : kbeg) * g.lda + rowc];
                    a[u][i] = (sfull || ok) ? v : 0.f;
                }
            }
            if (!TB) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool ok = sfull || i < kend_l;
                    const float v = Bb[static_cast<long long>(ok ? kb + i : kbeg) * g.ldb + colc];
                    b[u][i] = (sfull || ok) ? v : 0.f;
                }
            } else {
                const float* src = Bb + static_cast<long long>(colc) * g.ldb + kb;
                if (sfull && g.vecB) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    b[u][0] = v.x; b[u][1] = v.y; b[u][2] = v.z; b[u][3] = v.w;
                } else if (sfull) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) b[u][i] = src[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const float v = src[i < kend_l ? i : 0];
                        b[u][i] = i < kend_l ? v : 0.f;
                    }
                }
            }
        }
    };
    // Pipelined passes (K > 512) keep the per-element guarded loads: with
    // them the compiler overlaps the next pass's loads with this pass's MFMAs
    // (measured: 15 us for the C2 dxf product against 23 us with the
    // unmasked loads above).
    auto load_pass_guarded = [&](int kp, float (&a)[U][4], float (&b)[U][4]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kl = kp + 16 * NW * u + 4 * q;
            const bool kfull = kl + 3 < kend;
            const int kend_l = kend - kl;
            int kb = kl;
            const float* __restrict__ Ab = A;
            const float* __restrict__ Bb = B;
            if (BR) {
                // block of this k: with Kb % 16 == 0 a 16-deep step lies in one
                // block, so the index is the wave-uniform step start's
                int j;
                if (g.Kb % 16 == 0) {
                    const int ks = __builtin_amdgcn_readfirstlane(kp + 16 * NW * u);
                    j = ks / g.Kb;
                } else {
                    j = kl / g.Kb;
                }
                kb = kl - j * g.Kb;
                Ab = A + j * g.sAk;
                Bb = B + j * g.sBk;
            }
            if (!TA) {
                const float* src = Ab + static_cast<long long>(row) * g.lda + kb;
                if (g.vecA && rok && kfull) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) a[u][i] = (rok && i < kend_l) ? src[i] : 0.f;
                }
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    a[u][i] = (rok && i < kend_l) ? Ab[static_cast<long long>(kb + i) * g.lda + row] : 0.f;
            }
            if (!TB) {
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    b[u][i] = (cok && i < kend_l) ? Bb[static_cast<long long>(kb + i) * g.ldb + col] : 0.f;
            } else {
                const float* src = Bb + static_cast<long long>(col) * g.ldb + kb;
                if (g.vecB && cok && kfull) {
                    const float4 v = *reinterpret_cast<const float4*>(src);
                    b[u][0] = v.x; b[u][1] = v.y; b[u][2] = v.z; b[u][3] = v.w;
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) b[u][i] = (cok && i < kend_l) ? src[i] : 0.f;
                }
            }
        }
    };
    // When every live step of the pass is a full 16-deep step (the slice
    // length kend - kbeg a multiple of 16: steps start at kbeg + 16j, so a
    // step that starts before kend also ends by it), the operands' contiguous
    // loads are float4-aligned and, for
    // batch-reduce, a step never straddles a block, the pass loads with no
    // selects: each load's register is final, dead steps are skipped by
    // wave-uniform branches, and all the pass's loads issue before the first
    // wait.
    const bool fast_ops = (TA || g.vecA) && (!TB || g.vecB) && (!BR || g.Kb % 16 == 0);
    auto load_pass_full = [&](int kp, float (&a)[U][4], float (&b)[U][4]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int ks = kp + 16 * NW * u;
            if (ks >= kend) break;
            const int kl = ks + 4 * q;
            int kb = kl;
            const float* __restrict__ Ab = A;
            const float* __restrict__ Bb = B;
            if (BR) {
                const int j = ks / g.Kb;
                kb = kl - j * g.Kb;
                Ab = A + j * g.sAk;
                Bb = B + j * g.sBk;
            }
            if (!TA) {
                const float4 v = *reinterpret_cast<const float4*>(Ab + static_cast<long long>(rowc) * g.lda + kb);
                a[u][0] = v.x; a[u][1] = v.y; a[u][2] = v.z; a[u][3] = v.w;
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) a[u][i] = Ab[static_cast<long long>(kb + i) * g.lda + rowc];
            }
            if (!TB) {
#pragma unroll
                for (int i = 0; i < 4; ++i) b[u][i] = Bb[static_cast<long long>(kb + i) * g.ldb + colc];
            } else {
                const float4 v = *reinterpret_cast<const float4*>(Bb + static_cast<long long>(colc) * g.ldb + kb);
                b[u][0] = v.x; b[u][1] = v.y; b[u][2] = v.z; b[u][3] = v.w;
            }
        }
    };
    auto mma_pass = [&](int kp, const float (&a)[U][4], const float (&b)[U][4]) {
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (kp + 16 * NW * u >= kend) break;   // wave-uniform: nothing left in this pass
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][i], b[u][i], acc, 0, 0, 0);
        }
    };
    int kp = kbeg + 16 * wave;
    if (!PIPE) {   // K fits one pass: one register set
        if (fast_ops && (kend - kbeg) % 16 == 0 && kp < kend) {
            float a0[U][4], b0[U][4];
            load_pass_full(kp, a0, b0);
            __builtin_amdgcn_sched_barrier(0);   // keep every load ahead of the first MFMA
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (kp + 16 * NW * u >= kend) break;
#pragma unroll
                for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0[u][i], b0[u][i], acc, 0, 0, 0);
            }
        } else if (kp < kend) {
            float a0[U][4], b0[U][4];
            load_pass(kp, a0, b0);
            mma_pass(kp, a0, b0);
        }
    } else if (kp < kend) {
        float a0[U][4], b0[U][4], a1[U][4], b1[U][4];
        load_pass_guarded(kp, a0, b0);
        while (true) {
            const int k1 = kp + 16 * NW * U;
            if (k1 < kend) load_pass_guarded(k1, a1, b1);
            mma_pass(kp, a0, b0);
            if (k1 >= kend) break;
            const int k2 = k1 + 16 * NW * U;
            if (k2 < kend) load_pass_guarded(k2, a0, b0);
            mma_pass(k1, a1, b1);
            if (k2 >= kend) break;
            kp = k2;
        }
    }

    // thread (wave w < 4, lane l) finishes accumulator register w of lane l,
    // summing the NW waves' partial tiles in wave order
#pragma unroll
    for (int r = 0; r < 4; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    if (wave >= 4) return;
    float v = red[0][wave][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) v += red[w][wave][lane];
    const int orow = m0 + 4 * q + wave;
    const int ocol = n0 + lr;
    if (orow >= M || ocol >= N) return;
    if (g.splits > 1) {
        float* wz = g.ws + (static_cast<long long>(blockIdx.z) * gridDim.y + blockIdx.y) * (static_cast<long long>(M) * N);
        wz[static_cast<long long>(orow) * N + ocol] = v;
        return;
    }
    float* __restrict__ C = g.C + coff;
    const float* R = g.R ? g.R + coff : C;
    const int ldr = g.R ? g.ldr : g.ldc;
    const float o = g.alpha * v;
    C[static_cast<long long>(orow) * g.ldc + ocol] =
        (g.beta != 0.f) ? o + g.beta * R[static_cast<long long>(orow) * ldr + ocol] : o;
}

// Eight waves share K once it is long enough for each to get a full pass.
constexpr int kSmallWavesLongK = 8;
inline bool small_long_k(const GemmArgs& g) { return g.kchunk >= 8 * 4 * kSmallU; }

template <bool TA, bool TB, bool BR>
void launch_small_t(const GemmArgs& g, dim3 grid, hipStream_t stream)
{
    if (small_long_k(g))
        klaunch(sgemm_small_kernel<TA, TB, BR, kSmallWavesLongK>, grid, dim3(64 * kSmallWavesLongK), 0, stream, g);
    else
        klaunch(sgemm_small_kernel<TA, TB, BR, 4>, grid, dim3(256), 0, stream, g);
}

int launch_reduce(const GemmArgs& g, int batch, hipStream_t stream);

// PIPE: K needs more than one pass of the four waves (64 * kSmallU deep)
template <bool PIPE, int NW>
void launch_tiny_t(int ta, int tb, const GemmArgs& g, dim3 grid, hipStream_t stream)
{
    const dim3 block(64 * NW);
    if (g.Kb != g.K) {
        if (!tb) klaunch(sgemm_tiny_kernel<false, false, true, PIPE, NW>, grid, block, 0, stream, g);
        else klaunch(sgemm_tiny_kernel<false, true, true, PIPE, NW>, grid, block, 0, stream, g);
    } else if (!ta && !tb) klaunch(sgemm_tiny_kernel<false, false, false, PIPE, NW>, grid, block, 0, stream, g);
    else if (ta && !tb) klaunch(sgemm_tiny_kernel<true, false, false, PIPE, NW>, grid, block, 0, stream, g);
    else if (!ta && tb) klaunch(sgemm_tiny_kernel<false, true, false, PIPE, NW>, grid, block, 0, stream, g);
    else klaunch(sgemm_tiny_kernel<true, true, false, PIPE, NW>, grid, block, 0, stream, g);
}

int launch_tiny(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    g.tiles_m = ceil_div(g.M, 16);
    g.tiles_n = ceil_div(g.N, 16);
    const long long nwg = static_cast<long long>(g.tiles_m) * g.tiles_n;
    if (nwg > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm: %lld workgroups exceed the grid limit", nwg);
    if (g.splits <= 1) { g.splits = 1; g.kchunk = g.K; g.ws = nullptr; }
    dim3 grid(static_cast<unsigned>(nwg), batch, g.splits);
    // one pass of four waves covers 64 * kSmallU of K; a one-pass slice deeper
    // than 256 runs on eight waves (half the loads and MFMAs per wave)
    if (g.kchunk > 64 * kSmallU) launch_tiny_t<true, 4>(ta, tb, g, grid, stream);
    else if (g.kchunk > 256) launch_tiny_t<false, 8>(ta, tb, g, grid, stream);
    else launch_tiny_t<false, 4>(ta, tb, g, grid, stream);
    int rc = check_launch("sgemm (tiny): kernel launch");
    if (rc != LHIP_OK || g.splits <= 1 || g.skip_reduce) return rc;
    return launch_reduce(g, batch, stream);
}

int launch_small(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    g.tiles_m = ceil_div(g.M, 32);
    g.tiles_n = ceil_div(g.N, 32);
    const long long nwg = static_cast<long long>(g.tiles_m) * g.tiles_n;
    if (nwg > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm: %lld workgroups exceed the grid limit", nwg);
    if (g.splits <= 1) { g.splits = 1; g.kchunk = g.K; g.ws = nullptr; }
    dim3 grid(static_cast<unsigned>(nwg), batch, g.splits);
    if (g.Kb != g.K) {   // batch-reduce (sgemm_run admits it for non-transposed A only)
        if (!tb) launch_small_t<false, false, true>(g, grid, stream);
        else launch_small_t<false, true, true>(g, grid, stream);
    } else if (!ta && !tb) launch_small_t<false, false, false>(g, grid, stream);
    else if (ta && !tb) launch_small_t<true, false, false>(g, grid, stream);
    else if (!ta && tb) launch_small_t<false, true, false>(g, grid, stream);
    else launch_small_t<true, true, false>(g, grid, stream);
    int rc = check_launch("sgemm (small): kernel launch");
    if (rc != LHIP_OK || g.splits <= 1 || g.skip_reduce) return rc;
    return launch_reduce(g, batch, stream);
}

// Skinny path: M <= 64, B not transposed, one product (no batch, no
// batch-reduce), at least one full wave of columns.
bool skinny_ok(int ta, int tb, int m, int n, int batch, int kblocks)
{
    (void)ta;
    return !tb && m >= 1 && m <= kSkinnyMax && n >= kSkinnyCols && batch == 1 && kblocks == 1;
}

// 33..64 rows with long K and wide N: one 64-row tile band of 64x64 tiles on
// four wave sets, split over K so that tiles x slices fill the CUs (M = 64,
// K = N = 4096: 64 tiles x 4 slices, 31.8 us against 45 us on the skinny MFMA
// form and its reduce).
bool ks_split_ok(int m, int n, int k, int batch)
{
    return batch == 1 && m > 32 && m <= 64 && n >= 1024 && k >= 2048;
}

int ks_split_plan(int m, int n, int k, size_t ws_floats, int* kchunk_out)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long tiles = ceil_div(n, 64);
    long long s = std::max<long long>(1, cus / tiles);
    s = std::min<long long>(s, k / 512);
    s = std::min<long long>(s, 16);
    const long long mn = static_cast<long long>(m) * n;
    s = std::min<long long>(s, static_cast<long long>(ws_floats / mn));
    if (s < 2) return 1;
    const int kchunk = ceil_div(ceil_div(k, static_cast<int>(s)), 32) * 32;
    *kchunk_out = kchunk;
    return ceil_div(k, kchunk);
}

// Rows of C up to which the VALU form is used; 3..64 rows take the MFMA form.
constexpr int kSkinnyValuMax = 2;

// K slices of the skinny path: about two workgroups per CU, at least 64 K rows
// per workgroup, and partials (written, then read back by the reduce) at most
// a quarter of B's bytes: 2 * s * m * n <= k * n / 4.
int skinny_plan(int m, int n, int k, size_t ws_floats, int* kchunk_out)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long cb = ceil_div(n, m <= kSkinnyValuMax ? kSkinnyCols : kSkinnyMfmaCols);
    // about two workgroups per CU for the VALU form and the one-group (M <= 16)
    // MFMA form; one for the eight-wave MFMA form on 2-4 groups (M = 4, 8, 16
    // at K = N = 4096: 24.1, 24.5, 21.1 us on one per CU, 19.6, 19.6, 19.3 on
    // two; M = 32: 29.2 on one, 30.7 on two)
    const long long per_cu = m <= 16 ? 2 : 1;
    long long s = (per_cu * cus + cb - 1) / cb;
    s = std::min<long long>(s, k / 64);
    s = std::min<long long>(s, std::max<long long>(1, k / (8LL * m)));
    const long long mn = static_cast<long long>(m) * n;
    if (mn > 0) s = std::min<long long>(s, static_cast<long long>(ws_floats / mn));
    if (s < 2) {
        *kchunk_out = k;
        return 1;
    }
    const int kchunk = ceil_div(ceil_div(k, s), 4) * 4;
    *kchunk_out = kchunk;
    return ceil_div(k, kchunk);
}

template <bool TA, bool VEC>
void launch_skinny_t(const GemmArgs& g, dim3 grid, hipStream_t stream)
{
    if (g.M == 1) klaunch(sgemm_skinny_kernel<1, TA, VEC>, grid, 256, 0, stream, g);
    else klaunch(sgemm_skinny_kernel<2, TA, VEC>, grid, 256, 0, stream, g);
}

int launch_skinny(int ta, GemmArgs g, hipStream_t stream)
{
    g.kchunk = g.K;
    g.splits = g.ws ? skinny_plan(g.M, g.N, g.K, g.ws_floats_avail, &g.kchunk) : 1;
    if (g.splits <= 1) { g.splits = 1; g.kchunk = g.K; }
    const bool vec = g.vecB;
    if (g.M <= kSkinnyValuMax) {
        const dim3 grid(ceil_div(g.N, kSkinnyCols), g.splits);
        if (ta) { if (vec) launch_skinny_t<true, true>(g, grid, stream); else launch_skinny_t<true, false>(g, grid, stream); }
        else { if (vec) launch_skinny_t<false, true>(g, grid, stream); else launch_skinny_t<false, false>(g, grid, stream); }
    } else {
        const dim3 grid(ceil_div(g.N, kSkinnyMfmaCols), g.splits);
        auto go = [&](auto mgc) {
            constexpr int MG = decltype(mgc)::value;
            constexpr int T = 64 * kSkinnyLdsWaves;
            if (ta) {
                if (vec) klaunch(sgemm_skinny_mfma_lds_kernel<true, true, MG>, grid, T, 0, stream, g);
                else klaunch(sgemm_skinny_mfma_lds_kernel<true, false, MG>, grid, T, 0, stream, g);
            } else {
                if (vec) klaunch(sgemm_skinny_mfma_lds_kernel<false, true, MG>, grid, T, 0, stream, g);
                else klaunch(sgemm_skinny_mfma_lds_kernel<false, false, MG>, grid, T, 0, stream, g);
            }
        };
        const int mg = ceil_div(g.M, 16);
        if (mg == 1) go(std::integral_constant<int, 1>{});
        else if (mg == 2) go(std::integral_constant<int, 2>{});
        else if (mg == 3) go(std::integral_constant<int, 3>{});
        else go(std::integral_constant<int, 4>{});
    }
    int rc = check_launch("sgemm (skinny): kernel launch");
    if (rc != LHIP_OK || g.splits <= 1) return rc;
    return launch_reduce(g, 1, stream);
}

template <int BM, int BN, int BK, int KS>
int launch_cfg_ks(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    g.tiles_m = ceil_div(g.M, BM);
    g.tiles_n = ceil_div(g.N, BN);
    const long long nwg = static_cast<long long>(g.tiles_m) * g.tiles_n;
    if (nwg > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm: %lld workgroups exceed the grid limit", nwg);
    if (g.splits <= 1) { g.splits = 1; g.kchunk = g.K; g.ws = nullptr; }
    dim3 grid(static_cast<unsigned>(nwg), batch, g.splits), block(KS * kThreads, 1, 1);
    // NN (A's 32-deep chunk is 64 row segments of 128 bytes) loads two chunks
    // ahead: 1024^3 32.3 -> 30.8 us and 2048x1024x512 31.9 -> 31.3 (medians of
    // six alternating rounds on one box); TN and NT measured 0.4-0.5 us slower
    // that way
    // Whole chunks with float4-loadable operands: unconditional
    // loads two chunks ahead (1024^3 NN 29.5 -> 26.6 us, NT 26.9 -> 24.2, TN
    // 27.5 -> 26.0, 2048x1024x512 30.6 -> 25.8, the M = 64 band 29.4 -> 27.3;
    // with the loads behind a branch each LDS store waited for every load in
    // flight, the chunk two ahead included)
    // (M and N need not be whole tiles: rows and columns past them are
    // clamped into the operands; M % 4 == 0 when A is stored K-major and
    // N % 4 == 0 when B is.  The tied head of the C2 step, 512x2000x128 NT,
    // 7.2 -> 6.8 us; a 60x4000x4096 band 31.5 -> 27.8.)
    const bool full = (!ta || g.M % 4 == 0) && (tb || g.N % 4 == 0) && g.K % BK == 0 && g.kchunk % BK == 0 &&
                      g.vecA && g.vecB && g.Kb == g.K;
    if (full) {
        if (!ta && !tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, false, false, KS, 2, true>, grid, block, 0, stream, g);
        else if (ta && !tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, true, false, KS, 2, true>, grid, block, 0, stream, g);
        else if (!ta && tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, false, true, KS, 2, true>, grid, block, 0, stream, g);
        else klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, true, true, KS, 2, true>, grid, block, 0, stream, g);
    } else if (!ta && !tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, false, false, KS, 2>, grid, block, 0, stream, g);
    else if (ta && !tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, true, false, KS>, grid, block, 0, stream, g);
    else if (!ta && tb) klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, false, true, KS>, grid, block, 0, stream, g);
    else klaunch(sgemm_mfma_ks_kernel<BM, BN, BK, true, true, KS>, grid, block, 0, stream, g);
    int rc = check_launch("sgemm: kernel launch");
    if (rc != LHIP_OK || g.splits <= 1 || g.skip_reduce) return rc;
    return launch_reduce(g, batch, stream);
}

template <int BM, int BN, int BK>
int launch_cfg(int ta, int tb, GemmArgs g, int batch, hipStream_t stream)
{
    g.tiles_m = ceil_div(g.M, BM);
    g.tiles_n = ceil_div(g.N, BN);
    const long long nwg = static_cast<long long>(g.tiles_m) * g.tiles_n;
    if (nwg > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm: %lld workgroups exceed the grid limit", nwg);
    if (g.splits <= 1) { g.splits = 1; g.kchunk = g.K; g.ws = nullptr; }
    dim3 grid(static_cast<unsigned>(nwg), batch, g.splits), block(kThreads, 1, 1);
    if (!ta && !tb) klaunch(sgemm_mfma_kernel<BM, BN, BK, false, false>, grid, block, 0, stream, g);
    else if (ta && !tb) klaunch(sgemm_mfma_kernel<BM, BN, BK, true, false>, grid, block, 0, stream, g);
    else if (!ta && tb) klaunch(sgemm_mfma_kernel<BM, BN, BK, false, true>, grid, block, 0, stream, g);
    else klaunch(sgemm_mfma_kernel<BM, BN, BK, true, true>, grid, block, 0, stream, g);
    int rc = check_launch("sgemm: kernel launch");
    if (rc != LHIP_OK || g.splits <= 1 || g.skip_reduce) return rc;
    return launch_reduce(g, batch, stream);
}

int launch_reduce(const GemmArgs& g, int batch, hipStream_t stream)
{
    const bool vec4 = batch == 1 && g.N % 4 == 0 && g.ldc % 4 == 0 && aligned16(g.C) && aligned16(g.ws) &&
                      (!g.R || (g.ldr % 4 == 0 && aligned16(g.R)));
    if (vec4) {
        const long long total4 = static_cast<long long>(g.M) * g.N / 4;
        long long rg = (total4 + 255) / 256;
        const long long cap = static_cast<long long>(st().cu_count > 0 ? st().cu_count : 256) * 4;
        if (rg > cap) rg = cap;
        klaunch(splitk_reduce4, static_cast<int>(rg), 256, 0, stream, g);
        return check_launch("sgemm: split-K reduce");
    }
    const long long total = static_cast<long long>(g.M) * g.N * batch;
    long long rg = (total + 255) / 256;
    const long long cap = static_cast<long long>(st().cu_count > 0 ? st().cu_count : 256) * 4;
    if (rg > cap) rg = cap;
    klaunch(splitk_reduce, static_cast<int>(rg), 256, 0, stream, g, batch);
    return check_launch("sgemm: split-K reduce");
}

// Grouped transposed-A products (the weight gradients of the LMTrain step:
// dW = X^T . dY with X, dY row-major over the same B*T rows, every layer's and
// the tied embedding's in one launch).  Workgroup id -> (group, tile) through
// the groups' first-tile table; each 32x32 tile is computed like
// sgemm_small_kernel<TA, !TB>: NW waves split K into 8-deep steps, lane l
// (row or column l%32, half h = l/32) holding A^T[row][k0+4h..+3] (four loads
// down a column of the stored A, coalesced over the 32 rows) and
// B[k0+4h..+3][col], v_mfma_f32_32x32x2f32, partial tiles summed in LDS in
// wave order.  (Fallback for operands that cannot take float4 loads.)
constexpr int kGroupedTile = 32;

struct GroupedTNArgs {
    GroupedTN e[kGroupedMax];
    int tile0[kGroupedMax + 1];
    int tiles_n[kGroupedMax];
    int ngroups, K;
    ColsumSet cs;     // column sums run by the workgroups after the last tile
    int cs_cb;        // 32-column blocks per column-sum job
    int cs_blocks;    // cs.njobs * cs_cb
    int tp, cp;       // 64x64 kernel: tiles, column-sum workgroups per XCD
    int cs_per_wg;    // 64x64 kernel: column-sum blocks per workgroup
    int do_sc;        // 64x64 kernel: run the groups' scatters
    double* ss_out;   // 64x64 kernel: per-workgroup sums of squares of the stored values (or NULL)
};

template <int NW>
__global__ void __launch_bounds__(64 * NW) sgemm_grouped_tn_kernel(const GroupedTNArgs ga)
{
    __shared__ float red[NW][16][64];
    // XCD-contiguous tiles: workgroups are dispatched round-robin over the 8
    // XCDs, so id p runs on XCD p % 8; XCD x takes the tiles
    // [x*G/8, (x+1)*G/8) (G padded to a multiple of 8), i.e. whole groups and
    // row bands, whose operands then stay in that XCD's L2.
    const int per_xcd = gridDim.x / 8;
    const int id = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (id >= ga.tile0[ga.ngroups]) return;   // padding
    int gi = 0;
    for (int i = 1; i < ga.ngroups; ++i)
        if (id >= ga.tile0[i]) gi = i;
    const GroupedTN& e = ga.e[gi];
    const int local = id - ga.tile0[gi];
    const int tm = local / ga.tiles_n[gi], tn = local - tm * ga.tiles_n[gi];
    const int K = ga.K;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, lr = lane & 31, h = lane >> 5;
    const int m0 = tm * kGroupedTile, n0 = tn * kGroupedTile;
    const int row = m0 + lr, col = n0 + lr;
    const bool rok = row < e.M, cok = col < e.N;
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    constexpr int U = kSmallU;
    for (int kp = 8 * wave; kp < K; kp += 8 * NW * U) {
        float a[U][4], b[U][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int kl = kp + 8 * NW * u + 4 * h;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const bool kin = kl + i < K;
                a[u][i] = (rok && kin) ? e.A[static_cast<long long>(kl + i) * e.lda + row] : 0.f;
                b[u][i] = (cok && kin) ? e.B[static_cast<long long>(kl + i) * e.ldb + col] : 0.f;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (kp + 8 * NW * u >= K) break;   // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a[u][i], b[u][i], acc, 0, 0, 0);
        }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    // thread (wave w, lane l) finishes accumulator registers (16/NW)w .. of lane l
    constexpr int RPW = 16 / NW;
    const int ocol = n0 + (lane & 31);
    const int lk = lane >> 5;
#pragma unroll
    for (int q = 0; q < RPW; ++q) {
        const int r = RPW * wave + q;
        float v = red[0][r][lane];
#pragma unroll
        for (int w = 1; w < NW; ++w) v += red[w][r][lane];
        const int orow = m0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (orow < e.M && ocol < e.N) e.C[static_cast<long long>(orow) * e.ldc + ocol] = v;
    }
}

// LDS-staged form of the grouped kernel, for groups whose operands allow
// float4 loads (leading dimensions % 4 == 0, 16-byte aligned bases).  Both
// operands are stored K-major (A is K x M, B is K x N), so a 64-deep chunk of
// each is copied into LDS unchanged with float4 loads (four per thread per
// chunk), double-buffered; wave w then runs the 8 MFMA steps of chunk rows
// 16w .. 16w+15 on the whole 32x32 tile, reading each operand fragment as one
// conflict-free ds_read_b32 (lanes 0-31 row k, 32-63 row k+1).  The waves'
// tiles are summed in LDS in wave order.  Workgroups past the last tile run the
// column-sum jobs of ga.cs, one 32-column block each (colsum4_block).
constexpr int kGroupedBK = 64;

__global__ void __launch_bounds__(256) sgemm_grouped_tn_lds_kernel(const GroupedTNArgs ga)
{
    constexpr int T = kGroupedTile, BK = kGroupedBK;
    __shared__ float As[2][BK][T];
    __shared__ float Bs[2][BK][T];
    __shared__ float red[4][16][64];
    const int per_xcd = gridDim.x / 8;
    const int id = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (id >= ga.tile0[ga.ngroups]) {
        const int cid = id - ga.tile0[ga.ngroups];
        if (cid >= ga.cs_blocks) return;   // padding
        const int job = cid / ga.cs_cb, cb = cid - job * ga.cs_cb;
        colsum4_block(ga.cs.partial[job], ga.cs.nparts[job], ga.cs.out[job], ga.cs.cols, 32 * cb, ga.cs.acc,
                      reinterpret_cast<float4 (*)[8]>(&red[0][0][0]));
        return;
    }
    int gi = 0;
    for (int i = 1; i < ga.ngroups; ++i)
        if (id >= ga.tile0[i]) gi = i;
    const GroupedTN& e = ga.e[gi];
    const int local = id - ga.tile0[gi];
    const int tm = local / ga.tiles_n[gi], tn = local - tm * ga.tiles_n[gi];
    const int K = ga.K;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, lr = lane & 31, lk = lane >> 5;
    const int m0 = tm * T, n0 = tn * T;
    // chunk loader: thread t covers chunk rows t/8 and t/8 + 32, float4 column (t%8)*4
    const int lrow = tid >> 3, lc4 = (tid & 7) * 4;
    const bool am_ok = m0 + lc4 < e.M, bn_ok = n0 + lc4 < e.N;   // M, N % 4 == 0 (host check)
    float4 ra[2], rb[2];
    auto gload = [&](int k0) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int k = k0 + lrow + 32 * p;
            const bool kin = k < K;
            ra[p] = (kin && am_ok) ? *reinterpret_cast<const float4*>(e.A + static_cast<long long>(k) * e.lda + m0 + lc4)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
            rb[p] = (kin && bn_ok) ? *reinterpret_cast<const float4*>(e.B + static_cast<long long>(k) * e.ldb + n0 + lc4)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto lstore = [&](int buf) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            *reinterpret_cast<float4*>(&As[buf][lrow + 32 * p][lc4]) = ra[p];
            *reinterpret_cast<float4*>(&Bs[buf][lrow + 32 * p][lc4]) = rb[p];
        }
    };
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    const int nk = (K + BK - 1) / BK;
    gload(0);
    lstore(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) gload((kt + 1) * BK);
#pragma unroll
        for (int st = 0; st < 8; ++st) {
            const int kr = 16 * wave + 2 * st + lk;
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[cur][kr][lr], Bs[cur][kr][lr], acc, 0, 0, 0);
        }
        if (more) lstore(cur ^ 1);
        __syncthreads();
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][r][lane] = acc[r];
    __syncthreads();
    // thread (wave w, lane l) finishes accumulator registers 4w .. 4w+3 of lane l
    const int ocol = n0 + lr;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int r = 4 * wave + q;
        const float v = ((red[0][r][lane] + red[1][r][lane]) + red[2][r][lane]) + red[3][r][lane];
        const int orow = m0 + 8 * (r >> 2) + 4 * lk + (r & 3);
        if (orow < e.M && ocol < e.N) e.C[static_cast<long long>(orow) * e.ldc + ocol] = v;
    }
}

// Sum over the workgroup of each thread's double (wave order, then wave 0's
// thread 0 adds the waves in order) into ss_out[blockIdx.x].
template <int NW>
__device__ __forceinline__ void block_sumsq_out(double v, double* ss_out, double* red)
{
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        double t = 0.0;
#pragma unroll
        for (int w = 0; w < NW; ++w) t += red[w];
        ss_out[blockIdx.x] = t;
    }
}

// 64x64 tiles for the same float4-loadable groups.  The tile's 32x32
// quadrants belong to four waves, and KS sets of four waves take the BK-deep
// K chunks in turn (set s: chunks s, s+KS, ..., each set with its own
// double-buffered LDS), so each chain of dependent chunk loads is 1/KS as
// long; the partial quadrants are added in LDS in set order.  KS = 2 with
// 64-deep chunks for short K; KS = 4 with 32-deep chunks from K = 512 on
// (four waves per SIMD: the C2 step's launch, K = 512, 19.3 -> 18.1 us).  At
// the LM step's shapes (K = batch*seq rows) this is about one workgroup per
// CU, and nothing is re-read by a neighbouring tile as often as with 32x32
// tiles.
// Placement: XCD x (blocks b with b % 8 == x) takes tiles [x*tp, (x+1)*tp)
// first and then cp workgroups of column-sum jobs, each running up to
// cs_per_wg 32-column blocks in turn, so no XCD holds more tiles than CUs.
// BUF: the chunk loads are buffer loads whose records end at each operand's
// last element, so rows past K read as zeros from the hardware's range check
// with no branch, and every chunk load is issued on every path (past the last
// chunk a load fetches zeros); the compiler's memory-count waits then hold
// each LDS store for its own chunk only.  (Behind the per-lane bounds branches
// it waited for every load in flight, the chunk two ahead included, before
// each store and again before each iteration's loads.)  Columns past M or N
// read whatever lies there instead of zeros: they only reach output rows and
// columns that are never stored or counted.  The host takes this form when
// every operand's byte offsets stay below 2^31.
template <int KS, int BK, bool BUF = false>
__global__ void __launch_bounds__(256 * KS) sgemm_grouped_tn_lds64_kernel(const GroupedTNArgs ga)
{
    constexpr int T = 64, P = BK / 16;
    static_assert(BK % 16 == 0 && (KS - 1) * 4096 <= KS * 2 * BK * T, "reduction area");
    __shared__ __align__(16) float As[KS][2][BK][T];
    __shared__ __align__(16) float Bs[KS][2][BK][T];
    __shared__ double ssred[4 * KS];
    __shared__ int sclst[4][1024];   // per wave of set 0: a scatter round's (token, row) list
    const int xcd = blockIdx.x % 8, j = blockIdx.x / 8;
    const int ntiles = ga.tile0[ga.ngroups];
    if (j >= ga.tp) {
        const int w = xcd * ga.cp + (j - ga.tp);
        double sq = 0.0;
        for (int q = 0; q < ga.cs_per_wg; ++q) {
            const int cid = w * ga.cs_per_wg + q;
            if (cid >= ga.cs_blocks) break;   // uniform
            const int job = cid / ga.cs_cb, cb = cid - job * ga.cs_cb;
            const float4 t = colsum4_block<256 * KS>(ga.cs.partial[job], ga.cs.nparts[job], ga.cs.out[job],
                                                     ga.cs.cols, 32 * cb, ga.cs.acc,
                                                     reinterpret_cast<float4 (*)[8]>(&As[0][0][0][0]));
            sq += static_cast<double>(t.x) * t.x + static_cast<double>(t.y) * t.y +
                  static_cast<double>(t.z) * t.z + static_cast<double>(t.w) * t.w;
            __syncthreads();   // red is reused by the next block
        }
        if (ga.ss_out) block_sumsq_out<4 * KS>(sq, ga.ss_out, ssred);
        return;
    }
    const int id = xcd * ga.tp + j;
    if (id >= ntiles) {   // padding
        if (ga.ss_out && threadIdx.x == 0) ga.ss_out[blockIdx.x] = 0.0;
        return;
    }
    int gi = 0;
    for (int i = 1; i < ga.ngroups; ++i)
        if (id >= ga.tile0[i]) gi = i;
    const GroupedTN& e = ga.e[gi];
    const int local = id - ga.tile0[gi];
    const int tm = local / ga.tiles_n[gi], tn = local - tm * ga.tiles_n[gi];
    const int K = ga.K;
    const int tid = threadIdx.x, lane = tid & 63, lr = lane & 31, lk = lane >> 5;
    const int grp = __builtin_amdgcn_readfirstlane(tid >> 8), gt = tid & 255;
    const int wave = __builtin_amdgcn_readfirstlane((tid >> 6) & 3);
    const int wm = 32 * (wave & 1), wn = 32 * (wave >> 1);
    const int m0 = tm * T, n0 = tn * T;
    // chunk loader of a set: thread t covers chunk rows t/16 + 16p (p < 4), float4 column (t%16)*4
    const int lrow = gt >> 4, lc4 = (gt & 15) * 4;
    const bool am_ok = m0 + lc4 < e.M, bn_ok = n0 + lc4 < e.N;   // M, N % 4 == 0 (host check)
    // two register sets: a set's next-but-one chunk is in flight while the
    // current chunk's MFMAs run and the next chunk goes to LDS
    float4 ra0[P], rb0[P], ra1[P], rb1[P];
    typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
    // buffer records: (K - 1) full rows plus the last row's M (N) columns
    const __amdgpu_buffer_rsrc_t rsa = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(e.A), 0, BUF ? ((K - 1) * e.lda + e.M) * 4 : 0, 0x00020000);
    const __amdgpu_buffer_rsrc_t rsb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(e.B), 0, BUF ? ((K - 1) * e.ldb + e.N) * 4 : 0, 0x00020000);
    auto gload = [&](int k0, float4 (&ra)[P], float4 (&rb)[P]) {
        if constexpr (BUF) {
#pragma unroll
            for (int p = 0; p < P; ++p) {
                const int k = k0 + lrow + 16 * p;
                ra[p] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rsa, (k * e.lda + m0 + lc4) * 4, 0, 0));
                rb[p] = __builtin_bit_cast(float4, __builtin_amdgcn_raw_buffer_load_b128(
                                                       rsb, (k * e.ldb + n0 + lc4) * 4, 0, 0));
            }
            return;
        }
#pragma unroll
        for (int p = 0; p < P; ++p) {
            const int k = k0 + lrow + 16 * p;
            const bool kin = k < K;
            ra[p] = (kin && am_ok) ? *reinterpret_cast<const float4*>(e.A + static_cast<long long>(k) * e.lda + m0 + lc4)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
            rb[p] = (kin && bn_ok) ? *reinterpret_cast<const float4*>(e.B + static_cast<long long>(k) * e.ldb + n0 + lc4)
                                   : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto lstore = [&](int buf, const float4 (&ra)[P], const float4 (&rb)[P]) {
#pragma unroll
        for (int p = 0; p < P; ++p) {
            *reinterpret_cast<float4*>(&As[grp][buf][lrow + 16 * p][lc4]) = ra[p];
            *reinterpret_cast<float4*>(&Bs[grp][buf][lrow + 16 * p][lc4]) = rb[p];
        }
    };
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;
    // Scatter C[id_i] += scale * rows[i] over the tokens i whose id falls in
    // this wave's 32 rows, in token order.  A round lists the matches among 512
    // tokens in LDS (slot = rank in token order).  The first SC matches of the
    // first round are fetched before the products start, so their loads
    // overlap the chunk loads, and added after the products; any others are
    // fetched after the products, eight at a time.
    constexpr int SC = 24;
    const bool scat = ga.do_sc && e.sc_n > 0 && grp == 0;
    const int ocol = n0 + wn + lr;
    const int rlo = m0 + wm;
    int* lst = &sclst[wave][0];
    int idpre[8];
    if (scat) {
        // unconditional loads (clamped index) keep the memory-count waits of
        // the chunk loads exact
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = 64 * u + lane;
            const int v = e.sc_ids[min(i, e.sc_n - 1)];
            idpre[u] = i < e.sc_n ? v : -1;
        }
    }
    auto build_list = [&](int base) -> int {   // wave-uniform match count
        int total = 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int i = base + 64 * u + lane;
            const int idv = base == 0 ? idpre[u] : (i < e.sc_n ? e.sc_ids[i] : -1);
            const int rel = idv - rlo;
            const bool hit = i < e.sc_n && rel >= 0 && rel < 32 && idv < e.M;
            const unsigned long long mask = __ballot(hit);
            if (hit) {
                const int slot = total + __popcll(mask & ((1ull << lane) - 1ull));
                lst[2 * slot] = i;
                lst[2 * slot + 1] = rel;
            }
            total += __popcll(mask);
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        return total;
    };
    const float scl = e.sc_scale;
    const int nk = (K + BK - 1) / BK;
    const int iters = (nk + KS - 1) / KS;   // every set passes the same barriers
    gload(grp * BK, ra0, rb0);
    if (BUF || iters > 1) gload((grp + KS) * BK, ra1, rb1);
    float sv[SC];             // rows of the first SC matches, fetched during the products
    unsigned srel[SC / 4];    // their rows within the wave's 32, 8 bits each (0xff: none)
    int first_total = 0;
    if (scat) {
        first_total = build_list(0);
        const int ccol = min(ocol, e.N - 1);
        int2 ent[SC];   // (token, row) pairs, read unconditionally so the reads batch
#pragma unroll
        for (int c = 0; c < SC; ++c) ent[c] = reinterpret_cast<const int2*>(lst)[c];
#pragma unroll
        for (int c = 0; c < SC; ++c) {
            const int tok = c < first_total ? ent[c].x : 0;   // row 0 stands in (its value is not used)
            sv[c] = e.sc_rows[static_cast<long long>(tok) * e.sc_ld + ccol];
        }
#pragma unroll
        for (int q = 0; q < SC / 4; ++q) {
            unsigned w = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int c = 4 * q + b;
                w |= static_cast<unsigned>(c < first_total ? ent[c].y : 0xff) << (8 * b);
            }
            srel[q] = w;
        }
        __builtin_amdgcn_wave_barrier();   // the list is rewritten after the products
    }
    lstore(0, ra0, rb0);
    __syncthreads();
    auto chunk_mfma = [&](int buf, int kt) {
        if (kt < nk) {
#pragma unroll
            for (int st = 0; st < BK / 2; ++st) {
                const int kr = 2 * st + lk;   // lanes 0-31 read row k, 32-63 row k+1
                acc = __builtin_amdgcn_mfma_f32_32x32x2f32(As[grp][buf][kr][wm + lr], Bs[grp][buf][kr][wn + lr], acc,
                                                           0, 0, 0);
            }
        }
    };
    // iteration it computes the set's chunk it*KS + grp from LDS buffer it%2,
    // stores chunk it+1 (loaded an iteration earlier) into the other buffer
    // and issues the loads of chunk it+2
    for (int it = 0; it < iters; it += 2) {
        if (BUF || it + 2 < iters) gload(((it + 2) * KS + grp) * BK, ra0, rb0);
        chunk_mfma(0, it * KS + grp);
        if (it + 1 < iters) lstore(1, ra1, rb1);
        __syncthreads();
        if (!BUF && it + 1 >= iters) break;   // BUF: the second half's MFMAs skip themselves
        if (BUF || it + 3 < iters) gload(((it + 3) * KS + grp) * BK, ra1, rb1);
        chunk_mfma(1, (it + 1) * KS + grp);
        if (it + 2 < iters) lstore(0, ra0, rb0);
        __syncthreads();
    }
    if (KS > 1) {   // sets 1..KS-1's partial quadrants added to set 0's, in set order
        float* red = &As[0][0][0][0];
        if (grp > 0) {
#pragma unroll
            for (int r = 0; r < 16; ++r) red[((grp - 1) * 64 + wave * 16 + r) * 64 + lane] = acc[r];
        }
        __syncthreads();
        if (grp == 0) {
#pragma unroll
            for (int t = 0; t < KS - 1; ++t)
#pragma unroll
                for (int r = 0; r < 16; ++r) acc[r] += red[(t * 64 + wave * 16 + r) * 64 + lane];
        }
    }
    if (scat) {
        // register r of lane l holds C(8(r/4) + 4(l/32) + r%4, l%32) of the
        // wave's quadrant: listed row rel (wave-uniform) lands in register
        // 4(rel/8) + rel%4 of the lanes with l/32 == (rel/4)%2
        auto add_row = [&](int rel, float v) {
            const int rr = ((rel >> 3) << 2) | (rel & 3);
            const float a = v * scl;
            acc[rr] += lk == ((rel >> 2) & 1) ? a : 0.f;   // uniform index: one relative move
        };
#pragma unroll
        for (int q = 0; q < SC / 4; ++q) {
            const unsigned w = __builtin_amdgcn_readfirstlane(srel[q]);
#pragma unroll
            for (int b = 0; b < 4; ++b)
                if (4 * q + b < first_total) add_row((w >> (8 * b)) & 0xff, sv[4 * q + b]);
        }
        if (e.sc_n > 512 || first_total > SC) {
            for (int base = 0; base < e.sc_n; base += 512) {
                const int total = build_list(base);
                for (int c0 = base == 0 ? SC : 0; c0 < total; c0 += 8) {
                    float v[8];
#pragma unroll
                    for (int c = 0; c < 8; ++c) {
                        const int tok = lst[2 * (c0 + c)];
                        v[c] = c0 + c < total && ocol < e.N ? e.sc_rows[static_cast<long long>(tok) * e.sc_ld + ocol]
                                                           : 0.f;
                    }
#pragma unroll
                    for (int c = 0; c < 8; ++c)
                        if (c0 + c < total) add_row(__builtin_amdgcn_readfirstlane(lst[2 * (c0 + c) + 1]), v[c]);
                }
                __builtin_amdgcn_wave_barrier();   // the list is rewritten by the next round
            }
        }
    }
    double sq = 0.0;
    if (grp == 0 && ocol < e.N) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int orow = m0 + wm + 8 * (r >> 2) + 4 * lk + (r & 3);
            if (orow < e.M) {
                __builtin_nontemporal_store(acc[r], &e.C[static_cast<long long>(orow) * e.ldc + ocol]);
                sq += static_cast<double>(acc[r]) * acc[r];
            }
        }
    }
    if (ga.ss_out) block_sumsq_out<4 * KS>(sq, ga.ss_out, ssred);
}

}  // namespace

int sgemm_grouped_tn(const GroupedTN* g, int ngroups, int K, hipStream_t stream, const ColsumSet* cs,
                     GroupedExtras* ex)
{
    if (ex) {
        ex->fused = 0;
        ex->ss_parts = 0;
    }
    if (ngroups <= 0) {
        if (cs && cs->njobs > 0)
            return rmsnorm_bwd_colsum_multi(cs->partial, cs->nparts, cs->out, cs->njobs, cs->cols, cs->acc, stream);
        return LHIP_OK;
    }
    if (ngroups > kGroupedMax) return fail(LHIP_E_ARG, "sgemm_grouped_tn: %d groups (at most %d)", ngroups, kGroupedMax);
    if (K <= 0) return fail(LHIP_E_SHAPE, "sgemm_grouped_tn: K=%d", K);
    GroupedTNArgs ga{};
    bool vec = true;
    long long tiles64 = 0;
    for (int i = 0; i < ngroups; ++i) {
        const GroupedTN& e = g[i];
        if (e.M <= 0 || e.N <= 0) return fail(LHIP_E_SHAPE, "sgemm_grouped_tn: group %d is %dx%d", i, e.M, e.N);
        if (!e.A || !e.B || !e.C) return fail(LHIP_E_NULL, "sgemm_grouped_tn: group %d has a NULL operand", i);
        if (e.lda < e.M || e.ldb < e.N || e.ldc < e.N)
            return fail(LHIP_E_SHAPE, "sgemm_grouped_tn: group %d leading dimensions", i);
        vec = vec && e.lda % 4 == 0 && e.ldb % 4 == 0 && e.M % 4 == 0 && e.N % 4 == 0 && aligned16(e.A) &&
              aligned16(e.B);
        tiles64 += static_cast<long long>(ceil_div(e.M, 64)) * ceil_div(e.N, 64);
    }
    // 64x64 tiles once they give a quarter of the CUs work and fit one
    // workgroup per CU; 32x32 otherwise
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const bool wide = vec && 4 * tiles64 >= cus && tiles64 <= cus;
    const int tile = wide ? 64 : kGroupedTile;
    long long tiles = 0;
    for (int i = 0; i < ngroups; ++i) {
        const GroupedTN& e = g[i];
        ga.e[i] = e;
        ga.tile0[i] = static_cast<int>(tiles);
        ga.tiles_n[i] = ceil_div(e.N, tile);
        tiles += static_cast<long long>(ceil_div(e.M, tile)) * ga.tiles_n[i];
        if (tiles > 0x7fffffffLL) return fail(LHIP_E_CAPACITY, "sgemm_grouped_tn: too many tiles");
    }
    ga.tile0[ngroups] = static_cast<int>(tiles);
    ga.ngroups = ngroups;
    ga.K = K;
    // column sums in the same launch when they take the float4 form too
    bool cs_fused = false;
    if (vec && cs && cs->njobs > 0) {
        if (cs->njobs > kColsumJobs) return fail(LHIP_E_ARG, "sgemm_grouped_tn: %d column-sum jobs", cs->njobs);
        cs_fused = cs->cols > 0 && cs->cols % 4 == 0;
        for (int i = 0; i < cs->njobs && cs_fused; ++i)
            cs_fused = cs->nparts[i] > 0 && cs->partial[i] && cs->out[i] && aligned16(cs->partial[i]) &&
                       aligned16(cs->out[i]);
        if (cs_fused) {
            ga.cs = *cs;
            ga.cs_cb = ceil_div(cs->cols, 32);
            ga.cs_blocks = cs->njobs * ga.cs_cb;
        }
    }
    unsigned grid = static_cast<unsigned>((tiles + ga.cs_blocks + 7) / 8 * 8);   // whole XCD rounds
    if (wide) {
        // per XCD: its tiles, then column-sum workgroups on the CUs left over
        ga.tp = static_cast<int>((tiles + 7) / 8);
        ga.cp = 0;
        ga.cs_per_wg = 1;
        if (ga.cs_blocks > 0) {
            ga.cp = std::max(1, cus / 8 - ga.tp);
            ga.cp = std::min(ga.cp, (ga.cs_blocks + 7) / 8);
            ga.cs_per_wg = (ga.cs_blocks + 8 * ga.cp - 1) / (8 * ga.cp);
        }
        grid = static_cast<unsigned>(8 * (ga.tp + ga.cp));
        // the scatters and the per-workgroup sums of squares, when the column
        // sums run here too (every stored value then passes through this launch)
        if (ex && ex->ss_out && static_cast<int>(grid) <= ex->ss_cap && (!cs || cs->njobs == 0 || cs_fused)) {
            for (int i = 0; i < ngroups; ++i)
                if (g[i].sc_n > 0 && (!g[i].sc_ids || !g[i].sc_rows || g[i].sc_ld < g[i].N))
                    return fail(LHIP_E_ARG, "sgemm_grouped_tn: group %d scatter arguments", i);
            ga.do_sc = 1;
            ga.ss_out = ex->ss_out;
            ex->fused = 1;
            ex->ss_parts = static_cast<int>(grid);
        }
        // buffer loads when every byte offset a chunk load can form (rows up
        // to K plus the loads past the last chunk) stays below 2^31
        bool buf = true;
        for (int i = 0; i < ngroups; ++i) {
            const long long rows = static_cast<long long>(K) + 512;
            buf = buf && (rows * g[i].lda + 64) * 4 < (1LL << 31) && (rows * g[i].ldb + 64) * 4 < (1LL << 31);
        }
        if (K >= 512) {
            if (buf) klaunch(sgemm_grouped_tn_lds64_kernel<4, 32, true>, grid, 1024, 0, stream, ga);
            else klaunch(sgemm_grouped_tn_lds64_kernel<4, 32>, grid, 1024, 0, stream, ga);
        } else if (buf) {
            klaunch(sgemm_grouped_tn_lds64_kernel<2, kGroupedBK, true>, grid, 512, 0, stream, ga);
        } else {
            klaunch(sgemm_grouped_tn_lds64_kernel<2, kGroupedBK>, grid, 512, 0, stream, ga);
        }
    }
    else if (vec) klaunch(sgemm_grouped_tn_lds_kernel, grid, 256, 0, stream, ga);
    else if (K >= 256) klaunch(sgemm_grouped_tn_kernel<8>, grid, 512, 0, stream, ga);
    else klaunch(sgemm_grouped_tn_kernel<4>, grid, 256, 0, stream, ga);
    int rc = check_launch("sgemm_grouped_tn");
    if (rc != LHIP_OK || cs_fused || !cs || cs->njobs <= 0) return rc;
    return rmsnorm_bwd_colsum_multi(cs->partial, cs->nparts, cs->out, cs->njobs, cs->cols, cs->acc, stream);
}

// Below the 64x64-tile threshold, the 32x32 small kernel is used unless K is
// long AND both output dimensions exceed 64: its 32-wide tiles re-read A N/32
// times and B M/32 times, which for long K costs more L2/MALL traffic than
// the 64x64 tiles (+ split-K) save in latency.
bool use_small_kernel(int m, int n, int k) { return k <= 2048 || m <= 64 || n <= 64; }


// 256x256 tiles split over K (one batch): when the tiles alone would fill
// between a quarter and all of the CUs (e.g. 2048^3: 64 tiles), each tile's K
// is cut into slices of at least 512 so that tiles x slices covers the CUs;
// the slices are summed in order by the reduce.  K % 32 == 0 keeps every
// slice whole.  Returns the slice count (1: not this path).
int split256_plan(int m, int n, int k, int batch, size_t ws_floats, int* kchunk_out)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long tiles = static_cast<long long>(ceil_div(m, kBig)) * ceil_div(n, kBig);
    if (batch != 1 || tiles >= cus || 4 * tiles < cus || k % kBigK != 0) return 1;
    long long s = (cus + tiles - 1) / tiles;
    s = std::min<long long>(s, k / 512);
    const long long mn = static_cast<long long>(m) * n;
    if (mn > 0) s = std::min<long long>(s, static_cast<long long>(ws_floats / mn));
    if (s < 2) return 1;
    const int kchunk = ceil_div(ceil_div(k, static_cast<int>(s)), kBigK) * kBigK;
    const int splits = ceil_div(k, kchunk);
    if (splits < 2) return 1;
    *kchunk_out = kchunk;
    return splits;
}

// The 256x256-tile kernel on 128x128 tiles: when there are fewer 256x256
// tiles than CUs but at least ~3/4 of a CU's worth of 128x128 tiles, unless
// the 256x256 tiles split over K into slices of 1024 or more (long K: the
// big tiles' 84% beat the small ones' 79% at 2048x2048x8192).  Measured:
// 2048^3 151.8 (256x256 in 4 slices of 512) -> 143.1 us; the C3 logits
// 512x32000x128 57.3 -> 51.0 us; C3 dW 128x32000x512 52.4 -> 45.7 us.
// Few 128x128 tiles (at most an eighth of the CUs) over a long K: the same
// kernel split over K into one slice per CU's worth of tiles, slices of 448+
// (C3 dhidden 512x128x32000: 4 tiles x 64 slices of 512, 53-57 -> 48 us; a
// split count that leaves CUs idle or doubles up measured slower).  Batch 1.
int big128_split_plan(int m, int n, int k, size_t ws_floats, int* kchunk_out)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    if (m <= 64 || n <= 64) return 1;
    const long long t128 = static_cast<long long>(ceil_div(m, 128)) * ceil_div(n, 128);
    if (8 * t128 > cus) return 1;
    const long long s = cus / t128;
    const int kchunk = static_cast<int>(ceil_div(ceil_div(static_cast<long long>(k), s), 32LL) * 32);
    if (kchunk < 448) return 1;
    const int splits = ceil_div(k, kchunk);
    if (splits < 2 || static_cast<size_t>(splits) * m * n > ws_floats) return 1;
    *kchunk_out = kchunk;
    return splits;
}

bool big128_ok(int m, int n, int batch, int s256, int kc256)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long t256 = static_cast<long long>(ceil_div(m, kBig)) * ceil_div(n, kBig) * batch;
    const long long t128 = static_cast<long long>(ceil_div(m, 128)) * ceil_div(n, 128) * batch;
    return t256 < cus && 4 * t128 >= 3LL * cus && !(s256 > 1 && kc256 >= 1024);
}

// K per split slice from which a split 64x64-tile product runs on four wave sets.
constexpr int kKsSliceMin = 1024;

int splitk_plan(int m, int n, int k, int batch, size_t ws_floats, int* kchunk_out, bool unreduced)
{
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long tiles64 = static_cast<long long>(ceil_div(m, 64)) * ceil_div(n, 64) * batch;
    const long long big_tiles = static_cast<long long>(ceil_div(m, 128)) * ceil_div(n, 128) * batch;
    if (big_tiles >= cus || tiles64 >= cus) return 1;
    const long long mnb = static_cast<long long>(m) * n * batch;
    const long long tiles32 = static_cast<long long>(ceil_div(m, 32)) * ceil_div(n, 32) * batch;
    const int pass = 64 * kSmallU;
    if (unreduced && use_small_kernel(m, n, k) && tiles32 < cus && k > pass) {
        // 16x16 tiles whose consumer sums the slices itself (no reduce
        // launch): one software pass per slice, slices a multiple of 64 deep
        long long s = std::min<long long>(ceil_div(k, pass), 64);
        if (mnb > 0) s = std::min<long long>(s, static_cast<long long>(ws_floats / mnb));
        if (s < 2) return 1;
        const int kchunk = ceil_div(ceil_div(k, static_cast<int>(s)), 64) * 64;
        const int splits = ceil_div(k, kchunk);
        if (splits < 2) return 1;
        *kchunk_out = kchunk;
        return splits;
    }
    long long tiles, min_k;
    int unit;
    if (use_small_kernel(m, n, k)) {
        // 32x32 tiles, K shared by four waves: split only long K (each wave
        // walks K/4 serially; below 1024 the extra reduce launch costs more
        // than the shorter walk saves)
        if (k < 1024) return 1;
        tiles = static_cast<long long>(ceil_div(m, 32)) * ceil_div(n, 32) * batch;
        unit = 32;
        min_k = 256;
        // 16x16 tiles (fewer 32x32 tiles than CUs) take long K unsplit: their
        // passes are software-pipelined, which beats a split plus its reduce
        if (tiles < cus) return 1;
    } else {
        // 64x64 tiles, 32-deep K tiles walked by one workgroup
        tiles = tiles64;
        unit = 32;
        min_k = 128;
        // slices of 1024 or more K at one workgroup per CU run on four wave
        // sets (ks_slices), which beats two single-set workgroups per CU
        const long long s1 = (cus + tiles - 1) / tiles;
        if (k / s1 >= kKsSliceMin) {
            long long s = std::min<long long>(s1, 64);
            if (mnb > 0) s = std::min<long long>(s, static_cast<long long>(ws_floats / mnb));
            if (s >= 2) {
                const int kchunk = ceil_div(ceil_div(k, s), 32) * 32;
                const int splits = ceil_div(k, kchunk);
                if (splits >= 2) {
                    *kchunk_out = kchunk;
                    return splits;
                }
            }
        }
    }
    long long s = (2LL * cus + tiles - 1) / tiles;          // aim at ~2 workgroups per CU
    s = std::min<long long>(s, k / min_k);
    s = std::min<long long>(s, 64);
    if (mnb > 0) s = std::min<long long>(s, static_cast<long long>(ws_floats / mnb));
    if (s < 2) return 1;
    const int kchunk = ceil_div(ceil_div(k, s), unit) * unit;
    const int splits = ceil_div(k, kchunk);
    if (splits < 2) return 1;
    *kchunk_out = kchunk;
    return splits;
}

int sgemm_run(int ta, int tb, int m, int n, int k, float alpha,
              const float* A, int lda, long long sA, const float* B, int ldb, long long sB, float beta,
              float* C, int ldc, long long sC, int batch, const GemmOpts& o, hipStream_t stream)
{
    if (m < 0 || n < 0 || k < 0 || batch < 0)
        return fail(LHIP_E_SHAPE, "sgemm: negative size (m=%d n=%d k=%d batch=%d)", m, n, k, batch);
    if (m == 0 || n == 0 || batch == 0) return LHIP_OK;
    if (!C) return fail(LHIP_E_NULL, "sgemm: C is NULL");
    if (k > 0 && (!A || !B)) return fail(LHIP_E_NULL, "sgemm: A or B is NULL");
    const int a_cols = ta ? m : k;   // stored column count of A
    const int b_cols = tb ? k : n;
    if (k > 0 && lda < (a_cols > 0 ? a_cols : 1))
        return fail(LHIP_E_SHAPE, "sgemm: lda=%d < %d", lda, a_cols);
    if (k > 0 && ldb < (b_cols > 0 ? b_cols : 1))
        return fail(LHIP_E_SHAPE, "sgemm: ldb=%d < %d", ldb, b_cols);
    if (ldc < n) return fail(LHIP_E_SHAPE, "sgemm: ldc=%d < n=%d", ldc, n);
    if (o.R && o.ldr < n) return fail(LHIP_E_SHAPE, "sgemm: ldr=%d < n=%d", o.ldr, n);
    if (batch > 65535) return fail(LHIP_E_CAPACITY, "sgemm: batch %d > 65535", batch);
    if (batch > 1 && (sA < 0 || sB < 0 || sC < 0 || o.sA2 < 0 || o.sB2 < 0 || o.sC2 < 0))
        return fail(LHIP_E_SHAPE, "sgemm: negative batch stride");
    if (o.inner <= 0) return fail(LHIP_E_ARG, "sgemm: inner batch count must be > 0");
    if (o.kblocks <= 0) return fail(LHIP_E_ARG, "sgemm: kblocks must be > 0");
    const long long big_tiles = static_cast<long long>(ceil_div(m, 128)) * ceil_div(n, 128) * batch;
    const long long tiles64 = static_cast<long long>(ceil_div(m, 64)) * ceil_div(n, 64) * batch;
    const int cus = st().cu_count > 0 ? st().cu_count : 256;
    const long long k_all = static_cast<long long>(k) * o.kblocks;
    if (o.kblocks > 1 && k > 0) {
        // One launch when the small kernel takes the whole K range; otherwise
        // (transposed A, K not a multiple of 4, or a large problem) the blocks
        // are accumulated by successive launches.
        const bool one = !ta && k % 4 == 0 && k_all <= 0x7fffffffLL && big_tiles < cus && tiles64 < cus &&
                         use_small_kernel(m, n, static_cast<int>(k_all));
        if (!one) {
            GemmOpts oj = o;
            oj.kblocks = 1;
            for (int j = 0; j < o.kblocks; ++j) {
                if (j == 1) { oj.R = nullptr; oj.ldr = 0; }
                const int rc = sgemm_run(ta, tb, m, n, k, alpha, A + j * o.sAk, lda, sA, B + j * o.sBk, ldb, sB,
                                         j == 0 ? beta : 1.f, C, ldc, sC, batch, oj, stream);
                if (rc != LHIP_OK) return rc;
            }
            return LHIP_OK;
        }
    }
    const bool br = o.kblocks > 1 && k > 0;
    GemmArgs g{};
    g.M = m; g.N = n; g.K = static_cast<int>(br ? k_all : k); g.alpha = alpha; g.beta = beta;
    g.Kb = k; g.sAk = br ? o.sAk : 0; g.sBk = br ? o.sBk : 0;
    g.A = A; g.lda = lda; g.sA = sA; g.sA2 = o.sA2;
    g.B = B; g.ldb = ldb; g.sB = sB; g.sB2 = o.sB2;
    g.C = C; g.ldc = ldc; g.sC = sC; g.sC2 = o.sC2;
    g.R = o.R; g.ldr = o.ldr;
    g.inner = o.inner;
    g.vecA = (k > 0 && lda % 4 == 0 && aligned16(A) && (batch == 1 || (sA % 4 == 0 && o.sA2 % 4 == 0)) &&
              g.sAk % 4 == 0) ? 1 : 0;
    g.vecB = (k > 0 && ldb % 4 == 0 && aligned16(B) && (batch == 1 || (sB % 4 == 0 && o.sB2 % 4 == 0)) &&
              g.sBk % 4 == 0) ? 1 : 0;
    // Large problems: 128x128 tiles (64x64 per wave); mid-size: 64x64 tiles;
    // small (fewer 64x64 tiles than CUs): 32x32 tiles with K shared by the
    // four waves of a workgroup, split over workgroups when K is very long
    // (split-K partials in o.ws).
    if (!br && !o.splits_out && o.ws && ks_split_ok(m, n, k, batch)) {
        int kc = 0;
        const int s = ks_split_plan(m, n, k, o.ws_floats, &kc);
        if (s > 1) {
            g.splits = s; g.kchunk = kc; g.ws = o.ws;
            return launch_cfg_ks<64, 64, 32, 4>(ta, tb, g, batch, stream);
        }
    }
    if (skinny_ok(ta, tb, m, n, batch, br ? o.kblocks : 1) && !o.splits_out && k > 0) {
        g.ws = o.ws;
        g.ws_floats_avail = o.ws ? o.ws_floats : 0;
        return launch_skinny(ta, g, stream);
    }
    const long long tiles256 = static_cast<long long>(ceil_div(m, kBig)) * ceil_div(n, kBig) * batch;
    if (tiles256 >= cus) return launch_256(ta, tb, g, batch, stream);
    int kc256 = 0;
    const int s256 = (!br && o.ws && !o.splits_out) ? split256_plan(m, n, k, batch, o.ws_floats, &kc256) : 1;
    if (!br && big128_ok(m, n, batch, s256, kc256)) return launch_big<128>(ta, tb, g, batch, stream);
    if (s256 > 1) {
        g.splits = s256; g.kchunk = kc256; g.ws = o.ws;
        return launch_256(ta, tb, g, batch, stream);
    }
    if (!br && o.ws && !o.splits_out && batch == 1) {
        int kc128 = 0;
        const int s128 = big128_split_plan(m, n, k, o.ws_floats, &kc128);
        if (s128 > 1) {
            g.splits = s128; g.kchunk = kc128; g.ws = o.ws;
            return launch_big<128>(ta, tb, g, 1, stream);
        }
    }
    if (big_tiles >= cus) return launch_cfg<128, 128, 32>(ta, tb, g, batch, stream);
    // short K (e.g. the LM head, K = dim): the whole K range in one LDS tile,
    // so a workgroup waits on one load round trip instead of one per 32-deep chunk
    if (tiles64 >= cus) {
        // exactly one 64x64 tile per CU: two wave sets per tile, each taking
        // every other 32-deep chunk (the C2 tied head, 512x2000x128: 1 us less
        // per step; 1024^3 27.6-27.7 us against 28.9-29.1 on four sets, and
        // 3-5% at 512x2048x1024 and 2048x512x768); up to two tiles per CU with
        // long K: two wave sets as well
        if (g.K >= 64 && tiles64 <= cus) return launch_cfg_ks<64, 64, 32, 2>(ta, tb, g, batch, stream);
        if (g.K >= 512 && tiles64 <= 2 * cus) return launch_cfg_ks<64, 64, 32, 2>(ta, tb, g, batch, stream);
        // otherwise one wave set: the same kernel's two-chunk-ahead,
        // whole-chunk loads (1536^3 104.5 -> 84.7 us, 1600x1600x800 56.7 ->
        // 47.2 against the single-buffered 64x64 kernel)
        return launch_cfg_ks<64, 64, 32, 1>(ta, tb, g, batch, stream);
    }
    const bool small = use_small_kernel(m, n, g.K);
    g.splits = o.ws ? splitk_plan(m, n, g.K, batch, o.ws_floats, &g.kchunk, o.splits_out != nullptr) : 1;
    g.ws = o.ws;
    if (o.splits_out) {
        if (alpha != 1.f || beta != 0.f || batch != 1 || o.R)
            return fail(LHIP_E_ARG, "sgemm: unreduced split-K needs alpha 1, beta 0, batch 1");
        *o.splits_out = g.splits > 1 ? g.splits : 1;
        g.skip_reduce = g.splits > 1 ? 1 : 0;
    }
    const long long tiles32 = static_cast<long long>(ceil_div(m, 32)) * ceil_div(n, 32) * batch;
    if (small && tiles32 < cus) return launch_tiny(ta, tb, g, batch, stream);
    if (small) return launch_small(ta, tb, g, batch, stream);
    if (g.splits > 1 && g.kchunk >= kKsSliceMin) return launch_cfg_ks<64, 64, 32, 4>(ta, tb, g, batch, stream);
    return launch_cfg_ks<64, 64, 32, 1>(ta, tb, g, batch, stream);
}

int sgemm_launch(int ta, int tb, int m, int n, int k, float alpha,
                 const float* A, int lda, const float* B, int ldb, float beta,
                 float* C, int ldc, int batch, long long sA, long long sB, long long sC,
                 hipStream_t stream)
{
    GemmOpts o;
    o.inner = batch > 0 ? batch : 1;
    return sgemm_run(ta, tb, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, batch, o, stream);
}

// Fixed split-K scratch of lhip_sgemm_noalloc (the array itself is below, at file scope).
constexpr size_t kNoallocScratchBytes = static_cast<size_t>(64) << 20;   // 64 MiB
constexpr int kNoallocMaxDevices = 64;

}  // namespace lhip

// ---- scratch of the allocation-free entry point (lhip_sgemm_noalloc) ----------
// Split-K partials of lhip_sgemm_noalloc live in this file-scope device array
// instead of the library workspace, so that call never allocates.  Each GPU
// holds its own copy for the life of the process.  Host code never uses the
// array's name as an address (on the host it is only a stand-in for the
// symbol): lhip_init resolves its device address once per device with
// hipGetSymbolAddress (noalloc_scratch_init) and every launch takes that
// pointer.  The partials of a split are fully written before the reduce reads
// them, so nothing in the array needs to start at zero.
static __device__ __align__(256) float scratch[lhip::kNoallocScratchBytes / sizeof(float)];

namespace lhip {

static float* g_scratch_dev[kNoallocMaxDevices] = {};

int noalloc_scratch_init(int device)
{
    if (device < 0 || device >= kNoallocMaxDevices)
        return fail(LHIP_E_CAPACITY, "lhip_init: device %d beyond the %d devices the scratch table holds", device,
                    kNoallocMaxDevices);
    if (g_scratch_dev[device]) return LHIP_OK;
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
        (void)hipGetLastError();
        return fail(LHIP_E_DEVICE, "lhip_init: hipGetSymbolAddress(scratch) on device %d: %s", device,
                    e != hipSuccess ? hipGetErrorString(e) : "null address");
    }
    g_scratch_dev[device] = static_cast<float*>(p);
    return LHIP_OK;
}

// The split-K plan of an immediate product: the slice count (1 = unsplit) and
// the partials it needs, in floats.  lhip_sgemm and lhip_sgemm_noalloc share
// it, so both sum the same slices in the same order.
int immediate_plan(int transa, int transb, int m, int n, int k, int batch, size_t* need_floats)
{
    *need_floats = 0;
    if (m <= 0 || n <= 0 || k <= 0 || batch <= 0) return 1;
    const size_t cap = static_cast<size_t>(1) << 26;
    int kchunk = 0, splits = 1;
    if (ks_split_ok(m, n, k, batch)) {
        splits = ks_split_plan(m, n, k, cap, &kchunk);
        if (splits <= 1 && skinny_ok(transa, transb, m, n, batch, 1)) splits = skinny_plan(m, n, k, cap, &kchunk);
    } else if (skinny_ok(transa, transb, m, n, batch, 1)) {
        splits = skinny_plan(m, n, k, cap, &kchunk);
    } else {
        splits = split256_plan(m, n, k, batch, cap, &kchunk);
        if (big128_ok(m, n, batch, splits, kchunk)) splits = 1;
        else if (splits <= 1) {
            splits = batch == 1 ? big128_split_plan(m, n, k, cap, &kchunk) : 1;
            if (splits <= 1) splits = splitk_plan(m, n, k, batch, cap, &kchunk);
        }
    }
    if (splits > 1) *need_floats = static_cast<size_t>(splits) * m * n * batch;
    return splits;
}

}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

// Immediate calls: split-K partials live in the library workspace (sized here,
// before any launch).
static int sgemm_immediate(int transa, int transb, int m, int n, int k, float alpha, const float* A, int lda,
                           long long sA, const float* B, int ldb, long long sB, float beta, float* C, int ldc,
                           long long sC, int batch)
{
    lhip::GemmOpts o;
    o.inner = batch > 0 ? batch : 1;
    size_t need = 0;
    if (lhip::immediate_plan(transa, transb, m, n, k, batch, &need) > 1) {
        o.ws_floats = need;
        int rc = lhip::workspace(o.ws_floats * sizeof(float), reinterpret_cast<void**>(&o.ws));
        if (rc != LHIP_OK) return rc;
    }
    return lhip::sgemm_run(transa, transb, m, n, k, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, batch, o,
                           st().stream);
}

LHIP_API int lhip_sgemm_noalloc(int transa, int transb, int m, int n, int k, float alpha,
                                const float* A, int lda, const float* B, int ldb, float beta,
                                float* C, int ldc)
{
    LHIP_REQUIRE_READY();
    float* const ptr = lhip::g_scratch_dev[st().device];
    if (!ptr) return fail(LHIP_E_DEVICE, "lhip_sgemm_noalloc: scratch of device %d not resolved", st().device);
    lhip::GemmOpts o;
    size_t need = 0;
    if (lhip::immediate_plan(transa, transb, m, n, k, 1, &need) > 1) {
        if (need * sizeof(float) > lhip::kNoallocScratchBytes)
            return fail(LHIP_E_CAPACITY,
                        "lhip_sgemm_noalloc: m=%d n=%d k=%d needs %zu bytes of split-K scratch, beyond its fixed "
                        "%zu bytes; use lhip_sgemm", m, n, k, need * sizeof(float), lhip::kNoallocScratchBytes);
        o.ws = ptr;
        o.ws_floats = need;
    }
    return lhip::sgemm_run(transa, transb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, o,
                           st().stream);
}

LHIP_API int lhip_sgemm(int transa, int transb, int m, int n, int k, float alpha,
                        const float* A, int lda, const float* B, int ldb, float beta,
                        float* C, int ldc)
{
    LHIP_REQUIRE_READY();
    return sgemm_immediate(transa, transb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1);
}

LHIP_API int lhip_sgemm_strided_batched(int transa, int transb, int m, int n, int k, float alpha,
                                        const float* A, int lda, long long strideA,
                                        const float* B, int ldb, long long strideB, float beta,
                                        float* C, int ldc, long long strideC, int batch)
{
    LHIP_REQUIRE_READY();
    return sgemm_immediate(transa, transb, m, n, k, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                           batch);
}

LHIP_API int lhip_sgemm_batched_reduce(int transa, int transb, int m, int n, int k, float alpha,
                                       const float* A, int lda, long long strideA,
                                       const float* B, int ldb, long long strideB, float beta,
                                       float* C, int ldc, int count)
{
    LHIP_REQUIRE_READY();
    if (count <= 0) return fail(LHIP_E_ARG, "lhip_sgemm_batched_reduce: count %d must be >= 1", count);
    if (count > 1 && (strideA < 0 || strideB < 0))
        return fail(LHIP_E_SHAPE, "lhip_sgemm_batched_reduce: negative stride");
    lhip::GemmOpts o;
    o.kblocks = count;
    o.sAk = strideA;
    o.sBk = strideB;
    const long long kall = static_cast<long long>(k) * count;
    if (m > 0 && n > 0 && k > 0 && kall <= 0x7fffffffLL) {
        int kchunk = 0;
        const int splits = lhip::splitk_plan(m, n, static_cast<int>(kall), 1, static_cast<size_t>(1) << 26, &kchunk);
        if (splits > 1) {
            o.ws_floats = static_cast<size_t>(splits) * m * n;
            int rc = lhip::workspace(o.ws_floats * sizeof(float), reinterpret_cast<void**>(&o.ws));
            if (rc != LHIP_OK) return rc;
        }
    }
    return lhip::sgemm_run(transa, transb, m, n, k, alpha, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1, o, st().stream);
}


}  // extern "C"
