// lhip_internal.h -- shared state and helpers of liblanternl_hip.so (not part of the ABI).
//
// One process, one device, one library-owned HIP stream.  Every compute entry
// point validates its arguments on the host (shapes, null pointers, alignment
// assumptions of the chosen kernel) before it launches anything, records a
// message retrievable through lhip_last_error(), and returns a status code.
#pragma once

#include <tuple>
#include <type_traits>
#include <unordered_map>
#include <utility>
#include <vector>
#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

#include "../../include/lanternl_hip.h"

namespace lhip {

struct State {
    bool ready = false;
    int device = -1;
    hipStream_t stream = nullptr;
    int cu_count = 0;
    int clock_khz = 0;
    size_t lds_per_block = 0;
    char name[256] = {0};
    char arch[64] = {0};
    size_t total_mem = 0;
    int l2_bytes = 0;
    // host-table GEMM staging (lhip_matmul_host): grown on demand, freed at shutdown
    float* d_stage = nullptr;
    size_t d_stage_floats = 0;
    float* h_stage = nullptr;  // pinned
    size_t h_stage_floats = 0;
    // scratch for reductions of the immediate entry points (grown on demand)
    void* work = nullptr;
    size_t work_bytes = 0;
    // workspaces replaced by a larger one while recorded programs were live:
    // a program keeps the pointer it was recorded with, so these stay
    // allocated until no program is live (or shutdown)
    std::vector<void*> retired;
    size_t retired_bytes = 0;
    // executable programs made by lhip_program_end and not yet freed
    int live_programs = 0;
    // kOnesMax ones (the gain of the gain-free luaTL row operations), filled at init
    float* ones = nullptr;
    // a program (stream capture of the library stream) is being recorded
    bool recording = false;
    // accounting of lhip_malloc buffers (lhip_mem_stats)
    std::unordered_map<void*, size_t> live;
    unsigned long long bytes_in_use = 0, peak_in_use = 0, n_alloc = 0, n_free = 0;
};

constexpr int kOnesMax = 65536;

State& st();

// Kernel timer (lhip_ktimer_start/stop): while it is on, every launch made
// through klaunch records its dispatch's start and end on an event pair, the
// timestamps a kernel trace reports, for up to `cap` launches.  `total`
// counts every launch made while it is on, timed or not (past the capacity,
// or into a stream capture, where a launch is recorded, not dispatched), so
// that stop can report launches that went untimed.
struct KTimer {
    bool on = false;
    int cap = 0, used = 0, total = 0;
    std::vector<hipEvent_t> ev;   // 2 per launch
};
KTimer& ktimer();

template <typename K, typename Tup, size_t... I>
inline void klaunch_packed(K k, dim3 g, dim3 b, unsigned sh, hipStream_t s, Tup& t, std::index_sequence<I...>)
{
    void* argv[] = {static_cast<void*>(&std::get<I>(t))...};
    KTimer& kt = ktimer();
    bool timed = false;
    if (kt.on) {
        ++kt.total;
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        timed = kt.used < kt.cap && hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone;
    }
    if (timed) {
        hipEvent_t e0 = kt.ev[2 * kt.used], e1 = kt.ev[2 * kt.used + 1];
        ++kt.used;
        (void)hipExtLaunchKernel(reinterpret_cast<const void*>(k), g, b, argv, sh, s, e0, e1, 0);
    } else {
        (void)hipLaunchKernel(reinterpret_cast<const void*>(k), g, b, argv, sh, s);
    }
}

// Launch kernel k on stream s: the same as k<<<g, b, sh, s>>>(args...) (the
// arguments are converted to k's parameter types first); launch errors are
// read by check_launch as usual.
template <typename... KArgs, typename... Args>
inline void klaunch(void (*k)(KArgs...), dim3 g, dim3 b, unsigned sh, hipStream_t s, Args&&... args)
{
    static_assert(sizeof...(KArgs) == sizeof...(Args), "klaunch: argument count differs from the kernel's");
    std::tuple<std::decay_t<KArgs>...> t(std::forward<Args>(args)...);
    klaunch_packed(k, g, b, sh, s, t, std::index_sequence_for<KArgs...>{});
}

// The device ones vector for a gain-free row operation of n columns.
int ones_vector(int n, const float** out);

// Record an error message (printf-style) and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Map a HIP error to LHIP_E_DEVICE / LHIP_E_OOM with context.
int hip_fail(hipError_t e, const char* what);

#define LHIP_REQUIRE_READY()                                                     \
    do {                                                                          \
        if (!::lhip::st().ready)                                                  \
            return ::lhip::fail(LHIP_E_DEVICE, "%s: library not initialised (call lhip_init)", __func__); \
    } while (0)

// Entry points that synchronise the stream, allocate or free memory, or read
// results back to the host cannot be part of a recorded program.
#define LHIP_REFUSE_RECORDING()                                                   \
    do {                                                                          \
        if (::lhip::st().recording)                                               \
            return ::lhip::fail(LHIP_E_UNSUPPORTED,                               \
                                "%s: not allowed while a program is being recorded", __func__); \
    } while (0)

#define LHIP_CHECK_HIP(expr, what)                                                \
    do {                                                                          \
        hipError_t _e = (expr);                                                   \
        if (_e != hipSuccess) return ::lhip::hip_fail(_e, what);                  \
    } while (0)

// After a kernel launch: report launch errors (bad config etc.).
int check_launch(const char* what);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline int ceil_div(long long a, long long b) { return static_cast<int>((a + b - 1) / b); }

// Workgroup id -> (tile row, tile column), row-major over tiles_n columns, in
// XCD-contiguous chunks: workgroups are dispatched round-robin over the 8
// XCDs, so id p runs on XCD p % 8; giving each XCD one contiguous run of
// tiles (whole row bands) keeps each A row band in one XCD's L2.
// Workgroups are dealt to the 8 XCDs round-robin by index, and an XCD's L2
// keeps its lines across launches: the logical index (pid % 8) * (nwg / 8) +
// pid / 8 gives XCD x the contiguous range [x nwg/8, (x+1) nwg/8), so kernels
// that order their work the same way (for the LM step: window-major) read
// the previous kernel's output from their own L2.
__device__ __forceinline__ int xcd_pid(int pid, int nwg)
{
    constexpr int kXcds = 8;
    return (nwg % kXcds) == 0 ? (pid % kXcds) * (nwg / kXcds) + pid / kXcds : pid;
}

__device__ __forceinline__ void xcd_tile(int pid, int nwg, int tiles_n, int& tm, int& tn)
{
    pid = xcd_pid(pid, nwg);
    tm = pid / tiles_n;
    tn = pid - tm * tiles_n;
}

// Resolves, once per device, the device address of the fixed scratch array of
// lhip_sgemm_noalloc (called by lhip_init with the device current).
int noalloc_scratch_init(int device);
// Join the host conversion threads of lhip_matmul_host (lhip_shutdown).
void host_pool_shutdown();

// Library workspace of at least `bytes` (reused; growing it waits for the
// stream, so while a program is being recorded a call that would grow it fails
// with LHIP_E_UNSUPPORTED).  While recorded programs are live, the workspace
// they were recorded with is retired rather than freed when it grows.
int workspace(size_t bytes, void** out);

// Launchers shared by the immediate entry points and the LM step runner.  They
// validate their arguments and enqueue on `stream`; they never allocate.
int fill(float* p, long long n, float v, hipStream_t s);
int zero_bytes(void* p, size_t bytes, hipStream_t s);
int add(const float* a, const float* b, float* o, long long n, hipStream_t s);
int silu(const float* x, float* o, long long n, hipStream_t s);
int rmsnorm_fwd(const float* x, const float* w, float* y, float* inv, int rows, int cols, float eps,
                hipStream_t s);
int rmsnorm_bwd_parts(int rows, int cols);
int rmsnorm_bwd(const float* x, const float* w, const float* inv, const float* dy, float* dx, float* dw,
                int rows, int cols, int accumulate, float* work, size_t work_floats, hipStream_t s);
// The two halves of rmsnorm_bwd: dx = (dres ? dres : 0) + the norm's backward,
// with per-block dw partials into `partial` (skipped when NULL; *parts_out
// receives their count), then the ordered column sum of the partials into dw.
int rmsnorm_bwd_rows(const float* x, const float* w, const float* inv, const float* dy, float* dx,
                     const float* dres, float* partial, size_t partial_floats, int rows, int cols, int* parts_out,
                     hipStream_t s);
int rmsnorm_bwd_colsum(const float* partial, int parts, float* dw, int cols, int accumulate, hipStream_t s);
// several independent column sums in one launch (jobs with parts <= 0 are skipped)
constexpr int kColsumJobs = 16;
int rmsnorm_bwd_colsum_multi(const float* const* partials, const int* parts, float* const* dws, int njobs, int cols,
                             int accumulate, hipStream_t s);
int softmax_fwd(const float* x, float* y, int rows, int cols, float scale, int causal, int offset, int group,
                hipStream_t s);
int softmax_bwd(const float* y, const float* dy, float* dx, int rows, int cols, float scale, int causal,
                int offset, int group, int accumulate, hipStream_t s);
// amax (optional): first index of each row's maximum logit, written in the same pass
// row_len (may be NULL): per-window row counts, window = row / period; a
// counted row's gradient scale is then gscale / row_len[window]
int ce_fused(const float* logits, const int* tgt, float* losses, float* dlogits, int rows, int V,
             int ignore_index, float gscale, hipStream_t s, int* amax = nullptr, const int* row_len = nullptr,
             int period = 0);
int argmax_rows(const float* x, int* out, int rows, int cols, hipStream_t s);
int swiglu_fwd(const float* g, int ldg, const float* u, int ldu, float* h, int ldh, int rows, int cols,
               hipStream_t s);
int swiglu_bwd(const float* g, int ldg, const float* u, int ldu, const float* dh, int lddh, float* dg, int lddg,
               float* du, int lddu, int rows, int cols, int acc, hipStream_t s);
int rope(float* x, const int* pos_ids, int rows, int heads, int hd, int row_stride, int pos_offset, int period,
         double base, int interleaved, int inverse, hipStream_t s);
int embed_fwd(const float* table, const int* ids, float* out, int n, int dim, int vocab, hipStream_t s);
int embed_bwd(const float* g, const int* ids, float* dtable, int n, int dim, int vocab, float scale, int acc,
              hipStream_t s);
int sumsq_blocks(long long n);
int sumsq(const float* x, long long n, double* out, double* partial, int partial_len, hipStream_t s);
// stage 1 only: sumsq_blocks(n) partial sums into `partial`
int sumsq_partials(const float* x, long long n, double* partial, int partial_len, hipStream_t s);
// hyper_dev (may be NULL): device floats {lr, momentum, wd, clip_norm, nesterov}
// that override the by-value arguments (a replayed graph reads them there).
// nparts > 0: sumsq_dev holds that many stage-1 partials, summed in the kernel.
int sgd_step(float* p, float* g, float* v, long long n, const double* sumsq_dev, float lr, float momentum,
             float wd, float grad_scale, float clip_norm, int nesterov, float* gnorm_out, int* applied_out,
             hipStream_t s, const float* hyper_dev, int nparts = 0);
// AdamW (optim2.lua:116-147) with the same step logic; nparts as sgd_step.
// Step count: t_in when tcount is NULL, else read from tcount[parity] and the
// advanced count written to tcount[parity ^ 1].  hyper_dev: {lr, -, wd, clip,
// -, beta1, beta2, eps, parity} overriding the by-value arguments.
int adamw_step(float* p, float* g, float* m, float* v, long long n, const double* sumsq_dev, int nparts, float lr,
               float beta1, float beta2, float eps, float wd, float grad_scale, float clip_norm, int t_in,
               int* tcount, int parity, float* gnorm_out, int* applied_out, hipStream_t s, const float* hyper_dev);
int sum_f32(const float* x, int n, float scale, float* out, hipStream_t s);
// GEMMs of the LMTrain step with their neighbouring stages fused in (16x16
// tiles, K <= 512 in one pass).  Mode bits:
//   FB_NORM       A := rmsnorm(A; nw, eps); h (ld K) and inv receive the
//                 normalized rows and 1/rms
//   FB_DUAL       C = A'.B, C2 = A'.B2, Aout = silu(C) * C2 (batch 1)
//   FB_SWIGLU_BWD G = A'.B^T, then dZ, dU = SwiGLU backward of (Z, U) with G
//   FB_TB         B is N x K (NT)
//   FB_NORMBWD    A := dres + RMSNorm backward (x = nbx, gain nw, 1/rms nbinv,
//                 upstream dy = A); nbout (ld K) receives those rows and nbpart
//                 [ceil(M/16)][K] the per-16-row dw partials
// Otherwise C + y*sC = A'.(B + y*sB) for y < batch.  C/C2/Aout/Z/U/dZ/dU share ldc.
enum { FB_NORM = 1, FB_DUAL = 2, FB_SWIGLU_BWD = 4, FB_TB = 8, FB_NORMBWD = 16 };
enum {
    FUSE_NORM = FB_NORM,
    FUSE_NORM_SWIGLU = FB_NORM | FB_DUAL,
    FUSE_SWIGLU_BWD = FB_SWIGLU_BWD | FB_TB,
    FUSE_NB_SWIGLU_BWD = FB_NORMBWD | FB_SWIGLU_BWD | FB_TB,
    FUSE_NB_NT = FB_NORMBWD | FB_TB,
};
struct FuseCall {
    int mode = 0, M = 0, N = 0, K = 0, batch = 1;
    const float* A = nullptr; int lda = 0;
    const float* B = nullptr; int ldb = 0; long long sB = 0;
    float* C = nullptr; int ldc = 0; long long sC = 0;
    const float* nw = nullptr; float eps = 0.f; float* h = nullptr; float* inv = nullptr;
    const float* B2 = nullptr; float* C2 = nullptr; float* Aout = nullptr;
    const float* Z = nullptr; const float* U = nullptr; float* dZ = nullptr; float* dU = nullptr;
    const float* nbx = nullptr; const float* nbres = nullptr; const float* nbinv = nullptr;
    float* nbout = nullptr; float* nbpart = nullptr;
    int a_parts = 1; long long a_pstride = 0;   // A = sum of a_parts slices a_pstride apart (in order)
    // A row r = A row gather[r] (an embedding lookup; gather_rows rows in A),
    // and with FB_NORM the gathered rows are also written to xout (ld K)
    const int* gather = nullptr; int gather_rows = 0; float* xout = nullptr;
};
bool lm_fuse_ok(int K, int lda, int ldb_nt);
int lm_fused_gemm(const FuseCall& c, hipStream_t s);
// Checkpoint save (save = true) or load of a device parameter vector laid out
// for cfg, through one pinned staging buffer.
int lm_checkpoint_io(const lhip_lm_config_t& cfg, float* dev_params, const char* path, const lhip_ckpt_info_t* info,
                     lhip_ckpt_header_t* header, bool save);
// Fused attention of the LMTrain step (T <= 64, head_dim <= 64, even), one
// workgroup per (window, head, 16-row block); the backward reads the forward's
// ctx (O) for rowsum(dO o O).
bool attn_fused_ok(int T, int hd);
// wlen (may be NULL): keys of each window; keys at or past it are masked (the
// backward reads the masked P, so it needs no limit of its own)
int attn_fwd(const float* qkv, const float2* cs, float* P, float* ctx, int B, int H, int T, int hd, float scale,
             int causal, hipStream_t s, const int* wlen = nullptr);
int attn_bwd(const float* qkv, const float2* cs, const float* P, const float* ctx, const float* dctx, float* dqkv, int B,
             int H, int T, int hd, float scale, int causal, hipStream_t s);

// Options of the GEMM launcher.
//   inner / s?2 : second batch level -- blockIdx.y = outer * inner + i and operand
//                 X is offset by outer * sX2 + i * sX (e.g. window x head);
//   R / ldr     : the beta term reads R instead of C (C = alpha*AB + beta*R);
//   ws          : split-K.  Shapes with fewer output tiles than CUs and K >= 512
//                 are split over K into up to 64 slices; partials go to ws and a
//                 second kernel sums them in slice order (deterministic).
struct GemmOpts {
    int inner = 1;
    long long sA2 = 0, sB2 = 0, sC2 = 0;
    const float* R = nullptr;
    int ldr = 0;
    float* ws = nullptr;
    size_t ws_floats = 0;
    // batch-reduce: C = alpha * sum_{j<kblocks} op(A + j*sAk) . op(B + j*sBk) + beta * R
    int kblocks = 1;
    long long sAk = 0, sBk = 0;
    // split-K without the reduce launch (alpha 1, beta 0, batch 1 only): when K
    // is split, the slices stay in ws as [split][M][N] and *splits_out receives
    // their count (1: the product went to C as usual); the consumer sums them
    int* splits_out = nullptr;
};

// Grouped C_g = A_g^T . B_g (A_g stored K x M_g, B_g stored K x N_g, beta 0)
// for up to kGroupedMax products sharing K, in one launch of 16x16 tiles.
constexpr int kGroupedMax = 32;
struct GroupedTN {
    const float* A; int lda;
    const float* B; int ldb;
    float* C; int ldc;
    int M, N;
    // optional scatter into this product's rows, in token order:
    // C[sc_ids[i]] += sc_scale * sc_rows[i] (row stride sc_ld) for i < sc_n,
    // ids outside [0, M) skipped (the tied table's embedding backward); done
    // only when the launch reports GroupedExtras::fused
    const int* sc_ids = nullptr;
    const float* sc_rows = nullptr;
    int sc_ld = 0, sc_n = 0;
    float sc_scale = 1.f;
};
// Work a grouped launch can fold in on its 64x64-tile path: the groups'
// scatters, and one sum of squares (in double) of every value the launch
// stores per workgroup, into ss_out[0 .. ss_parts) (capacity ss_cap).  On
// return `fused` says whether that happened; if not, the caller runs the
// scatters and the norm itself.
struct GroupedExtras {
    double* ss_out = nullptr;
    int ss_cap = 0;
    int fused = 0;      // out
    int ss_parts = 0;   // out
};
// Column-sum jobs (the RMSNorm gains' dw from per-tile partials) that a
// grouped launch can run in extra workgroups: out_j[c] (+)= sum_b partial_j[b][c].
struct ColsumSet {
    const float* partial[kColsumJobs];
    int nparts[kColsumJobs];
    float* out[kColsumJobs];
    int njobs, cols, acc;
};
// cs (optional): column sums issued with the products -- in the same launch
// when both take their float4 forms, otherwise as a second launch.
int sgemm_grouped_tn(const GroupedTN* g, int ngroups, int K, hipStream_t stream, const ColsumSet* cs = nullptr,
                     GroupedExtras* ex = nullptr);
int sgemm_run(int transa, int transb, int m, int n, int k, float alpha,
              const float* A, int lda, long long sA, const float* B, int ldb, long long sB, float beta,
              float* C, int ldc, long long sC, int batch, const GemmOpts& o, hipStream_t stream);
// The split-K plan of an immediate product (lhip_sgemm's): slice count (1 =
// unsplit) and, in *need_floats, the partials it needs.
int immediate_plan(int transa, int transb, int m, int n, int k, int batch, size_t* need_floats);
// Number of K slices sgemm_run would use (1 = none); *kchunk receives the slice length.
int splitk_plan(int m, int n, int k, int batch, size_t ws_floats, int* kchunk, bool unreduced = false);
int split256_plan(int m, int n, int k, int batch, size_t ws_floats, int* kchunk);

int sgemm_launch(int transa, int transb, int m, int n, int k, float alpha,
                 const float* A, int lda, const float* B, int ldb, float beta,
                 float* C, int ldc, int batch, long long sA, long long sB, long long sC,
                 hipStream_t stream);

}  // namespace lhip
