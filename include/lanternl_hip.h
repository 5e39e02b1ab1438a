/*
 * lanternl_hip.h -- C ABI of liblanternl_hip.so, the MI355X (gfx950) backend
 * that takes the `luatl_adapter` slot of lanternl's ai.Matrix backend registry.
 *
 * Plain C: pointers, sizes and status codes only, so that the LuaJIT FFI
 * (ffi.cdef), ctypes or any C caller can bind it unchanged.
 *
 * Conventions (mirroring the reference luaTL ABI, cuda/luaTL_core.cu:108-166):
 *   - every entry point returns an int status (LHIP_OK or a negative code);
 *     the message of the last failure on the calling thread is available from
 *     lhip_last_error() until lhip_clear_error() or the next failure;
 *   - matrices are row-major fp32 with an explicit leading dimension (in
 *     elements); ids and labels are int32, 0-based;
 *   - "device" pointers come from lhip_malloc (or any hipMalloc'd memory on
 *     the same device); every compute call is enqueued on the library's own
 *     HIP stream (lhip_stream()) and returns without waiting: call
 *     lhip_sync() before reading results on the host.  lhip_upload /
 *     lhip_download are synchronous, like luaTL_tensor_upload/download
 *     (cuda/luaTL_core.cu:2031-2094);
 *   - arguments are validated on the host before any launch; a rejected call
 *     launches nothing.
 */
#ifndef LANTERNL_HIP_H
#define LANTERNL_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LHIP_API __attribute__((visibility("default")))

/* Status codes: same meaning and values as luaTL_status (cuda/luaTL_core.cu:108-118). */
enum {
    LHIP_OK = 0,
    LHIP_E_NULL = -1,        /* a required pointer was NULL                    */
    LHIP_E_SHAPE = -2,       /* inconsistent or negative dimensions / strides  */
    LHIP_E_DTYPE = -3,       /* unsupported element type                       */
    LHIP_E_DEVICE = -4,      /* HIP runtime error, or library not initialised  */
    LHIP_E_OOM = -5,         /* device or pinned-host allocation failed        */
    LHIP_E_ARG = -6,         /* invalid scalar argument                        */
    LHIP_E_CAPACITY = -7,    /* size beyond a documented limit                 */
    LHIP_E_UNSUPPORTED = -8  /* valid request this build does not implement    */
};

/* Device description (replaces luaTL_devinfo_t, cuda/luaTL_core.cu:170-203). */
typedef struct {
    char name[256];
    char arch[64];            /* e.g. "gfx950:sramecc+:xnack-"             */
    int device;
    int compute_units;
    int clock_khz;            /* peak shader clock                         */
    int wavefront_size;
    long long total_mem;      /* bytes of HBM                              */
    long long lds_per_block;  /* bytes                                     */
    int l2_bytes;
    double peak_fp32_matrix_tflops; /* CUs x 256 flop/clk x clock            */
    double peak_hbm_gbps;           /* published HBM3E figure for MI355X     */
} lhip_devinfo_t;

/* ---- lifecycle and errors ---------------------------------------------- */
/* Select `device`, create the library stream.  Idempotent for the same device.
 * Replaces luaTL_init (cuda/luaTL_core.cu:1678-1715). */
LHIP_API int lhip_init(int device);
/* Release the stream and staging buffers.  Safe to call twice; later compute
 * calls fail with LHIP_E_DEVICE.  Replaces luaTL_shutdown / luaTL_finalize
 * (cuda/luaTL_core.cu:1717-1736, cuda/luaTL_train.cu:1305-1323). */
LHIP_API int lhip_shutdown(void);
LHIP_API int lhip_is_ready(void);
/* Replaces luaTL_get_last_error / luaTL_clear_error (cuda/luaTL_core.cu:1738-1747). */
LHIP_API const char* lhip_last_error(void);
LHIP_API void lhip_clear_error(void);
/* Replaces luaTL_get_devinfo (cuda/luaTL_core.cu:1755-1763). */
LHIP_API int lhip_device_info(lhip_devinfo_t* out);
LHIP_API const char* lhip_version(void);

/* ---- memory and stream --------------------------------------------------- */
/* hipMalloc'd device buffer, 256-byte aligned.  Replaces the pool-backed
 * luaTL_tensor_alloc / luaTL_gpu_malloc and their frees
 * (cuda/luaTL_core.cu:1841-1853, 2149-2151) with plain owned buffers. */
LHIP_API int lhip_malloc(void** dptr, size_t bytes);
LHIP_API int lhip_free(void* dptr);
/* Device memory free / total in bytes (luaTL_mem_info, cuda/luaTL_core.cu:1765-1772). */
LHIP_API int lhip_mem_info(unsigned long long* free_bytes, unsigned long long* total_bytes);
/* Accounting of the library's device memory, the counterpart of the pool
 * statistics the reference adapter's stats() reports (luaTL_pool_get_stats,
 * cuda/luaTL_core.cu:1862-1869; fields luaTL_core.cu:218-234): there is no
 * caching pool here, so every lhip_malloc is a hipMalloc and every lhip_free
 * a hipFree of a buffer the caller owns. */
typedef struct {
    unsigned long long bytes_in_use;     /* live lhip_malloc buffers          */
    unsigned long long peak_in_use;      /* high-water mark of bytes_in_use   */
    unsigned long long live_buffers;
    unsigned long long n_alloc;          /* lhip_malloc calls that succeeded  */
    unsigned long long n_free;           /* lhip_free calls of live buffers   */
    unsigned long long workspace_bytes;  /* library scratch (split-K, reductions), incl. retired */
    unsigned long long staging_bytes;    /* host-table path device staging    */
} lhip_mem_stats_t;
LHIP_API int lhip_mem_stats(lhip_mem_stats_t* out);
/* Synchronous host<->device copies (replace luaTL_tensor_upload/download and
 * luaTL_to_gpu/to_cpu, cuda/luaTL_core.cu:2031-2094, 2153-2155). */
LHIP_API int lhip_upload(void* dst_device, const void* src_host, size_t bytes);
LHIP_API int lhip_download(void* dst_host, const void* src_device, size_t bytes);
/* Stream-ordered device->device copy and zero fill (luaTL_gpu_copy /
 * luaTL_gpu_zero, cuda/luaTL_core.cu:2157-2159, made asynchronous). */
LHIP_API int lhip_copy(void* dst_device, const void* src_device, size_t bytes);
LHIP_API int lhip_zero(void* dptr, size_t bytes);
/* Wait for all work enqueued on the library stream (luaTL_sync,
 * cuda/luaTL_core.cu:1749-1753). */
LHIP_API int lhip_sync(void);
/* The library's hipStream_t, for callers that interleave their own work. */
LHIP_API void* lhip_stream(void);
/* hipEvents on the library stream (the reference brackets Program runs with
 * cudaEventRecord, cuda/luaTL_train.cu:1574-1601). */
LHIP_API int lhip_event_create(void** ev);
LHIP_API int lhip_event_destroy(void* ev);
LHIP_API int lhip_event_record(void* ev);
LHIP_API int lhip_event_elapsed_ms(void* start, void* stop, float* ms);

/* ---- programs: record a sequence of calls once, replay it as a hipGraph ----
 * Between lhip_program_begin and lhip_program_end, compute calls are recorded
 * from the library stream instead of being executed; lhip_program_end turns
 * the recording into an executable program, and lhip_program_replay enqueues
 * it `times` times on the library stream (asynchronous, like every compute
 * call).  A program keeps the pointers and scalar arguments it was recorded
 * with.  While recording, calls that synchronise, allocate, free or read back
 * to the host (upload, download, sync, malloc, free, event timing,
 * lhip_matmul_host, every lhip_lm_* call) fail with LHIP_E_UNSUPPORTED, and
 * so does a call whose library workspace would have to grow: issue the same
 * calls once before recording them.  A program keeps the library workspace it
 * was recorded with: when a later eager call grows the workspace while
 * programs are live, the old one is retired, not freed, and released when the
 * last program is freed (or at lhip_shutdown).  lhip_program_end(NULL)
 * discards the recording.  Replaces the Program command buffer with its capture/replay
 * (ai/gpu/luaTL_train.lua:327-627; luaTL_prog_run / luaTL_prog_capture /
 * luaTL_prog_replay / luaTL_prog_graph_free, cuda/luaTL_train.cu:1505-1690). */
LHIP_API int lhip_program_begin(void);
LHIP_API int lhip_program_end(void** program);
LHIP_API int lhip_program_replay(void* program, int times);
LHIP_API int lhip_program_free(void* program);
LHIP_API int lhip_is_recording(void);

/* Kernel timer.  No counterpart in the reference (the reference's
 * luaTL.Program `timing` flag, ai/gpu/luaTL_train.lua:332-333, times a whole
 * program run; this times each kernel).  For benchmarks that must agree with
 * a kernel trace: between start and stop, each of the first `capacity` kernel
 * launches records its dispatch's start and end timestamps (launch gaps
 * excluded).  stop synchronises the stream, writes the durations of the
 * timed launches in launch order to ms[0 .. min(timed, capacity)) and the
 * number of kernels launched while the timer was on (timed or not) to
 * *count.  When ms is given and some launch went untimed (past either
 * capacity, or made into a stream capture, where nothing is dispatched),
 * stop still fills ms but returns LHIP_E_CAPACITY, so a caller cannot
 * under-report silently.  Not allowed while a program is being recorded
 * (lhip_program_begin refuses while the timer is on, and so does a
 * graph-mode lhip_lm_step_*). */
LHIP_API int lhip_ktimer_start(int capacity);
LHIP_API int lhip_ktimer_stop(float* ms, int capacity, int* count);

/* ---- GEMM family (fp32 on v_mfma_f32_32x32x2f32) ---------------------------
 * C(m x n) = alpha * op(A)(m x k) * op(B)(k x n) + beta * C, row-major.
 *   transa == 0: A is m x k, lda >= k;   transa != 0: A is stored k x m, lda >= m
 *   transb == 0: B is k x n, ldb >= n;   transb != 0: B is stored n x k, ldb >= k
 *   ldc >= n.  beta == 0 never reads C (NaN in C does not propagate).
 * k == 0 gives C = beta*C.  Replaces luaTL_gemm_ex (cuda/luaTL_train.cu:1075-1094),
 * whose strided views express the same three products matmul (NN), matmul_dx
 * (A.B^T) and matmul_dw (A^T.B) (ai/gpu/luaTL_train.lua:154-182). */
LHIP_API int lhip_sgemm(int transa, int transb, int m, int n, int k, float alpha,
                        const float* A, int lda, const float* B, int ldb, float beta,
                        float* C, int ldc);
/* Batched over blockIdx.z with element strides between consecutive matrices
 * (the batch/stride fields of luaTL_gemm_ex, cuda/luaTL_train.cu:143-146). */
LHIP_API int lhip_sgemm_strided_batched(int transa, int transb, int m, int n, int k, float alpha,
                                        const float* A, int lda, long long strideA,
                                        const float* B, int ldb, long long strideB, float beta,
                                        float* C, int ldc, long long strideC, int batch);
/* Batch-reduce: C = alpha * sum_{j<count} op(A + j*strideA) * op(B + j*strideB)
 * + beta * C, one launch (the products share C and are summed before alpha).
 * This is the accumulation the CPU backward performs one product at a time:
 * grad_of(a) receives matrix.matmul_nt(g, b, grad, acc = true) from every
 * consumer of a (ai/core/tensor2.lua:208-211,222-228), and the reference GPU
 * path chains luaTL.matmul_dx with beta = 1 (ai/gpu/luaTL_train.lua:175-177),
 * e.g. dX = dQ.Wq^T + dK.Wk^T + dV.Wv^T.  count >= 1; strides >= 0. */
LHIP_API int lhip_sgemm_batched_reduce(int transa, int transb, int m, int n, int k, float alpha,
                                       const float* A, int lda, long long strideA,
                                       const float* B, int ldb, long long strideB, float beta,
                                       float* C, int ldc, int count);
/* lhip_sgemm with no allocation of any kind: no counterpart in the reference.
 * It is for callers that cannot allocate device memory (code under graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, kernels and results as lhip_sgemm (bit-identical: the same K
 * slices summed in the same order), but split-K partials go to a fixed 64 MiB
 * device array that each GPU holds from lhip_init to process exit, never to
 * the library workspace.  A shape whose partials would exceed 64 MiB is
 * refused with LHIP_E_CAPACITY before anything is launched (e.g. 4096 x 3840
 * x 4096, two slices of 63 MB each); every unsplit shape fits.  All calls on
 * one GPU share the array and each overwrites what the previous left: they are
 * ordered on the library stream, and work that overlapped them on one GPU
 * (another stream replaying a recording of this call) would race.  Recordable
 * into a program at any time. */
LHIP_API int lhip_sgemm_noalloc(int transa, int transb, int m, int n, int k, float alpha,
                                const float* A, int lda, const float* B, int ldb, float beta,
                                float* C, int ldc);

/* Host-table GEMM for the flat-table backend contract (matrix.lua:178-202 ->
 * luatl_adapter.lua:128-135).  a, b, c are HOST double arrays, row-major:
 *   op 0 (matrix.multiply, matrix.lua:541-595): c(m x n)  = a(m x k)   . b(k x n)
 *   op 1 (matrix.matmul_nt, matrix.lua:597-625): c(m x n) = a(m x k)   . b(n x k)^T
 *   op 2 (matrix.matmul_tn, matrix.lua:627-660): c(k x n) = a(m x k)^T . b(m x n)
 * Inputs are rounded to fp32 (as luatl_adapter.as_tensor does), the product is
 * computed on the GPU in fp32 and widened back to double; acc != 0 adds it
 * into c in double (the Lua `acc` flag).  Synchronous. */
LHIP_API int lhip_matmul_host(int op, const double* a, const double* b, double* c,
                              int m, int k, int n, int acc);

/* How long, in microseconds, the host threads of lhip_matmul_host spin after
 * a call before they sleep (and how long a call spins waiting for their
 * parts before it sleeps).  No counterpart in the reference.  The default,
 * 1000, keeps three workers awake between back-to-back small calls, each
 * busy on a core while it spins; 0 puts them to sleep at once, for hosts that
 * need those cores (a small call then pays their wake-up).  *previous (may be
 * NULL) receives the old value.  Range [0, 100000]. */
LHIP_API int lhip_set_host_spin(int spin_us, int* previous);

/* ---- bandwidth-bound kernels (device pointers, fp32 rows, async) ----------
 * `accumulate` != 0 adds into the output(s) instead of overwriting them, the
 * way the CPU path's BACKWARD.* functions add into grad buffers. */

/* y = x * w / sqrt(mean_j x^2 + eps) per row; inv[row] = 1/sqrt(...) (may be
 * NULL).  CPU semantics: Tensor.rmsnorm (ai/core/tensor2.lua:609-634); replaces
 * luaTL_rmsnorm (cuda/luaTL_core.cu:2329-2341). */
LHIP_API int lhip_rmsnorm_fwd(const float* x, const float* w, float* y, float* inv,
                              int rows, int cols, float eps);
/* dx = dy*w*r - x*(r^3/cols)*sum_j(dy_j w_j x_j); dw = sum over rows of dy*x*r
 * (dw may be NULL).  Deterministic (no atomics).  CPU: BACKWARD.rmsnorm
 * (ai/core/tensor2.lua:641-666); replaces luaTL_rmsnorm_bwd (cuda/luaTL_train.cu:1096-1106). */
LHIP_API int lhip_rmsnorm_bwd(const float* x, const float* w, const float* inv, const float* dy,
                              float* dx, float* dw, int rows, int cols, int accumulate);
/* y = softmax(scale * x) over the kept prefix of each row, 0 beyond it (x and y
 * must not overlap; likewise y, dy and dx in the backward).  Without
 * `causal` the whole row is kept; with it row r keeps
 * min(max((r % group) + 1 + offset, 1), cols) columns (group <= 0 means rows).
 * CPU: Tensor.scale + Tensor.softmax_rows (ai/core/tensor2.lua:185-196, 332-383);
 * replaces luaTL_softmax_ex (cuda/luaTL_train.cu:1108-1118). */
LHIP_API int lhip_softmax_fwd(const float* x, float* y, int rows, int cols, float scale,
                              int causal, int offset, int group);
/* dx = scale * y * (dy - sum_{kept} dy*y) on the kept prefix, 0 beyond.
 * CPU: BACKWARD.softmax + BACKWARD.scale (ai/core/tensor2.lua:388-408, 185-196);
 * replaces luaTL_softmax_bwd (cuda/luaTL_train.cu:1120-1129). */
LHIP_API int lhip_softmax_bwd(const float* y, const float* dy, float* dx, int rows, int cols,
                              float scale, int causal, int offset, int group, int accumulate);
/* out = silu(gate) * up over rows x cols with leading dimensions (silu by the
 * sign-stable sigmoid).  CPU: Tensor.silu + Tensor.mul (ai/core/tensor2.lua:
 * 272-291, 167-170) as composed at ai/nn/transformer.lua:246-248; replaces
 * luaTL_swiglu_fwd (cuda/luaTL_train.cu:1131-1140). */
LHIP_API int lhip_swiglu_fwd(const float* gate, int ld_gate, const float* up, int ld_up,
                             float* out, int ld_out, int rows, int cols);
/* dgate = s*(1 + gate*(1-s)) * (up*dout), dup = silu(gate)*dout, s = sigmoid(gate).
 * CPU: BACKWARD.mul then BACKWARD.silu (ai/core/tensor2.lua:172-183, 293-303);
 * replaces luaTL_swiglu_bwd (cuda/luaTL_train.cu:1142-1152). */
LHIP_API int lhip_swiglu_bwd(const float* gate, int ld_gate, const float* up, int ld_up,
                             const float* dout, int ld_dout, float* dgate, int ld_dgate,
                             float* dup, int ld_dup, int rows, int cols, int accumulate);
/* In-place rotary embedding of `heads` heads of `head_dim` columns in each row
 * (row_stride >= heads*head_dim).  Position of row r: pos_ids[r] if pos_ids,
 * else (pos_period > 0 ? r % pos_period : r) + pos_offset.  Pair p rotates by
 * pos / base^(2p/head_dim) (angles in double, as ai/nn/transformer.lua:30-48).
 * interleaved != 0: pairs (2p, 2p+1) -- the CPU path (ai/core/tensor2.lua:410-446);
 * else half-split pairs (p, p+head_dim/2).  inverse != 0 rotates by -angle,
 * which is the backward (ai/core/tensor2.lua:451-473).  Replaces luaTL_rope
 * (cuda/luaTL_train.cu:1154-1167); head_dim <= 256, even. */
LHIP_API int lhip_rope(float* x, const int* pos_ids, int rows, int heads, int head_dim, int row_stride,
                       int pos_offset, int pos_period, double base, int interleaved, int inverse);
/* Fused softmax + cross-entropy per row: losses[r] = logsumexp(x_r) - x_r[t_r],
 * dlogits = grad_scale * (softmax(x_r) - onehot(t_r)); rows whose target is < 0,
 * >= vocab or == ignore_index give 0 and 0.  losses / dlogits may be NULL;
 * dlogits may alias logits.  CPU: Tensor.cross_entropy + BACKWARD
 * (ai/core/tensor2.lua:809-882); replaces luaTL_cross_entropy (cuda/luaTL_train.cu:1189-1201). */
LHIP_API int lhip_ce_fused(const float* logits, const int* targets, float* losses, float* dlogits,
                           int rows, int vocab, int ignore_index, float grad_scale);
/* out[r] = first index of the row maximum (strict '>' scan: NaN never wins, a
 * row of only -inf/NaN gives 0), int32.  CPU: the accuracy loop of
 * ai/optim/lmtrain.lua:1200-1209; replaces luaTL_argmax_rows (cuda/luaTL_train.cu:1241-1249). */
LHIP_API int lhip_argmax_rows(const float* x, int* out, int rows, int cols);
/* out[i] = table[ids[i]] (exact); ids outside [0, vocab) give a zero row.
 * CPU: Tensor.embed (ai/core/tensor2.lua:572-590); replaces luaTL_embed_fwd
 * (cuda/luaTL_train.cu:1169-1177). */
LHIP_API int lhip_embed_fwd(const float* table, const int* ids, float* out, int n, int dim, int vocab);
/* dtable[v] = (accumulate ? dtable[v] : 0) + scale * sum_{i: ids[i]==v} dout[i],
 * summed in token order, deterministic (no atomics).  CPU: BACKWARD.embed
 * (ai/core/tensor2.lua:592-607); replaces luaTL_embed_bwd (cuda/luaTL_train.cu:1179-1187). */
LHIP_API int lhip_embed_bwd(const float* dout, const int* ids, float* dtable, int n, int dim, int vocab,
                            float scale, int accumulate);

/* ---- elementwise helpers, reductions and the SGD step ------------------- */
/* x[0..n) = value (a kernel, safe inside graph capture). */
LHIP_API int lhip_fill(float* x, long long n, float value);
/* out = a + b elementwise (the residual adds of ai/nn/transformer.lua:243-249). */
LHIP_API int lhip_add(const float* a, const float* b, float* out, long long n);
/* out = silu(x) = x * sigmoid(x) elementwise over n floats (in place allowed),
 * sigmoid by sign as Tensor.silu (ai/core/tensor2.lua:272-291); the adapter's
 * silu_inplace (ai/gpu/luatl_adapter.lua:168, Tensor:silu_inplace
 * ai/gpu/luaTL.lua:669). */
LHIP_API int lhip_silu(const float* x, float* out, long long n);
/* *out (device double) = sum of x^2, deterministic two-stage reduction
 * (optim2.grad_norm squared, ai/optim/optim2.lua:27-38; replaces luaTL_l2_accum,
 * cuda/luaTL_train.cu:1215-1221). */
LHIP_API int lhip_sumsq(const float* x, long long n, double* out);
/* *out (device float) = scale * sum(x[0..n)) (luaTL_sum_f32, cuda/luaTL_train.cu:1233-1239). */
LHIP_API int lhip_sum(const float* x, int n, float scale, float* out);
/* One SGD step with the LMTrain step logic (ai/optim/lmtrain.lua:1212-1226,
 * ai/optim/optim2.lua:72-99): norm = grad_scale * sqrt(*grad_sumsq) (device
 * double holding the sum of squares of the raw grads); if the norm is not
 * finite nothing changes; else g = grads*grad_scale, clipped by clip_norm/norm
 * when norm > clip_norm > 0, written back to grads; then g += wd*p;
 * v = momentum*v + g; p -= lr*v (or lr*(g + momentum*v) with nesterov; p -= lr*g
 * when momentum == 0).  grad_norm_out / applied_out (device, may be NULL)
 * receive the pre-clip norm and 1/0. */
LHIP_API int lhip_sgd_step(float* params, float* grads, float* velocity, long long n,
                           const double* grad_sumsq, float lr, float momentum, float weight_decay,
                           float grad_scale, float clip_norm, int nesterov,
                           float* grad_norm_out, int* applied_out);
/* One AdamW step (ai/optim/optim2.lua:116-147, LMTrain's default optimizer,
 * optim2.create at :166-171) with the same step logic as lhip_sgd_step: if the
 * norm is finite, g = grads*grad_scale (clipped, written back), then
 * m = beta1*m + (1-beta1)*g, v = beta2*v + (1-beta2)*g^2,
 * p -= lr*wd*p, p -= (lr/(1-beta1^step)) * m / (sqrt(v/(1-beta2^step)) + eps).
 * `step` is the 1-based AdamW step count this update uses (optim2's self.t
 * after its increment); the caller advances it only when *applied_out is 1.
 * Replaces the reference's luaTL_adamw_kernel (cuda/luaTL_core.cu:1346-1380),
 * whose per-element clip and bias-correction arguments differ; this follows
 * the CPU path. */
LHIP_API int lhip_adamw_step(float* params, float* grads, float* m, float* v, long long n,
                             const double* grad_sumsq, float lr, float beta1, float beta2, float eps,
                             float weight_decay, float grad_scale, float clip_norm, int step,
                             float* grad_norm_out, int* applied_out);

/* ---- the luaTL operation set ----------------------------------------------
 * The calls behind the reference adapter's resident API
 * (ai/gpu/luatl_adapter.lua:126-187) and luaTL.Program's op list
 * (ai/gpu/luaTL_train.lua:365-606), with luaTL's semantics (fp32 only; every
 * reduction deterministic).  Device pointers, asynchronous on the library
 * stream like every compute call. */

/* Post-GEMM activations and GEMM prologues: the values of luaTL's act/pre
 * codes (cuda/luaTL_core.cu:76-90). */
enum { LHIP_ACT_NONE = 0, LHIP_ACT_RELU = 1, LHIP_ACT_GELU = 2, LHIP_ACT_SILU = 3, LHIP_ACT_TANH = 4,
       LHIP_ACT_SIGMOID = 5 };
enum { LHIP_PRE_NONE = 0, LHIP_PRE_RMSNORM = 1, LHIP_PRE_GELU = 2, LHIP_PRE_SILU = 3, LHIP_PRE_RELU = 4 };

/* C = act(alpha * pre(A) . B + bias) + beta * C over `batch` matrices, each
 * operand a strided view: element (i, j) of A (M x K) at A[i*a_rs + j*a_cs]
 * (+ b*a_bs for batch b), likewise B (K x N) and C (M x N).  pre RMSNORM
 * scales row i of A by rowscale[i] (or, when rowscale is NULL, by
 * 1/sqrt(mean_k A[i,k]^2 + eps)) and column k by gamma[k] (1 when NULL); the
 * other prologues map A elementwise.  bias (N floats) and act may be
 * NULL / NONE; beta == 0 never reads C.  Without a prologue each operand must
 * be row- or column-major (one unit stride; anything else is
 * LHIP_E_UNSUPPORTED); the product runs on the fp32 MFMA GEMM family, a
 * prologue or epilogue as an extra streaming pass.  Replaces luaTL_gemm_ex
 * (cuda/luaTL_train.cu:1075-1094; kernel semantics :127-234). */
LHIP_API int lhip_gemm_ex(const float* A, const float* B, float* C, const float* bias, const float* gamma,
                          const float* rowscale, int M, int N, int K, long long a_rs, long long a_cs,
                          long long b_rs, long long b_cs, long long c_rs, long long c_cs, long long a_bs,
                          long long b_bs, long long c_bs, int batch, float alpha, float beta, float eps,
                          int pre_op, int post_op);

/* Elementwise operators: the values of luaTL's EW codes (cuda/luaTL_core.cu:49-72). */
enum { LHIP_EW_COPY = 0, LHIP_EW_ADD = 1, LHIP_EW_SUB = 2, LHIP_EW_MUL = 3, LHIP_EW_DIV = 4, LHIP_EW_SCALE = 5,
       LHIP_EW_AXPY = 6, LHIP_EW_FILL = 7, LHIP_EW_RELU = 8, LHIP_EW_GELU = 9, LHIP_EW_SILU = 10,
       LHIP_EW_TANH = 11, LHIP_EW_SIGMOID = 12, LHIP_EW_EXP = 13, LHIP_EW_SQRT = 14, LHIP_EW_RSQRT = 15,
       LHIP_EW_NEG = 16, LHIP_EW_RECIP = 17, LHIP_EW_ABS = 18, LHIP_EW_CLAMP = 19, LHIP_EW_DRELU = 20,
       LHIP_EW_DSILU = 21, LHIP_EW_DGELU = 22 };
/* c[i] = op(a[i], b[i], alpha, beta) for i < n (a or b NULL reads as 0):
 * ADD alpha*a+beta*b, SUB alpha*a-beta*b, MUL alpha*a*b, DIV alpha*a/(b+1e-20),
 * SCALE alpha*a+beta, AXPY alpha*a+b, FILL alpha, CLAMP min(max(a,alpha),beta),
 * DRELU b*(a>0), DSILU b*silu'(a), DGELU b*gelu'(a), the rest unary in a
 * (GELU in its tanh form).  In place allowed.  Replaces luaTL_elementwise
 * (cuda/luaTL_core.cu:2308; operators :909-934). */
LHIP_API int lhip_elementwise(const float* a, const float* b, float* c, long long n, int op, float alpha, float beta);
/* y = x * w / sqrt(mean_j x^2 + eps) per row, w NULL meaning gain 1 (up to
 * 65536 columns), no 1/rms output.  Replaces luaTL_rmsnorm (cuda/luaTL_core.cu:
 * 2329-2341, kernel :1092-1114). */
LHIP_API int lhip_rmsnorm_ex(const float* x, const float* w, float* y, int rows, int cols, float eps);
/* luaTL's RMSNorm backward: 1/rms recomputed from x and eps, dx overwritten,
 * dw (may be NULL) accumulated (+=), w NULL meaning gain 1.  Replaces
 * luaTL_rmsnorm_bwd (cuda/luaTL_train.cu:1096-1106, kernel :489-526). */
LHIP_API int lhip_rmsnorm_bwd_ex(const float* x, const float* w, const float* dy, float* dx, float* dw, int rows,
                                 int cols, float eps);
/* out[r] = 1/sqrt(mean_k x[r*rs + k*cs]^2 + eps).  Replaces luaTL_row_rms
 * (cuda/luaTL_train.cu:1261, kernel :355-369). */
LHIP_API int lhip_row_rms(const float* x, float* out, int rows, int cols, long long rs, long long cs, float eps);
/* luaTL's softmax: v = x*scale + bias[j] (bias NULL: none) over the columns
 * j <= limit of row r, limit = ((group > 0 ? r % group : r) + mask_offset)
 * when causal, else cols-1; masked entries 0, a row with nothing kept all 0.
 * Replaces luaTL_softmax_ex (cuda/luaTL_train.cu:1108-1118, kernel :545-585). */
LHIP_API int lhip_softmax_ex(const float* x, const float* bias, float* y, int rows, int cols, float scale, int causal,
                             int group, int mask_offset);
/* dx = scale * y * (dy - sum_{j<=limit} dy_j y_j) on the kept columns, 0 beyond
 * (dx overwritten).  Replaces luaTL_softmax_bwd (cuda/luaTL_train.cu:1120-1129). */
LHIP_API int lhip_softmax_bwd_ex(const float* y, const float* dy, float* dx, int rows, int cols, float scale,
                                 int causal, int group, int mask_offset);
/* luaTL's SwiGLU backward with either output optional: da = dout*b*silu'(a)
 * (stored with lda), db = dout*silu(a) (stored with ldb).  Replaces
 * luaTL_swiglu_bwd (cuda/luaTL_train.cu:1142-1152). */
LHIP_API int lhip_swiglu_bwd_ex(const float* a, const float* b, const float* dout, float* da, float* db, int rows,
                                int cols, int lda, int ldb, int ldo);
/* out[c] = alpha * sum_r x[r*row_stride + c] + beta * out[c] (beta == 0 does
 * not read out).  Replaces luaTL_reduce_cols (cuda/luaTL_train.cu:1203-1213). */
LHIP_API int lhip_reduce_cols(const float* x, float* out, int rows, int cols, long long row_stride, float alpha,
                              float beta);
/* *acc (device float) += sum x^2.  Replaces luaTL_l2_accum (cuda/luaTL_train.cu:1215-1221). */
LHIP_API int lhip_l2_accum(const float* x, long long n, float* acc);
/* x *= max_norm / (sqrt(*nsq) + 1e-6) when sqrt(*nsq) > max_norm > 0 (nsq a
 * device float), else unchanged.  Replaces luaTL_clip_by_nsq (cuda/luaTL_train.cu:1223-1231). */
LHIP_API int lhip_clip_by_nsq(float* x, long long n, const float* nsq, float max_norm);
/* *acc (device float) += scale * sum x.  The accumulating form of luaTL_sum_f32
 * (cuda/luaTL_train.cu:1233-1239, kernel :969-979). */
LHIP_API int lhip_sum_accum(const float* x, long long n, float scale, float* acc);
/* out (cols x rows) = x (rows x cols)^T, out of place.  Replaces luaTL's
 * transpose op (cuda/luaTL_core.cu:1036-1060). */
LHIP_API int lhip_transpose(const float* x, float* out, int rows, int cols);
/* out[r][c] = x[r][c] + alpha * v[c] (v NULL reads as 0).  Replaces luaTL's
 * bcast_add (cuda/luaTL_core.cu:1018-1033). */
LHIP_API int lhip_bcast_add(const float* x, const float* v, float* out, int rows, int cols, float alpha);
/* luaTL's AdamW update: per-element gradient clamp to [-clip, clip] when
 * clip > 0, m/v moments, decoupled decay, then w -= lr * m*bc1 / (sqrt(v*bc2)
 * + eps) with bc = 1/(1 - beta^max(step,1)); w_mirror (may be NULL) gets a
 * copy of w.  Replaces luaTL_adamw_kernel (cuda/luaTL_core.cu:1346-1380) as
 * Program:adamw issues it (cuda/luaTL_train.cu:1427-1449).  The LMTrain
 * step's AdamW is lhip_adamw_step, which follows optim2 instead. */
LHIP_API int lhip_adamw_elementwise(float* w, const float* g, float* m, float* v, float* w_mirror, long long n,
                                    int step, float lr, float beta1, float beta2, float eps, float weight_decay,
                                    float clip);

/* ---- the CPU LMTrain step, resident on the GPU ------------------------------
 * One optimizer step of LMTrain with optimizer = "sgd" over `batch` windows of
 * `seq` tokens, with the CPU path's model (ai/nn/transformer.lua:84-257:
 * separate wq/wk/wv and w1/w3/w2, interleaved RoPE, tied head) and step logic
 * (ai/optim/lmtrain.lua:1183-1227: per-window mean CE, grads summed over
 * windows and scaled by 1/batch, global-norm skip and clip, SGD with momentum
 * and weight decay, ai/optim/optim2.lua:48-102).  Parameters are one flat fp32
 * vector in Transformer:parameters() order (ai/nn/transformer.lua:150-164):
 * emb, {ln1, wq, wk, wv, wo, ln2, w1, w3, w2} per layer, lnf.  The model owns
 * every device buffer; a step enqueues everything on the library stream with
 * no host round trip and no allocation (optionally as a replayed hipGraph).
 * The reference offers this only as Lua orchestration over luaTL calls; it has
 * no single C entry point for it. */
typedef struct {
    int vocab, dim, layers, heads, ffn;
    int causal;          /* transformer.lua:93 (default 1) */
    double eps;          /* RMSNorm eps, transformer.lua:98 (1e-5) */
    double rope_base;    /* transformer.lua:95 (10000) */
    int batch;           /* windows per optimizer step (LMTrain batch_size) */
    int seq;             /* tokens per window (LMTrain max_seq) */
} lhip_lm_config_t;

typedef struct {
    float loss;          /* sum_w len_w * (window w's mean CE) / sum_w len_w (LMTrain's batch loss) */
    float grad_norm;     /* global norm of the 1/batch-scaled grads, before clipping */
    int applied;         /* 1 when the update ran (finite norm), else 0 */
    int correct;         /* argmax hits over the batch's tokens */
    int steps;           /* steps enqueued since creation */
} lhip_lm_stats_t;

/* Number of parameters (-1 on a bad config) and each tensor's offset/shape
 * (2 + 9*layers tensors; any output may be NULL). */
LHIP_API long long lhip_lm_num_params(const lhip_lm_config_t* cfg);
LHIP_API int lhip_lm_param_offsets(const lhip_lm_config_t* cfg, long long* offsets, int* rows, int* cols);
LHIP_API int lhip_lm_create(const lhip_lm_config_t* cfg, void** model);
LHIP_API int lhip_lm_destroy(void* model);
/* Synchronous copies of the flat parameter / gradient / velocity vectors. */
LHIP_API int lhip_lm_set_params(void* model, const float* host, long long n);
LHIP_API int lhip_lm_get_params(void* model, float* host, long long n);
LHIP_API int lhip_lm_get_grads(void* model, float* host, long long n);
LHIP_API int lhip_lm_set_velocity(void* model, const float* host, long long n);
LHIP_API int lhip_lm_get_velocity(void* model, float* host, long long n);
/* Token ids and next-token targets, batch*seq each, 0-based, row b*seq + t:
 * `batch` full windows of `seq` tokens. */
LHIP_API int lhip_lm_set_batch(void* model, const int* ids, const int* targets);
/* The same with LMTrain's ragged batches: n_windows (1..batch) windows, window
 * b holding lengths[b] (1..seq) tokens at rows b*seq .. b*seq+lengths[b]-1
 * (the rest of its rows, and the slots past n_windows, are ignored);
 * lengths NULL means full windows.  Each window's loss is the mean CE over
 * its own tokens, the summed gradients are scaled by 1/n_windows when
 * n_windows > 1, and lhip_lm_stats reports LMTrain's token-weighted batch
 * loss: build_windows' short last window and the short last batch of the
 * batch loop (ai/optim/lmtrain.lua:535-558,1183-1212; tensor2.lua:845-857).
 * A non-causal model whose seq or head_dim exceeds the fused attention's
 * limit (64) takes only full windows (LHIP_E_UNSUPPORTED otherwise). */
LHIP_API int lhip_lm_set_batch_ex(void* model, const int* ids, const int* targets, const int* lengths,
                                  int n_windows);
/* Capture the step into a hipGraph on the next call and replay it afterwards. */
LHIP_API int lhip_lm_use_graph(void* model, int on);
/* Enqueue one step (asynchronous). */
LHIP_API int lhip_lm_step_sgd(void* model, float lr, float momentum, float weight_decay, float clip_norm,
                              int nesterov);
/* The same step with optimizer = "adamw" (ai/optim/optim2.lua:104-164; LMTrain
 * defaults lr 1e-3, beta1 0.9, beta2 0.95, eps 1e-8, wd 0.01,
 * ai/optim/lmtrain.lua:25-26).  The AdamW step count lives on the device and
 * advances only for applied steps, as optim2's self.t does. */
LHIP_API int lhip_lm_step_adamw(void* model, float lr, float beta1, float beta2, float eps, float weight_decay,
                                float clip_norm);
/* AdamW moments (n = parameter count each; either pointer may be NULL) and the
 * step count: set (e.g. on resume) and get (synchronous). */
LHIP_API int lhip_lm_set_adam_state(void* model, const float* m, const float* v, long long n, int step);
LHIP_API int lhip_lm_get_adam_state(void* model, float* m, float* v, long long n, int* step);
/* Wait and report the last step; window_losses (may be NULL) gets `batch`
 * values, each window's mean CE (0 for empty slots). */
LHIP_API int lhip_lm_stats(void* model, lhip_lm_stats_t* out, float* window_losses, int nwin);
/* Row argmax of the last step's logits (batch*seq int32). */
LHIP_API int lhip_lm_get_argmax(void* model, int* host, int n);

/* ---- LMTrain checkpoints (lmio v3) -------------------------------------------
 * The checkpoint format of ai/optim/lmio.lua (tag line "lanternl-checkpoint 3",
 * a key=value header, then every tensor of Transformer:parameters() as
 * "<rows> <cols>\n" + raw little-endian fp32 (format bin) or
 * "<rows> <cols>|v,v,...\n" with %.9g (format text); lmio.lua:5-13,226-313).
 * Writes are atomic: "<path>.tmp<pid>" in the same directory, every write
 * checked, the older files rotated (keep = K > 1: path.(K-1) removed,
 * path.i -> path.(i+1), path -> path.1), then renamed over path
 * (lmio.lua:127-135,320-368).  Reads take v3 and v2 (tagged) and v1 (untagged)
 * files, bin or text, f32 or f64 values (lmio.lua:393-611), and check the
 * model sizes, the tensor count and every tensor's shape.  The model is the
 * tied-head RoPE transformer of lhip_lm_config_t; a checkpoint with pos other
 * than rope or tie=0 is refused (LHIP_E_UNSUPPORTED). */
typedef struct {
    int format;          /* 0 = bin (lmio's default with ffi), 1 = text */
    int keep;            /* keep_last rotation depth; <= 1 overwrites path only */
    int epoch;           /* header epoch= */
    double loss;         /* header loss= (%.9g; non-finite -> nan) */
    double best_loss;    /* header best_loss= (%.9g; non-finite -> nan) */
    const char* backend; /* header backend= (NULL -> "luatl_adapter") */
    const char* extra;   /* appended to the header line as is (may be NULL) */
} lhip_ckpt_info_t;

typedef struct {
    int version;         /* 1, 2 or 3 */
    int format;          /* 0 bin, 1 text */
    int dtype_bytes;     /* 4 (f32) or 8 (f64) */
    int epoch;           /* -1 when absent */
    double loss, best_loss;   /* NaN when absent or nan */
    int causal, tie, max_seq; /* -1 when absent */
    double rope_base;    /* NaN when absent */
} lhip_ckpt_header_t;

/* Host-side save/load of a flat parameter vector of lhip_lm_num_params(cfg)
 * values (no device involved; the LMTrain:_write_checkpoint / LMTrain:load
 * counterparts, lmio.lua:315-368,393-611).  cfg->seq is written as max_seq. */
LHIP_API int lhip_ckpt_save_host(const char* path, const lhip_lm_config_t* cfg, const lhip_ckpt_info_t* info,
                                 const float* params, long long n);
LHIP_API int lhip_ckpt_load_host(const char* path, const lhip_lm_config_t* cfg, float* params, long long n,
                                 lhip_ckpt_header_t* header);
/* The same for a device model, streamed through a fixed pinned buffer (the GPU
 * path's _param_get/_param_set hooks, lmio.lua:186-211, lmtrain_gpu.lua:46-59).
 * A failed load may leave the parameters partly replaced, as LMTrain:load does. */
LHIP_API int lhip_lm_save(void* model, const char* path, const lhip_ckpt_info_t* info);
LHIP_API int lhip_lm_load(void* model, const char* path, lhip_ckpt_header_t* header);

#ifdef __cplusplus
}
#endif
#endif /* LANTERNL_HIP_H */
