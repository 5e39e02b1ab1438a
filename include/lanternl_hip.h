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

#ifdef __cplusplus
}
#endif
#endif /* LANTERNL_HIP_H */
