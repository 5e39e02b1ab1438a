// lhip_internal.h -- shared state and helpers of liblanternl_hip.so (not part of the ABI).
//
// One process, one device, one library-owned HIP stream.  Every compute entry
// point validates its arguments on the host (shapes, null pointers, alignment
// assumptions of the chosen kernel) before it launches anything, records a
// message retrievable through lhip_last_error(), and returns a status code.
#pragma once

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
};

State& st();

// Record an error message (printf-style) and return `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
// Map a HIP error to LHIP_E_DEVICE / LHIP_E_OOM with context.
int hip_fail(hipError_t e, const char* what);

#define LHIP_REQUIRE_READY()                                                     \
    do {                                                                          \
        if (!::lhip::st().ready)                                                  \
            return ::lhip::fail(LHIP_E_DEVICE, "%s: library not initialised (call lhip_init)", __func__); \
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

// GEMM launcher shared by the immediate entry points and the LM step runner.
int sgemm_launch(int transa, int transb, int m, int n, int k, float alpha,
                 const float* A, int lda, const float* B, int ldb, float beta,
                 float* C, int ldc, int batch, long long sA, long long sB, long long sC,
                 hipStream_t stream);

}  // namespace lhip
