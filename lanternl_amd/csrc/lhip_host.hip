// lhip_host.hip -- the host-table GEMM of the flat-table backend contract
// (lhip_matmul_host): host double arrays in and out, fp32 on the GPU.
//
// Replaces the reference adapter's flat-table matmul (ai/gpu/luatl_adapter.lua:
// 103-135: as_tensor rounds each Lua double to fp32 into a device tensor, the
// GEMM runs, the result is read back and widened).  Here the fp64 <-> fp32
// conversions run on a pool of host threads straight into / out of pinned
// staging, in chunks: each chunk's upload (or download) is queued on the
// library stream as soon as it is converted (or waited for just before it is
// widened), so conversion overlaps the PCIe copies and the GEMM.  Small calls
// (the C1 shapes) convert each operand in one pass split over the calling
// thread and the pool's spinning workers, copy A and B in with one kernel and
// have the GEMM store the product straight into pinned memory.
#include "lhip_internal.h"
#include "lhip_pool.h"

namespace lhip {
namespace {

// ---------------------------------------------------------------- conversions
// The same loops compiled twice: for AVX2 hosts (4 doubles per conversion
// instruction) and for the x86-64 baseline; the AVX2 form is chosen at run time.
__attribute__((target("avx2"))) void f64_to_f32_avx2(const double* __restrict__ s, float* __restrict__ d,
                                                     long long n)
{
    for (long long i = 0; i < n; ++i) d[i] = static_cast<float>(s[i]);
}
void f64_to_f32_base(const double* __restrict__ s, float* __restrict__ d, long long n)
{
    for (long long i = 0; i < n; ++i) d[i] = static_cast<float>(s[i]);
}
__attribute__((target("avx2"))) void f32_to_f64_avx2(const float* __restrict__ s, double* __restrict__ d,
                                                     long long n, int acc)
{
    if (acc) for (long long i = 0; i < n; ++i) d[i] += static_cast<double>(s[i]);
    else for (long long i = 0; i < n; ++i) d[i] = static_cast<double>(s[i]);
}
void f32_to_f64_base(const float* __restrict__ s, double* __restrict__ d, long long n, int acc)
{
    if (acc) for (long long i = 0; i < n; ++i) d[i] += static_cast<double>(s[i]);
    else for (long long i = 0; i < n; ++i) d[i] = static_cast<double>(s[i]);
}

bool host_avx2()
{
    static const bool v = __builtin_cpu_supports("avx2");
    return v;
}

void narrow(const double* s, float* d, long long n)
{
    if (host_avx2()) f64_to_f32_avx2(s, d, n);
    else f64_to_f32_base(s, d, n);
}

void widen(const float* s, double* d, long long n, int acc)
{
    if (host_avx2()) f32_to_f64_avx2(s, d, n, acc);
    else f32_to_f64_base(s, d, n, acc);
}

HostPool g_pool;   // three spinning workers

// Copy n floats from pinned host memory into device memory with the GPU's own
// loads (one float4 per thread): for a small call this costs a kernel launch
// instead of a DMA transfer's ~11 us of fixed latency.
__global__ void __launch_bounds__(256) stage_in_kernel(const float* __restrict__ src, float* __restrict__ dst,
                                                       long long n)
{
    const long long i = (static_cast<long long>(blockIdx.x) * 256 + threadIdx.x) * 4;
    if (i + 3 < n) {
        *reinterpret_cast<float4*>(dst + i) = *reinterpret_cast<const float4*>(src + i);
    } else {
        for (long long j = i; j < n; ++j) dst[j] = src[j];
    }
}

// Below this many elements in all three operands together a call is small:
// one conversion pass per operand (split over the calling thread and the
// spinning workers), one upload kernel, the product stored into pinned memory.
constexpr long long kPoolMin = 1LL << 20;
// Elements per pipelined chunk (16 MiB of fp32).
constexpr long long kChunk = 1LL << 22;

// Convert [0, n) with the pool: slices of at least 64 Ki elements over every
// thread, or (small calls) of at least 8 Ki over the calling thread and the
// spinning workers.
int conv_parts(long long n, bool small)
{
    const long long unit = small ? 8192 : 65536;
    const int cap = small ? g_pool.spinners() + 1 : g_pool.threads();
    return static_cast<int>(std::max<long long>(1, std::min<long long>(cap, (n + unit - 1) / unit)));
}

void par_narrow(const double* s, float* d, long long n, bool small = false)
{
    const int parts = conv_parts(n, small);
    const long long per = (n + parts - 1) / parts;
    g_pool.run(parts, [&](int p) {
        const long long b = p * per, e = std::min(n, b + per);
        if (b < e) narrow(s + b, d + b, e - b);
    });
}

// A and B of a small call in one run: the parts split the two arrays as one
// index range (A's elements, then B's).
void par_narrow2(const double* a, float* ha, long long na, const double* b, float* hb, long long nb)
{
    const long long n = na + nb;
    const int parts = conv_parts(n, true);
    const long long per = (n + parts - 1) / parts;
    g_pool.run(parts, [&](int p) {
        const long long lo = p * per, hi = std::min(n, lo + per);
        if (lo < std::min(hi, na)) narrow(a + lo, ha + lo, std::min(hi, na) - lo);
        if (std::max(lo, na) < hi) narrow(b + (std::max(lo, na) - na), hb + (std::max(lo, na) - na), hi - std::max(lo, na));
    });
}

void par_widen(const float* s, double* d, long long n, int acc, bool small = false)
{
    const int parts = conv_parts(n, small);
    const long long per = (n + parts - 1) / parts;
    g_pool.run(parts, [&](int p) {
        const long long b = p * per, e = std::min(n, b + per);
        if (b < e) widen(s + b, d + b, e - b, acc);
    });
}

}  // namespace

void host_pool_shutdown() { g_pool.stop(); }

}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

LHIP_API int lhip_matmul_host(int op, const double* a, const double* b, double* c,
                              int m, int k, int n, int acc)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (op < 0 || op > 2) return fail(LHIP_E_ARG, "lhip_matmul_host: op %d not in {0,1,2}", op);
    if (m < 0 || k < 0 || n < 0) return fail(LHIP_E_SHAPE, "lhip_matmul_host: negative size");
    // Result shape and operand sizes per op.
    const long long rows = (op == 2) ? k : m;
    const long long inner = (op == 2) ? m : k;
    const long long na = static_cast<long long>(m) * k;
    const long long nb = (op == 0) ? static_cast<long long>(k) * n
                                   : (op == 1 ? static_cast<long long>(n) * k : static_cast<long long>(m) * n);
    const long long nc = rows * n;
    if (nc == 0) return LHIP_OK;
    if (!c) return fail(LHIP_E_NULL, "lhip_matmul_host: c is NULL");
    if (inner == 0) {
        if (!acc) for (long long i = 0; i < nc; ++i) c[i] = 0.0;
        return LHIP_OK;
    }
    if (!a || !b) return fail(LHIP_E_NULL, "lhip_matmul_host: a or b is NULL");
    auto& s = st();
    // Staging: [A | B | C] in fp32, each section padded to 64 floats so every
    // operand starts 256-byte aligned.
    auto pad = [](long long x) { return (x + 63) / 64 * 64; };
    const size_t need = static_cast<size_t>(pad(na) + pad(nb) + pad(nc));
    if (need > s.d_stage_floats) {
        if (s.d_stage) {
            LHIP_CHECK_HIP(hipStreamSynchronize(s.stream), "lhip_matmul_host: sync");
            LHIP_CHECK_HIP(hipFree(s.d_stage), "lhip_matmul_host: free device staging");
            s.d_stage = nullptr;
            s.d_stage_floats = 0;
        }
        LHIP_CHECK_HIP(hipMalloc(&s.d_stage, need * sizeof(float)), "lhip_matmul_host: device staging");
        s.d_stage_floats = need;
    }
    if (need > s.h_stage_floats) {
        if (s.h_stage) {
            LHIP_CHECK_HIP(hipStreamSynchronize(s.stream), "lhip_matmul_host: sync");
            LHIP_CHECK_HIP(hipHostFree(s.h_stage), "lhip_matmul_host: free pinned staging");
            s.h_stage = nullptr;
            s.h_stage_floats = 0;
        }
        LHIP_CHECK_HIP(hipHostMalloc(&s.h_stage, need * sizeof(float), hipHostMallocDefault),
                       "lhip_matmul_host: pinned staging");
        s.h_stage_floats = need;
    }
    float* ha = s.h_stage;
    float* hb = ha + pad(na);
    float* hc = hb + pad(nb);
    float* da = s.d_stage;
    float* db = da + pad(na);
    float* dc = db + pad(nb);
    const bool pooled = na + nb + nc >= lhip::kPoolMin;
    lhip::g_pool.start();

    // upload: convert a chunk, queue its copy, convert the next meanwhile
    auto upload = [&](const double* src, float* h, float* d, long long cnt) -> int {
        for (long long off = 0; off < cnt; off += lhip::kChunk) {
            const long long len = std::min(lhip::kChunk, cnt - off);
            lhip::par_narrow(src + off, h + off, len);
            LHIP_CHECK_HIP(hipMemcpyAsync(d + off, h + off, len * sizeof(float), hipMemcpyHostToDevice, s.stream),
                           "lhip_matmul_host: upload");
        }
        return LHIP_OK;
    };
    if (!pooled) {
        lhip::par_narrow2(a, ha, na, b, hb, nb);
    } else {
        if (int rc = upload(a, ha, da, na)) return rc;
        if (int rc = upload(b, hb, db, nb)) return rc;
    }
    if (!pooled) {   // A and B (adjacent in the staging) in one kernel-side copy
        const long long cnt = pad(na) + nb;
        lhip::klaunch(lhip::stage_in_kernel, dim3(static_cast<unsigned>((cnt + 1023) / 1024)), dim3(256), 0, s.stream,
                      ha, da, cnt);
        if (int rc = lhip::check_launch("lhip_matmul_host: upload")) return rc;
    }
    // A small call's product is stored by the GEMM straight into the pinned
    // staging (the GPU writes host memory over PCIe): no download copy, whose
    // fixed cost (~11 us) is most of such a call.
    float* cout = pooled ? dc : hc;
    int rc;
    if (op == 0)       // c(m x n) = a(m x k) b(k x n)
        rc = lhip::sgemm_launch(0, 0, m, n, k, 1.f, da, k, db, n, 0.f, cout, n, 1, 0, 0, 0, s.stream);
    else if (op == 1)  // c(m x n) = a(m x k) b(n x k)^T
        rc = lhip::sgemm_launch(0, 1, m, n, k, 1.f, da, k, db, k, 0.f, cout, n, 1, 0, 0, 0, s.stream);
    else               // c(k x n) = a(m x k)^T b(m x n)
        rc = lhip::sgemm_launch(1, 0, k, n, m, 1.f, da, k, db, n, 0.f, cout, n, 1, 0, 0, 0, s.stream);
    if (rc != LHIP_OK) return rc;
    if (!pooled) {
        LHIP_CHECK_HIP(hipStreamSynchronize(s.stream), "lhip_matmul_host: sync");
        lhip::par_widen(hc, c, nc, acc, true);
        return LHIP_OK;
    }
    // download: queue every chunk's copy with an event behind it, then widen
    // each chunk as soon as its event has fired
    const int nch = static_cast<int>((nc + lhip::kChunk - 1) / lhip::kChunk);
    std::vector<hipEvent_t> ev(nch, nullptr);
    int err = LHIP_OK;
    for (int i = 0; i < nch && err == LHIP_OK; ++i) {
        const long long off = i * lhip::kChunk, len = std::min(lhip::kChunk, nc - off);
        hipError_t e = hipEventCreateWithFlags(&ev[i], hipEventDisableTiming);
        if (e == hipSuccess)
            e = hipMemcpyAsync(hc + off, dc + off, len * sizeof(float), hipMemcpyDeviceToHost, s.stream);
        if (e == hipSuccess) e = hipEventRecord(ev[i], s.stream);
        if (e != hipSuccess) err = lhip::hip_fail(e, "lhip_matmul_host: download");
    }
    for (int i = 0; i < nch && err == LHIP_OK; ++i) {
        const long long off = i * lhip::kChunk, len = std::min(lhip::kChunk, nc - off);
        const hipError_t e = hipEventSynchronize(ev[i]);
        if (e != hipSuccess) {
            err = lhip::hip_fail(e, "lhip_matmul_host: download wait");
            break;
        }
        lhip::par_widen(hc + off, c + off, len, acc);
    }
    if (err != LHIP_OK) (void)hipStreamSynchronize(s.stream);   // no copy may still target the staging
    for (hipEvent_t e : ev)
        if (e) (void)hipEventDestroy(e);
    return err;
}

LHIP_API int lhip_set_host_spin(int spin_us, int* previous)
{
    if (spin_us < 0 || spin_us > 100000)
        return fail(LHIP_E_ARG, "lhip_set_host_spin: spin_us %d outside [0, 100000]", spin_us);
    if (previous) *previous = lhip::g_pool.spin_us();
    lhip::g_pool.set_spin_us(spin_us);
    return LHIP_OK;
}

}  // extern "C"
