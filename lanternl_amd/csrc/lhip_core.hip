// lhip_core.hip -- lifecycle, errors, memory, stream and events of liblanternl_hip.so.
//
// Replaces the runtime half of the reference's luaTL core (cuda/luaTL_core.cu:
// error plumbing 122-166, luaTL_init 1678-1715, devinfo 1755-1763, copies
// 2031-2094 and 2149-2159).  The reference keeps a caching pool and an arena;
// here buffers are plain hipMalloc allocations owned by the caller (the LuaJIT
// side frees them from an ffi.gc finaliser), and all compute work is ordered
// on one library-owned stream.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>

#include "lhip_internal.h"

namespace lhip {

static State g_state;
static KTimer g_ktimer;
static thread_local char t_err[1024] = {0};

State& st() { return g_state; }
KTimer& ktimer() { return g_ktimer; }

int fail(int code, const char* fmt, ...)
{
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(t_err, sizeof(t_err), fmt, ap);
    va_end(ap);
    return code;
}

int hip_fail(hipError_t e, const char* what)
{
    const int code = (e == hipErrorOutOfMemory || e == hipErrorMemoryAllocation) ? LHIP_E_OOM : LHIP_E_DEVICE;
    return fail(code, "%s: %s (%s)", what, hipGetErrorString(e), hipGetErrorName(e));
}

int check_launch(const char* what)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, what);
    return LHIP_OK;
}

int workspace(size_t bytes, void** out)
{
    auto& s = g_state;
    if (bytes == 0) bytes = 256;
    if (bytes > s.work_bytes) {
        if (s.recording)
            return fail(LHIP_E_UNSUPPORTED,
                        "workspace: %zu bytes needed (%zu held) while a program is being recorded; run the same "
                        "calls once before recording them", bytes, s.work_bytes);
        if (s.work) {
            if (s.live_programs > 0) {
                // a live program may hold this pointer: keep it until the last
                // program is freed (lhip_program_free) or shutdown
                s.retired.push_back(s.work);
                s.retired_bytes += s.work_bytes;
            } else {
                LHIP_CHECK_HIP(hipStreamSynchronize(s.stream), "workspace: stream sync");
                LHIP_CHECK_HIP(hipFree(s.work), "workspace: hipFree");
            }
            s.work = nullptr;
            s.work_bytes = 0;
        }
        const size_t grow = (bytes + (1u << 20) - 1) & ~static_cast<size_t>((1u << 20) - 1);
        hipError_t e = hipMalloc(&s.work, grow);
        if (e != hipSuccess) {
            s.work = nullptr;
            return fail(LHIP_E_OOM, "workspace: %zu bytes: %s", grow, hipGetErrorString(e));
        }
        s.work_bytes = grow;
    }
    *out = s.work;
    return LHIP_OK;
}

}  // namespace lhip

using lhip::fail;
using lhip::st;

extern "C" {

LHIP_API const char* lhip_version(void) { return "lanternl_hip 0.1.0 (gfx950)"; }

LHIP_API const char* lhip_last_error(void) { return lhip::t_err; }

LHIP_API void lhip_clear_error(void) { lhip::t_err[0] = 0; }

LHIP_API int lhip_is_ready(void) { return st().ready ? 1 : 0; }

LHIP_API int lhip_init(int device)
{
    auto& s = st();
    if (s.ready) {
        if (s.device == device) return LHIP_OK;
        return fail(LHIP_E_ARG, "lhip_init: already initialised on device %d (asked for %d); call lhip_shutdown first",
                    s.device, device);
    }
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0)
        return fail(LHIP_E_DEVICE, "lhip_init: no HIP device visible (%s)",
                    e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
    if (device < 0 || device >= count)
        return fail(LHIP_E_ARG, "lhip_init: device %d out of range [0, %d)", device, count);
    LHIP_CHECK_HIP(hipSetDevice(device), "lhip_init: hipSetDevice");
    hipDeviceProp_t p;
    LHIP_CHECK_HIP(hipGetDeviceProperties(&p, device), "lhip_init: hipGetDeviceProperties");
    if (std::strncmp(p.gcnArchName, "gfx950", 6) != 0)
        return fail(LHIP_E_UNSUPPORTED, "lhip_init: device %d is %s; this library is built for gfx950 (MI355X) only",
                    device, p.gcnArchName);
    // Default-priority, non-blocking stream: independent of the null stream.
    {
        const int rc = lhip::noalloc_scratch_init(device);
        if (rc != LHIP_OK) return rc;
    }
    LHIP_CHECK_HIP(hipStreamCreateWithFlags(&s.stream, hipStreamNonBlocking), "lhip_init: hipStreamCreate");
    {
        hipError_t eo = hipMalloc(reinterpret_cast<void**>(&s.ones), lhip::kOnesMax * sizeof(float));
        if (eo != hipSuccess) {
            s.ones = nullptr;
            (void)hipStreamDestroy(s.stream);
            s.stream = nullptr;
            return lhip::hip_fail(eo, "lhip_init: ones vector");
        }
        int rc = lhip::fill(s.ones, lhip::kOnesMax, 1.0f, s.stream);
        if (rc == LHIP_OK && hipStreamSynchronize(s.stream) != hipSuccess)
            rc = fail(LHIP_E_DEVICE, "lhip_init: filling the ones vector failed");
        if (rc != LHIP_OK) {
            (void)hipFree(s.ones);
            s.ones = nullptr;
            (void)hipStreamDestroy(s.stream);
            s.stream = nullptr;
            return rc;
        }
    }
    s.device = device;
    s.cu_count = p.multiProcessorCount;
    s.clock_khz = p.clockRate;
    s.lds_per_block = p.sharedMemPerBlock;
    s.total_mem = p.totalGlobalMem;
    s.l2_bytes = p.l2CacheSize;
    std::snprintf(s.name, sizeof(s.name), "%s", p.name);
    std::snprintf(s.arch, sizeof(s.arch), "%s", p.gcnArchName);
    s.ready = true;
    return LHIP_OK;
}

LHIP_API int lhip_shutdown(void)
{
    auto& s = st();
    if (!s.ready) return LHIP_OK;
    if (s.recording) {   // abandon the recording: its graph is discarded
        hipGraph_t g = nullptr;
        if (hipStreamEndCapture(s.stream, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
        (void)hipGetLastError();
        s.recording = false;
    }
    (void)hipStreamSynchronize(s.stream);
    lhip::host_pool_shutdown();
    if (s.d_stage) (void)hipFree(s.d_stage);
    if (s.h_stage) (void)hipHostFree(s.h_stage);
    if (s.work) (void)hipFree(s.work);
    for (void* p : s.retired) (void)hipFree(p);
    if (s.ones) (void)hipFree(s.ones);
    for (hipEvent_t e : lhip::ktimer().ev) (void)hipEventDestroy(e);
    lhip::ktimer() = lhip::KTimer();
    (void)hipStreamDestroy(s.stream);
    s = lhip::State();
    return LHIP_OK;
}

LHIP_API int lhip_device_info(lhip_devinfo_t* out)
{
    LHIP_REQUIRE_READY();
    if (!out) return fail(LHIP_E_NULL, "lhip_device_info: out is NULL");
    auto& s = st();
    std::memset(out, 0, sizeof(*out));
    std::snprintf(out->name, sizeof(out->name), "%s", s.name);
    std::snprintf(out->arch, sizeof(out->arch), "%s", s.arch);
    out->device = s.device;
    out->compute_units = s.cu_count;
    out->clock_khz = s.clock_khz;
    out->wavefront_size = 64;
    out->total_mem = static_cast<long long>(s.total_mem);
    out->lds_per_block = static_cast<long long>(s.lds_per_block);
    out->l2_bytes = s.l2_bytes;
    // CDNA4 fp32 MFMA: 256 flop per clock per CU (4 SIMDs x 64).
    out->peak_fp32_matrix_tflops = s.cu_count * 256.0 * (s.clock_khz * 1e3) / 1e12;
    out->peak_hbm_gbps = 8000.0;
    return LHIP_OK;
}

LHIP_API int lhip_malloc(void** dptr, size_t bytes)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!dptr) return fail(LHIP_E_NULL, "lhip_malloc: dptr is NULL");
    *dptr = nullptr;
    if (bytes == 0) return fail(LHIP_E_ARG, "lhip_malloc: zero-byte allocation");
    hipError_t e = hipMalloc(dptr, bytes);
    if (e != hipSuccess) {
        *dptr = nullptr;
        (void)hipGetLastError();
        return fail(LHIP_E_OOM, "lhip_malloc: %zu bytes: %s", bytes, hipGetErrorString(e));
    }
    auto& s = st();
    s.live[*dptr] = bytes;
    s.bytes_in_use += bytes;
    if (s.bytes_in_use > s.peak_in_use) s.peak_in_use = s.bytes_in_use;
    ++s.n_alloc;
    return LHIP_OK;
}

LHIP_API int lhip_free(void* dptr)
{
    if (!dptr) return LHIP_OK;
    if (!st().ready) return LHIP_OK;  // after shutdown a late finaliser is a no-op
    LHIP_REFUSE_RECORDING();
    // Work already enqueued may still read the buffer.
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_free: stream sync");
    LHIP_CHECK_HIP(hipFree(dptr), "lhip_free: hipFree");
    auto& s = st();
    const auto it = s.live.find(dptr);
    if (it != s.live.end()) {
        s.bytes_in_use -= it->second;
        ++s.n_free;
        s.live.erase(it);
    }
    return LHIP_OK;
}

LHIP_API int lhip_mem_info(unsigned long long* free_bytes, unsigned long long* total_bytes)
{
    LHIP_REQUIRE_READY();
    size_t f = 0, t = 0;
    LHIP_CHECK_HIP(hipMemGetInfo(&f, &t), "lhip_mem_info: hipMemGetInfo");
    if (free_bytes) *free_bytes = f;
    if (total_bytes) *total_bytes = t;
    return LHIP_OK;
}

LHIP_API int lhip_mem_stats(lhip_mem_stats_t* out)
{
    if (!out) return fail(LHIP_E_NULL, "lhip_mem_stats: out is NULL");
    const auto& s = st();
    std::memset(out, 0, sizeof(*out));
    out->bytes_in_use = s.bytes_in_use;
    out->peak_in_use = s.peak_in_use;
    out->live_buffers = s.live.size();
    out->n_alloc = s.n_alloc;
    out->n_free = s.n_free;
    out->workspace_bytes = s.work_bytes + s.retired_bytes;
    out->staging_bytes = s.d_stage_floats * sizeof(float);
    return LHIP_OK;
}

LHIP_API int lhip_upload(void* dst, const void* src, size_t bytes)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (bytes == 0) return LHIP_OK;
    if (!dst || !src) return fail(LHIP_E_NULL, "lhip_upload: NULL pointer");
    LHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, st().stream), "lhip_upload");
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_upload: sync");
    return LHIP_OK;
}

LHIP_API int lhip_download(void* dst, const void* src, size_t bytes)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (bytes == 0) return LHIP_OK;
    if (!dst || !src) return fail(LHIP_E_NULL, "lhip_download: NULL pointer");
    LHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, st().stream), "lhip_download");
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_download: sync");
    return LHIP_OK;
}

LHIP_API int lhip_copy(void* dst, const void* src, size_t bytes)
{
    LHIP_REQUIRE_READY();
    if (bytes == 0) return LHIP_OK;
    if (!dst || !src) return fail(LHIP_E_NULL, "lhip_copy: NULL pointer");
    LHIP_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, st().stream), "lhip_copy");
    return LHIP_OK;
}

LHIP_API int lhip_zero(void* dptr, size_t bytes)
{
    LHIP_REQUIRE_READY();
    if (bytes == 0) return LHIP_OK;
    if (!dptr) return fail(LHIP_E_NULL, "lhip_zero: NULL pointer");
    // a fill kernel rather than hipMemsetAsync, so the call is safe to record
    // into a captured graph
    return lhip::zero_bytes(dptr, bytes, st().stream);
}

LHIP_API int lhip_sync(void)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_sync");
    return LHIP_OK;
}

LHIP_API void* lhip_stream(void) { return st().ready ? static_cast<void*>(st().stream) : nullptr; }

LHIP_API int lhip_event_create(void** ev)
{
    LHIP_REQUIRE_READY();
    if (!ev) return fail(LHIP_E_NULL, "lhip_event_create: ev is NULL");
    hipEvent_t e;
    LHIP_CHECK_HIP(hipEventCreate(&e), "lhip_event_create");
    *ev = static_cast<void*>(e);
    return LHIP_OK;
}

LHIP_API int lhip_event_destroy(void* ev)
{
    if (!ev || !st().ready) return LHIP_OK;
    LHIP_CHECK_HIP(hipEventDestroy(static_cast<hipEvent_t>(ev)), "lhip_event_destroy");
    return LHIP_OK;
}

LHIP_API int lhip_event_record(void* ev)
{
    LHIP_REQUIRE_READY();
    if (!ev) return fail(LHIP_E_NULL, "lhip_event_record: ev is NULL");
    LHIP_CHECK_HIP(hipEventRecord(static_cast<hipEvent_t>(ev), st().stream), "lhip_event_record");
    return LHIP_OK;
}

LHIP_API int lhip_event_elapsed_ms(void* start, void* stop, float* ms)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!start || !stop || !ms) return fail(LHIP_E_NULL, "lhip_event_elapsed_ms: NULL argument");
    LHIP_CHECK_HIP(hipEventSynchronize(static_cast<hipEvent_t>(stop)), "lhip_event_elapsed_ms: sync");
    LHIP_CHECK_HIP(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(stop)),
                   "lhip_event_elapsed_ms");
    return LHIP_OK;
}


// ---- programs: recorded sequences of compute calls, replayed as a hipGraph ----
// The counterpart of luaTL's command-buffer Program with capture/replay
// (ai/gpu/luaTL_train.lua:327-627, luaTL_prog_capture / luaTL_prog_replay):
// instead of an op list that a C interpreter walks, the calls themselves are
// captured from the library stream into a graph, so every entry point that
// only enqueues work can be recorded.

LHIP_API int lhip_program_begin(void)
{
    LHIP_REQUIRE_READY();
    auto& s = st();
    if (s.recording) return fail(LHIP_E_ARG, "lhip_program_begin: a program is already being recorded");
    if (lhip::ktimer().on) return fail(LHIP_E_UNSUPPORTED, "lhip_program_begin: the kernel timer is on");
    LHIP_CHECK_HIP(hipStreamBeginCapture(s.stream, hipStreamCaptureModeRelaxed), "lhip_program_begin");
    s.recording = true;
    return LHIP_OK;
}

LHIP_API int lhip_program_end(void** program)
{
    LHIP_REQUIRE_READY();
    auto& s = st();
    if (!s.recording) return fail(LHIP_E_ARG, "lhip_program_end: no program is being recorded");
    if (program) *program = nullptr;
    hipGraph_t g = nullptr;
    hipError_t e = hipStreamEndCapture(s.stream, &g);
    s.recording = false;
    if (e != hipSuccess) {
        if (g) (void)hipGraphDestroy(g);
        return lhip::hip_fail(e, "lhip_program_end: end capture");
    }
    if (!program) {   // recording discarded
        (void)hipGraphDestroy(g);
        return LHIP_OK;
    }
    hipGraphExec_t x = nullptr;
    e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
    (void)hipGraphDestroy(g);
    if (e != hipSuccess) return lhip::hip_fail(e, "lhip_program_end: instantiate");
    *program = static_cast<void*>(x);
    ++s.live_programs;
    return LHIP_OK;
}

LHIP_API int lhip_program_replay(void* program, int times)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    if (!program) return fail(LHIP_E_NULL, "lhip_program_replay: program is NULL");
    if (times < 1) return fail(LHIP_E_ARG, "lhip_program_replay: times %d must be >= 1", times);
    for (int i = 0; i < times; ++i)
        LHIP_CHECK_HIP(hipGraphLaunch(static_cast<hipGraphExec_t>(program), st().stream), "lhip_program_replay");
    return LHIP_OK;
}

LHIP_API int lhip_program_free(void* program)
{
    if (!program || !st().ready) return LHIP_OK;
    LHIP_REFUSE_RECORDING();
    // a replay still in flight uses the executable graph
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_program_free: stream sync");
    LHIP_CHECK_HIP(hipGraphExecDestroy(static_cast<hipGraphExec_t>(program)), "lhip_program_free");
    auto& s = st();
    if (s.live_programs > 0) --s.live_programs;
    if (s.live_programs == 0 && !s.retired.empty()) {
        // no program can reach the retired workspaces any more (the stream
        // was synchronised above)
        for (void* p : s.retired) LHIP_CHECK_HIP(hipFree(p), "lhip_program_free: retired workspace");
        s.retired.clear();
        s.retired_bytes = 0;
    }
    return LHIP_OK;
}

LHIP_API int lhip_is_recording(void) { return st().recording ? 1 : 0; }

// ---- kernel timer ----
// Each kernel launched while the timer is on gets its dispatch's start and
// end timestamps recorded (hipExtLaunchKernel with an event pair), which is
// what a kernel trace reports as its duration; launch gaps are not included.

LHIP_API int lhip_ktimer_start(int capacity)
{
    LHIP_REQUIRE_READY();
    LHIP_REFUSE_RECORDING();
    auto& kt = lhip::ktimer();
    if (kt.on) return fail(LHIP_E_ARG, "lhip_ktimer_start: the timer is already on");
    if (capacity < 1 || capacity > (1 << 16))
        return fail(LHIP_E_ARG, "lhip_ktimer_start: capacity %d outside [1, 65536]", capacity);
    while (kt.ev.size() < static_cast<size_t>(2 * capacity)) {
        hipEvent_t e = nullptr;
        LHIP_CHECK_HIP(hipEventCreate(&e), "lhip_ktimer_start: hipEventCreate");
        kt.ev.push_back(e);
    }
    kt.cap = capacity;
    kt.used = 0;
    kt.total = 0;
    kt.on = true;
    return LHIP_OK;
}

LHIP_API int lhip_ktimer_stop(float* ms, int capacity, int* count)
{
    LHIP_REQUIRE_READY();
    auto& kt = lhip::ktimer();
    if (!kt.on) return fail(LHIP_E_ARG, "lhip_ktimer_stop: the timer is not on");
    kt.on = false;
    if (count) *count = kt.total;
    LHIP_CHECK_HIP(hipStreamSynchronize(st().stream), "lhip_ktimer_stop: stream sync");
    const int filled = (ms && capacity > 0) ? std::min(kt.used, capacity) : 0;
    for (int i = 0; i < filled; ++i)
        LHIP_CHECK_HIP(hipEventElapsedTime(&ms[i], kt.ev[2 * i], kt.ev[2 * i + 1]), "lhip_ktimer_stop: elapsed");
    if (ms && kt.total > filled)
        return fail(LHIP_E_CAPACITY,
                    "lhip_ktimer_stop: %d kernels were launched but only %d timed (timer capacity %d, "
                    "caller capacity %d; launches into a graph capture are never timed)",
                    kt.total, filled, kt.cap, capacity);
    return LHIP_OK;
}

}  // extern "C"
