--  luatl_adapter.lua -- lanternl's `luatl_adapter` backend, served by liblanternl_hip.so
--  (MI355X / gfx950) through the LuaJIT FFI.
--
--  Drop-in for ai/gpu/luatl_adapter.lua: ai/core/matrix.lua probes it by name
--  (BACKEND_NAMES, matrix.lua:25), requires `available == true` and a
--  `matmul` function (matrix.lua:28-48), and calls
--  matmul(a_flat, m, k, b_flat, n) -> new flat table (matrix.lua:178-202).
--  matmul_nt / matmul_tn serve the transposed products with the same calling
--  convention (a dispatch that matrix.lua gains with the patch shown in
--  INTEGRATION.md).  The resident-handle API below keeps the names of
--  luatl_adapter.lua:46-246 for the calls this backend implements.
--
--  Errors: every C status is checked; a failure raises
--  "lanternl_hip[<what>]: <message> (<STATUS>)" (the reference's ck(),
--  ai/gpu/luaTL.lua:240-246), which the registry counts (matrix.lua:169-176).

local M = { name = "lanternl_hip", priority = 100, available = false, reason = "not loaded" }

local okffi, ffi = pcall(require, "ffi")
if not okffi then M.reason = "LuaJIT FFI unavailable" return M end

ffi.cdef[[
int lhip_init(int device);
int lhip_shutdown(void);
int lhip_is_ready(void);
const char* lhip_last_error(void);
void lhip_clear_error(void);
int lhip_malloc(void** dptr, size_t bytes);
int lhip_free(void* dptr);
int lhip_upload(void* dst_device, const void* src_host, size_t bytes);
int lhip_download(void* dst_host, const void* src_device, size_t bytes);
int lhip_zero(void* dptr, size_t bytes);
int lhip_sync(void);
int lhip_sgemm(int transa, int transb, int m, int n, int k, float alpha,
               const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc);
int lhip_matmul_host(int op, const double* a, const double* b, double* c,
                     int m, int k, int n, int acc);
int lhip_rmsnorm_fwd(const float* x, const float* w, float* y, float* inv, int rows, int cols, float eps);
int lhip_rmsnorm_bwd(const float* x, const float* w, const float* inv, const float* dy,
                     float* dx, float* dw, int rows, int cols, int accumulate);
int lhip_softmax_fwd(const float* x, float* y, int rows, int cols, float scale,
                     int causal, int offset, int group);
int lhip_softmax_bwd(const float* y, const float* dy, float* dx, int rows, int cols,
                     float scale, int causal, int offset, int group, int accumulate);
int lhip_swiglu_fwd(const float* gate, int ld_gate, const float* up, int ld_up,
                    float* out, int ld_out, int rows, int cols);
int lhip_swiglu_bwd(const float* gate, int ld_gate, const float* up, int ld_up,
                    const float* dout, int ld_dout, float* dgate, int ld_dgate,
                    float* dup, int ld_dup, int rows, int cols, int accumulate);
int lhip_rope(float* x, const int* pos_ids, int rows, int heads, int head_dim, int row_stride,
              int pos_offset, int pos_period, double base, int interleaved, int inverse);
int lhip_ce_fused(const float* logits, const int* targets, float* losses, float* dlogits,
                  int rows, int vocab, int ignore_index, float grad_scale);
int lhip_argmax_rows(const float* x, int* out, int rows, int cols);
int lhip_add(const float* a, const float* b, float* out, long long n);
int lhip_program_begin(void);
int lhip_program_end(void** program);
int lhip_program_replay(void* program, int times);
int lhip_program_free(void* program);
int lhip_silu(const float* x, float* out, long long n);
int lhip_mem_info(unsigned long long* free_bytes, unsigned long long* total_bytes);
typedef struct {
    unsigned long long bytes_in_use, peak_in_use, live_buffers, n_alloc, n_free,
                       workspace_bytes, staging_bytes;
} lhip_mem_stats_t;
int lhip_mem_stats(lhip_mem_stats_t* out);
typedef struct {
    char name[256];
    char arch[64];
    int device;
    int compute_units;
    int clock_khz;
    int wavefront_size;
    long long total_mem;
    long long lds_per_block;
    int l2_bytes;
    double peak_fp32_matrix_tflops;
    double peak_hbm_gbps;
} lhip_devinfo_t;
int lhip_device_info(lhip_devinfo_t* out);
]]

local STATUS = { [0] = "OK", [-1] = "NULL", [-2] = "SHAPE", [-3] = "DTYPE", [-4] = "DEVICE",
                 [-5] = "OOM", [-6] = "ARG", [-7] = "CAPACITY", [-8] = "UNSUPPORTED" }

-- library candidates: $LANTERNL_HIP_LIB, then next to this file, then the loader path
local function candidates()
    local list = {}
    local env = os.getenv("LANTERNL_HIP_LIB")
    if env and env ~= "" then list[#list + 1] = env end
    local src = debug.getinfo(1, "S").source
    if src:sub(1, 1) == "@" then
        local dir = src:sub(2):match("^(.*)[/\\]") or "."
        list[#list + 1] = dir .. "/../liblanternl_hip.so"
        list[#list + 1] = dir .. "/liblanternl_hip.so"
    end
    list[#list + 1] = "liblanternl_hip.so"
    list[#list + 1] = "lanternl_hip"
    return list
end

local C, load_err
for _, path in ipairs(candidates()) do
    local ok, lib = pcall(ffi.load, path)
    if ok then C = lib break end
    load_err = tostring(lib)
end
if not C then M.reason = "liblanternl_hip.so not found (" .. tostring(load_err) .. ")" return M end

local function ck(rc, what)
    if rc ~= 0 then
        local msg = ffi.string(C.lhip_last_error())
        error(("lanternl_hip[%s]: %s (%s)"):format(what, msg, STATUS[rc] or tostring(rc)), 2)
    end
    return rc
end

local okinit, initerr = pcall(function() ck(C.lhip_init(0), "init") end)
if not okinit then M.reason = tostring(initerr) return M end

M.available = true
M.reason = "ready"
M.C = C

local ok_tnew, tnew = pcall(require, "table.new")
if not ok_tnew then tnew = function() return {} end end

local f64_ct = ffi.typeof("double[?]")
local f32_ct = ffi.typeof("float[?]")
local i32_ct = ffi.typeof("int32_t[?]")

--  cached host staging (no per-call cdata churn, as luatl_adapter.lua:24-32)
local stage, stage_n = {}, {}
local function host_f64(slot, n)
    if not stage[slot] or stage_n[slot] < n then
        stage[slot] = f64_ct(n)
        stage_n[slot] = n
    end
    return stage[slot]
end

local function fill_f64(dst, src, n)
    for i = 1, n do dst[i - 1] = src[i] end
end

local function host_gemm(op, a, m, k, b, n, na, nb, nc, what)
    if #a < na then error(("lanternl_hip: %s: a has %d elements, expected %d"):format(what, #a, na), 3) end
    if #b < nb then error(("lanternl_hip: %s: b has %d elements, expected %d"):format(what, #b, nb), 3) end
    local A = host_f64("a", na)
    local B = host_f64("b", nb)
    local Cb = host_f64("c", nc)
    fill_f64(A, a, na)
    fill_f64(B, b, nb)
    ck(C.lhip_matmul_host(op, A, B, Cb, m, k, n, 0), what)
    local out = tnew(nc, 0)
    for i = 1, nc do out[i] = Cb[i - 1] end
    return out
end

--  LEGACY-COMPATIBLE ENTRY POINTS (matrix.lua's backend contract)

--  a(m x k) . b(k x n) -> new flat table of m*n numbers (luatl_adapter.lua:128-135)
function M.matmul(a, m, k, b, n)
    return host_gemm(0, a, m, k, b, n, m * k, k * n, m * n, "matmul")
end

--  a(m x k) . b(n x k)^T -> m*n numbers (matrix.matmul_nt, matrix.lua:597-625)
function M.matmul_nt(a, m, k, b, n)
    return host_gemm(1, a, m, k, b, n, m * k, n * k, m * n, "matmul_nt")
end

--  a(m x k)^T . b(m x n) -> k*n numbers (matrix.matmul_tn, matrix.lua:627-660)
function M.matmul_tn(a, m, k, b, n)
    return host_gemm(2, a, m, k, b, n, m * k, m * n, k * n, "matmul_tn")
end

--  RESIDENT HANDLES (luatl_adapter.lua:46-101): a device fp32 matrix with a
--  finaliser; flat Lua tables cross the boundary only on pin/upload/toflat.
local Handle = {}
Handle.__index = Handle
M.HandleClass = Handle

local function is_handle(x) return type(x) == "table" and getmetatable(x) == Handle end
M.is_handle = is_handle

local function dev_alloc(bytes)
    local pp = ffi.new("void*[1]")
    ck(C.lhip_malloc(pp, bytes), "alloc")
    return ffi.gc(pp[0], function(p) C.lhip_free(p) end)
end

local function new_handle(rows, cols)
    local h = setmetatable({ rows = rows, cols = cols }, Handle)
    h.ptr = dev_alloc(math.max(rows * cols, 1) * 4)
    return h
end

function M.alloc(rows, cols)
    local h = new_handle(rows, cols)
    ck(C.lhip_zero(h.ptr, math.max(rows * cols, 1) * 4), "zero")
    return h
end

function M.pin(flat, rows, cols)
    local h = new_handle(rows, cols)
    h:upload(flat)
    return h
end

function Handle:upload(flat)
    local n = self.rows * self.cols
    if #flat < n then error(("lanternl_hip.upload: %d elements < %dx%d"):format(#flat, self.rows, self.cols), 2) end
    local buf = f32_ct(n)
    for i = 1, n do buf[i - 1] = flat[i] end
    ck(C.lhip_upload(self.ptr, buf, n * 4), "upload")
    return self
end

function Handle:toflat()
    local n = self.rows * self.cols
    local buf = f32_ct(n)
    ck(C.lhip_download(buf, self.ptr, n * 4), "download")
    local out = tnew(n, 0)
    for i = 1, n do out[i] = buf[i - 1] end
    return out
end

function Handle:zero() ck(C.lhip_zero(self.ptr, self.rows * self.cols * 4), "zero") return self end
function Handle:free()
    if self.ptr and self.owned ~= false then C.lhip_free(ffi.gc(self.ptr, nil)) end
    self.ptr = nil
end
function Handle:shape() return self.rows, self.cols end

local function fp(h) return ffi.cast("float*", h.ptr) end

--  C = A . B (+ beta C); gemm_dx: dY . W^T; gemm_dw: X^T . dY (+= with beta = 1),
--  the three products of luatl_adapter.lua:163-165 / luaTL_train.lua:154-182.
function M.gemm(A, B, Cm, beta)
    Cm = Cm or M.alloc(A.rows, B.cols)
    ck(C.lhip_sgemm(0, 0, A.rows, B.cols, A.cols, 1.0, fp(A), A.cols, fp(B), B.cols, beta or 0.0,
                    fp(Cm), Cm.cols), "gemm")
    return Cm
end

function M.gemm_dx(dY, W, dX, beta)
    dX = dX or M.alloc(dY.rows, W.rows)
    ck(C.lhip_sgemm(0, 1, dY.rows, W.rows, dY.cols, 1.0, fp(dY), dY.cols, fp(W), W.cols, beta or 0.0,
                    fp(dX), dX.cols), "gemm_dx")
    return dX
end

function M.gemm_dw(X, dY, dW, beta)
    dW = dW or M.alloc(X.cols, dY.cols)
    ck(C.lhip_sgemm(1, 0, X.cols, dY.cols, X.rows, 1.0, fp(X), X.cols, fp(dY), dY.cols, beta or 1.0,
                    fp(dW), dW.cols), "gemm_dw")
    return dW
end

function M.rmsnorm(X, W, eps, Y, inv)
    Y = Y or M.alloc(X.rows, X.cols)
    inv = inv or M.alloc(X.rows, 1)
    ck(C.lhip_rmsnorm_fwd(fp(X), fp(W), fp(Y), fp(inv), X.rows, X.cols, eps or 1e-5), "rmsnorm")
    return Y, inv
end

function M.rmsnorm_bwd(X, W, inv, dY, dX, dW, accumulate)
    dX = dX or M.alloc(X.rows, X.cols)
    ck(C.lhip_rmsnorm_bwd(fp(X), fp(W), fp(inv), fp(dY), fp(dX), dW and fp(dW) or nil, X.rows, X.cols,
                          accumulate and 1 or 0), "rmsnorm_bwd")
    return dX, dW
end

function M.softmax(X, Y, scale)
    Y = Y or M.alloc(X.rows, X.cols)
    ck(C.lhip_softmax_fwd(fp(X), fp(Y), X.rows, X.cols, scale or 1.0, 0, 0, 0), "softmax")
    return Y
end

function M.softmax_causal(X, Y, scale, offset, group)
    Y = Y or M.alloc(X.rows, X.cols)
    ck(C.lhip_softmax_fwd(fp(X), fp(Y), X.rows, X.cols, scale or 1.0, 1, offset or 0, group or 0),
       "softmax_causal")
    return Y
end

function M.softmax_bwd(Y, dY, dX, scale, causal, offset, group)
    dX = dX or M.alloc(Y.rows, Y.cols)
    ck(C.lhip_softmax_bwd(fp(Y), fp(dY), fp(dX), Y.rows, Y.cols, scale or 1.0, causal and 1 or 0,
                          offset or 0, group or 0, 0), "softmax_bwd")
    return dX
end

function M.swiglu(G, U, H)
    H = H or M.alloc(G.rows, G.cols)
    ck(C.lhip_swiglu_fwd(fp(G), G.cols, fp(U), U.cols, fp(H), H.cols, G.rows, G.cols), "swiglu")
    return H
end

--  in place; interleaved pairs (the CPU path's) unless opts.half_split
function M.rope(X, heads, head_dim, opts)
    opts = opts or {}
    ck(C.lhip_rope(fp(X), nil, X.rows, heads, head_dim, X.cols, opts.pos_offset or 0, opts.period or 0,
                   opts.base or 10000.0, opts.half_split and 0 or 1, opts.inverse and 1 or 0), "rope")
    return X
end

--  per-row CE losses and dlogits (written over the logits when dlogits == nil)
function M.cross_entropy(logits, targets0, grad_scale)
    local n = logits.rows
    local tg = i32_ct(n)
    for i = 1, n do tg[i - 1] = targets0[i] end
    local dtg = dev_alloc(n * 4)
    ck(C.lhip_upload(dtg, tg, n * 4), "cross_entropy: targets")
    local losses = M.alloc(n, 1)
    ck(C.lhip_ce_fused(fp(logits), ffi.cast("int*", dtg), fp(losses), fp(logits), n, logits.cols, -1,
                       grad_scale or 1.0), "cross_entropy")
    local l = losses:toflat()
    local s = 0
    for i = 1, n do s = s + l[i] end
    return s / n
end

function M.add_inplace(A, B)
    ck(C.lhip_add(fp(A), fp(B), fp(A), A.rows * A.cols), "add_inplace")
    return A
end

function M.silu_inplace(h)
    ck(C.lhip_silu(fp(h), fp(h), h.rows * h.cols), "silu_inplace")
    return h
end

function M.sync() ck(C.lhip_sync(), "sync") end

--  Memory and device queries (luatl_adapter.lua:184-185,243-246).  There is
--  no caching pool: stats() reports the library's own accounting of the
--  buffers it allocated (lhip_mem_stats), under the reference's key names
--  where they mean the same thing.
local mstats = ffi.new("lhip_mem_stats_t")
function M.stats()
    ck(C.lhip_mem_stats(mstats), "stats")
    local s = mstats
    return {
        in_use = tonumber(s.bytes_in_use), peak = tonumber(s.peak_in_use),
        blocks = tonumber(s.live_buffers), allocs = tonumber(s.n_alloc), frees = tonumber(s.n_free),
        workspace = tonumber(s.workspace_bytes), staging = tonumber(s.staging_bytes),
        reserved = tonumber(s.bytes_in_use + s.workspace_bytes + s.staging_bytes),
    }
end

local devinfo = ffi.new("lhip_devinfo_t")
function M.hardware()
    ck(C.lhip_device_info(devinfo), "hardware")
    local d = devinfo
    return {
        name = ffi.string(d.name), arch = ffi.string(d.arch), device = d.device,
        sm_count = d.compute_units, compute_units = d.compute_units, clock_mhz = d.clock_khz / 1000,
        warp_size = d.wavefront_size, total_mem = tonumber(d.total_mem),
        smem_per_block = tonumber(d.lds_per_block), l2_bytes = d.l2_bytes,
        gflops_fp32_matrix = d.peak_fp32_matrix_tflops * 1000, hbm_gbps = d.peak_hbm_gbps,
    }
end

local u64a, u64b = ffi.new("unsigned long long[1]"), ffi.new("unsigned long long[1]")
function M.mem()
    ck(C.lhip_mem_info(u64a, u64b), "mem")
    return tonumber(u64a[0]), tonumber(u64b[0])
end

--  Resident-tensor toolkit (luatl_adapter.lua:188-241): allocation-free views
--  over device memory.  A view is { ptr, rows, cols, rs, cs, bs } in
--  elements; wrap() makes a non-owning Handle over a raw device pointer.
local function base_ptr(t)
    if is_handle(t) or (type(t) == "table" and t.ptr ~= nil) then return t.ptr end
    return t
end

--- Element-offset pointer into a handle's (or view's) float32 storage.
function M.offset(t, elems)
    return ffi.cast("char*", base_ptr(t)) + elems * 4
end

--- Explicit stride view: rs = row stride, cs = column stride, bs = batch stride (elements).
function M.view(ptr, rows, cols, rs, cs, bs)
    return { ptr = ptr, rows = rows, cols = cols, rs = rs, cs = cs, bs = bs or 0 }
end

--- Column slice [col0, col0 + w) of a handle, keeping the parent's leading dimension.
function M.cols(t, col0, w)
    return M.view(M.offset(t, col0), t.rows, w, t.cols, 1, 0)
end

--- Non-owning handle over a raw device pointer (free() leaves the memory alone).
function M.wrap(ptr, rows, cols)
    return setmetatable({ rows = rows, cols = cols, ptr = ffi.cast("void*", ptr), owned = false }, Handle)
end

--- int32 index buffer (4 bytes per entry, as float32).
function M.ids(n)
    local h = M.alloc(n, 1)
    h.is_ids = true
    return h
end

function M.upload_i32(t, cbuf, n)
    ck(C.lhip_upload(base_ptr(t), cbuf, n * 4), "upload_i32")
end

function M.download_i32(t, cbuf, n)
    ck(C.lhip_download(cbuf, base_ptr(t), n * 4), "download_i32")
end

function M.download_f32(ptr, cbuf, n)
    ck(C.lhip_download(cbuf, base_ptr(ptr), n * 4), "download_f32")
end

--- One float read back from device memory (the loss, the gradient norm).
local one = ffi.new("float[1]")
function M.scalar(t)
    ck(C.lhip_download(one, base_ptr(t), 4), "scalar")
    return one[0]
end

-- Program (luaTL.Program capture/replay, ai/gpu/luaTL_train.lua:327-627):
-- fn() issues adapter calls, which are recorded rather than run; the result
-- replays them as one graph launch.  Calls that synchronise or allocate fail
-- while recording, so run fn() once eagerly first.
local Program = {}
Program.__index = Program

function M.program(fn)
    ck(C.lhip_program_begin(), "program")
    local ok, err = pcall(fn)
    if not ok then
        C.lhip_program_end(nil)             -- discard the partial recording
        error(err, 2)
    end
    local h = ffi.new("void*[1]")
    ck(C.lhip_program_end(h), "program")
    return setmetatable({ h = ffi.gc(h[0], C.lhip_program_free) }, Program)
end

function Program:replay(times)
    ck(C.lhip_program_replay(self.h, times or 1), "program.replay")
    return self
end

function Program:free()
    if self.h ~= nil then
        C.lhip_program_free(ffi.gc(self.h, nil))
        self.h = nil
    end
end

function M.shutdown()
    C.lhip_shutdown()
    M.available = false
    M.reason = "shut down"
end

return M
