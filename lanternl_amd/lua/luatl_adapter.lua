--  luatl_adapter.lua -- lanternl's `luatl_adapter` backend, served by liblanternl_hip.so
--  (MI355X / gfx950) through the LuaJIT FFI.
--
--  Drop-in for ai/gpu/luatl_adapter.lua, call for call: the same names, argument
--  lists and return conventions.
--    * Module contract (ai/core/matrix.lua:28-48,178-202): `available`,
--      `reason`/`error`, and matmul(a, m, k, b, n), where a and b are flat
--      tables or resident handles; two handles give a new handle, otherwise a
--      NEW flat table (luatl_adapter.lua:102-135).  matmul_nt / matmul_tn serve
--      the transposed products with the same convention, and
--      matmul_into(op, a, m, k, b, n, rd, acc) serves every product that
--      writes into a caller's table (`out`, with or without `acc`): the
--      dispatch that matrix.lua gains with lanternl_amd/lua/matrix_patch.lua.
--    * Legacy flat calls rmsnorm(x, rows, cols, w, eps), softmax(x, rows, cols),
--      softmax_causal(x, rows, cols, scale, group) (:137-159).
--    * Resident calls gemm(hA, hB, hC, opts), gemm_dx, gemm_dw, add_inplace,
--      silu_inplace, gelu_inplace, scale_inplace, rope(h, o),
--      swiglu(ha, hb, ho, o), rmsnorm_bwd(hx, hg, hdy, hdx, hdg, eps),
--      softmax_bwd(hy, hdy, hdx, o), program(cap, timing), sync, stats,
--      hardware, shutdown (:161-187), and the resident-tensor toolkit
--      offset, view, cols, wrap, ids, upload_i32, download_i32, download_f32,
--      scalar, mem (:188-246).
--    * program(cap, timing) returns a Program with luaTL.Program's op list
--      (ai/gpu/luaTL_train.lua:332-632): ops queue library calls; run() issues
--      them on the library stream, capture() records them once into a hipGraph,
--      replay() launches it.
--  Handles and tensors carry .t.data / .data (the device address), rows and
--  cols as the reference's do.  One reference field has no counterpart:
--  M.luaTL, the reference's own low-level module, stays nil, so callers that
--  reach past the adapter into it (ai/gpu/gpu_transformer.lua:58-60,
--  ai/optim/lmtrain_gpu.lua, ai/benchmarks/bench_gpu_transformer.lua:41-44)
--  do not run on this backend.
--
--  Marshaling: flat tables reach the device through grow-only host lanes
--  (cdata arrays, one per element type and operand) and grow-only device
--  lanes (one buffer per operand), both sized to the next power of two that
--  fits; handles are used in place.
--
--  Errors: every C status is checked; a failure raises
--  "lanternl_hip[<what>]: <message> (<STATUS>)" (the reference's ck(),
--  ai/gpu/luaTL.lua:240-246), which the registry counts (matrix.lua:169-176).

local M = { name = "luatl", priority = 100, available = false, reason = "not loaded" }

local okffi, ffi = pcall(require, "ffi")
if not okffi then M.reason = "LuaJIT FFI unavailable" M.error = M.reason return M end

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
int lhip_copy(void* dst_device, const void* src_device, size_t bytes);
int lhip_zero(void* dptr, size_t bytes);
int lhip_sync(void);
int lhip_event_create(void** ev);
int lhip_event_destroy(void* ev);
int lhip_event_record(void* ev);
int lhip_event_elapsed_ms(void* start, void* stop, float* ms);
int lhip_sgemm(int transa, int transb, int m, int n, int k, float alpha,
               const float* A, int lda, const float* B, int ldb, float beta,
               float* C, int ldc);
int lhip_matmul_host(int op, const double* a, const double* b, double* c,
                     int m, int k, int n, int acc);
int lhip_set_host_spin(int spin_us, int* previous);
int lhip_gemm_ex(const float* A, const float* B, float* C, const float* bias, const float* gamma,
                 const float* rowscale, int M, int N, int K, long long a_rs, long long a_cs,
                 long long b_rs, long long b_cs, long long c_rs, long long c_cs, long long a_bs,
                 long long b_bs, long long c_bs, int batch, float alpha, float beta, float eps,
                 int pre_op, int post_op);
int lhip_elementwise(const float* a, const float* b, float* c, long long n, int op, float alpha, float beta);
int lhip_rmsnorm_ex(const float* x, const float* w, float* y, int rows, int cols, float eps);
int lhip_rmsnorm_bwd_ex(const float* x, const float* w, const float* dy, float* dx, float* dw, int rows,
                        int cols, float eps);
int lhip_row_rms(const float* x, float* out, int rows, int cols, long long rs, long long cs, float eps);
int lhip_softmax_ex(const float* x, const float* bias, float* y, int rows, int cols, float scale, int causal,
                    int group, int mask_offset);
int lhip_softmax_bwd_ex(const float* y, const float* dy, float* dx, int rows, int cols, float scale,
                        int causal, int group, int mask_offset);
int lhip_swiglu_fwd(const float* gate, int ld_gate, const float* up, int ld_up,
                    float* out, int ld_out, int rows, int cols);
int lhip_swiglu_bwd_ex(const float* a, const float* b, const float* dout, float* da, float* db, int rows,
                       int cols, int lda, int ldb, int ldo);
int lhip_rope(float* x, const int* pos_ids, int rows, int heads, int head_dim, int row_stride,
              int pos_offset, int pos_period, double base, int interleaved, int inverse);
int lhip_ce_fused(const float* logits, const int* targets, float* losses, float* dlogits,
                  int rows, int vocab, int ignore_index, float grad_scale);
int lhip_argmax_rows(const float* x, int* out, int rows, int cols);
int lhip_embed_fwd(const float* table, const int* ids, float* out, int n, int dim, int vocab);
int lhip_embed_bwd(const float* dout, const int* ids, float* dtable, int n, int dim, int vocab,
                   float scale, int accumulate);
int lhip_reduce_cols(const float* x, float* out, int rows, int cols, long long row_stride, float alpha,
                     float beta);
int lhip_l2_accum(const float* x, long long n, float* acc);
int lhip_clip_by_nsq(float* x, long long n, const float* nsq, float max_norm);
int lhip_sum_accum(const float* x, long long n, float scale, float* acc);
int lhip_transpose(const float* x, float* out, int rows, int cols);
int lhip_bcast_add(const float* x, const float* v, float* out, int rows, int cols, float alpha);
int lhip_adamw_elementwise(float* w, const float* g, float* m, float* v, float* w_mirror, long long n,
                           int step, float lr, float beta1, float beta2, float eps, float weight_decay,
                           float clip);
int lhip_program_begin(void);
int lhip_program_end(void** program);
int lhip_program_replay(void* program, int times);
int lhip_program_free(void* program);
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
if not C then
    M.reason = "liblanternl_hip.so not found (" .. tostring(load_err) .. ")"
    M.error = M.reason
    return M
end

local function ck(rc, what)
    if rc ~= 0 then
        local msg = ffi.string(C.lhip_last_error())
        error(("lanternl_hip[%s]: %s (%s)"):format(what, msg, STATUS[rc] or tostring(rc)), 2)
    end
    return rc
end

local okinit, initerr = pcall(function() ck(C.lhip_init(0), "init") end)
if not okinit then M.reason = tostring(initerr) M.error = M.reason return M end

local devinfo = ffi.new("lhip_devinfo_t")
ck(C.lhip_device_info(devinfo), "device_info")

M.available = true
M.reason = "ready"
M.device = ffi.string(devinfo.name)
M.C = C
M.luaTL = nil

local F32 = 0
M.F32 = F32
-- luaTL.EW / act / pre codes (cuda/luaTL_core.cu:49-90) = LHIP_EW_* / LHIP_ACT_* / LHIP_PRE_*
M.EW = { COPY = 0, ADD = 1, SUB = 2, MUL = 3, DIV = 4, SCALE = 5, AXPY = 6, FILL = 7, RELU = 8, GELU = 9,
         SILU = 10, TANH = 11, SIGMOID = 12, EXP = 13, SQRT = 14, RSQRT = 15, NEG = 16, RECIP = 17,
         ABS = 18, CLAMP = 19, DRELU = 20, DSILU = 21, DGELU = 22 }
M.ACT = { NONE = 0, RELU = 1, GELU = 2, SILU = 3, TANH = 4, SIGMOID = 5 }
M.PRE = { NONE = 0, RMSNORM = 1, GELU = 2, SILU = 3, RELU = 4 }
local EW = M.EW

local ok_tnew, tnew = pcall(require, "table.new")
if not ok_tnew then tnew = function() return {} end end

local f64_ct = ffi.typeof("double[?]")
local f32_ct = ffi.typeof("float[?]")

--  HOST LANES.  Marshaling goes through one grow-only cdata array per element
--  type and operand lane (LANE_A / LANE_B first and second operand, LANE_C the
--  result).  A lane grows to the next power of two that fits and never
--  shrinks, so calls of varied shapes settle on a handful of allocations.
local LANE_A, LANE_B, LANE_C = 1, 2, 3

local function pow2_at_least(n)
    local c = 256
    while c < n do c = c * 2 end
    return c
end

local HostLane = {}
HostLane.__index = HostLane
local function host_lane(ct) return setmetatable({ ct = ct, cap = 0, buf = nil }, HostLane) end
function HostLane:reserve(n)
    if n > self.cap then
        self.cap = pow2_at_least(n)
        self.buf = self.ct(self.cap)
    end
    return self.buf
end

local lanes = {
    f64 = { host_lane(f64_ct), host_lane(f64_ct), host_lane(f64_ct) },
    f32 = { host_lane(f32_ct), host_lane(f32_ct), host_lane(f32_ct) },
}

-- numbers [1..n] of a Lua table into elements [0..n-1] of a cdata array
local function pack(dst, src, n)
    for i = 0, n - 1 do dst[i] = src[i + 1] end
    return dst
end

-- elements [0..n-1] of a cdata array as a new 1-based Lua table
local function unpack_new(src, n)
    local t = tnew(n, 0)
    for i = 1, n do t[i] = src[i - 1] end
    return t
end

local function count_or_fail(tbl, need, what, level)
    local have = type(tbl) == "table" and #tbl or -1
    if have < need then
        error(("lanternl_hip: %s needs %d numbers, the table holds %d"):format(what, need, have), level + 1)
    end
end

--  TENSORS: a device fp32 matrix { data, rows, cols, dtype, nelem, nbytes } --
--  the role of a luaTL tensor.  Owning tensors free their memory from an FFI
--  finaliser; wrap() makes non-owning ones.
local Tensor = {}
Tensor.__index = Tensor
M.TensorClass = Tensor

local function new_tensor(rows, cols)
    local pp = ffi.new("void*[1]")
    ck(C.lhip_malloc(pp, math.max(rows * cols, 1) * 4), "alloc")
    local t = setmetatable({ rows = rows, cols = cols, dtype = F32, nelem = rows * cols,
                             nbytes = rows * cols * 4 }, Tensor)
    t.owner = ffi.gc(pp[0], function(p) C.lhip_free(p) end)
    t.data = ffi.cast("float*", t.owner)
    return t
end

--- Logical transpose as a stride view (luaTL_train.lua:120-122).
function Tensor:t() return M.view(self.data, self.cols, self.rows, 1, self.cols, 0) end
function Tensor:free()
    if self.owner ~= nil then C.lhip_free(ffi.gc(self.owner, nil)) end
    self.owner, self.data = nil, nil
end

-- device <-> Lua table, fp32 on the device, through a host lane
local function put_f32(dptr_, src, n, lane)
    local buf = pack(lanes.f32[lane]:reserve(n), src, n)
    ck(C.lhip_upload(dptr_, buf, n * 4), "upload")
end

local function fetch_f32(dptr_, n, lane)
    local buf = lanes.f32[lane]:reserve(n)
    ck(C.lhip_download(buf, dptr_, n * 4), "download")
    return unpack_new(buf, n)
end

--  DEVICE LANES: the flat-table calls' device operands, one grow-only buffer
--  per lane (the same policy as the host lanes).  Each call gets a
--  non-owning tensor shaped for it over its lane's buffer.
local dev_lanes = {}
local function dev_lane(lane, rows, cols)
    local need = math.max(rows * cols, 1)
    local store = dev_lanes[lane]
    if store == nil or store.nelem < need then
        if store ~= nil then store:free() end
        store = new_tensor(pow2_at_least(need), 1)
        dev_lanes[lane] = store
    end
    return setmetatable({ data = store.data, rows = rows, cols = cols, dtype = F32, nelem = rows * cols,
                          nbytes = rows * cols * 4 }, Tensor)
end

--  HANDLES (luatl_adapter.lua:46-101): a persistent GPU tensor exposed to lanternl
local Handle = {}
Handle.__index = Handle
M.HandleClass = Handle

local function is_handle(x) return type(x) == "table" and getmetatable(x) == Handle end
M.is_handle = is_handle

local function new_handle(t, rows, cols)
    return setmetatable({ t = t, rows = rows, cols = cols, __luatl_handle = true }, Handle)
end
M.new_handle = new_handle

--- Upload a flat Lua array once and keep it resident (luatl_adapter.lua:63-73):
--- the table must hold exactly rows*cols numbers.
function M.pin(flat, rows, cols)
    local n = rows * cols
    if type(flat) ~= "table" or #flat ~= n then
        error(("lanternl_hip.pin: a %dx%d matrix takes exactly %d numbers, the table holds %s")
              :format(rows, cols, n, type(flat) == "table" and tostring(#flat) or type(flat)), 2)
    end
    local h = new_handle(new_tensor(rows, cols), rows, cols)
    put_f32(h.t.data, flat, n, LANE_A)
    return h
end

--- A resident zero tensor (activations, grads, optimizer state) (:75-78).
function M.alloc(rows, cols)
    return new_handle(new_tensor(rows, cols), rows, cols):zero()
end

function Handle:toflat() return fetch_f32(self.t.data, self.rows * self.cols, LANE_C) end

function Handle:upload(flat)
    local n = self.rows * self.cols
    count_or_fail(flat, n, ("Handle:upload into %dx%d"):format(self.rows, self.cols), 2)
    put_f32(self.t.data, flat, n, LANE_A)
    return self
end

function Handle:zero() ck(C.lhip_zero(self.t.data, self.rows * self.cols * 4), "zero") return self end
function Handle:free()
    local t = self.t
    self.t = nil
    if t ~= nil then t:free() end
end
function Handle:tensor() return self.t end
function Handle:shape() return self.rows, self.cols end

-- a handle's tensor (resident), or a flat table copied into a device lane
local function operand(x, rows, cols, lane)
    if is_handle(x) then return x.t, true end
    local n = rows * cols
    count_or_fail(x, n, ("a %dx%d operand"):format(rows, cols), 2)
    local t = dev_lane(lane, rows, cols)
    put_f32(t.data, x, n, lane)
    return t, false
end

-- the call's result: a new handle over t when the inputs were resident,
-- otherwise a new flat table read back from t
local function deliver(t, rows, cols, resident)
    if resident then return new_handle(t, rows, cols) end
    return fetch_f32(t.data, rows * cols, LANE_C)
end

-- run `launch(X, O)` on a flat table or a handle; the output takes the input's form
local function row_call(x, rows, cols, launch)
    local X, resident = operand(x, rows, cols, LANE_A)
    local O = resident and new_tensor(rows, cols) or dev_lane(LANE_C, rows, cols)
    launch(X, O)
    return deliver(O, rows, cols, resident)
end

--  THE FLAT-TABLE PRODUCTS through lhip_matmul_host (double in and out).
--  op 0 = a(m x k).b(k x n), 1 = a(m x k).b(n x k)^T, 2 = a(m x k)^T.b(m x n)
local OPCODE = { nn = 0, nt = 1, tn = 2 }
local OPNAME = { [0] = "matmul", [1] = "matmul_nt", [2] = "matmul_tn" }

local function extents(code, m, k, n)
    if code == 0 then return m * k, k * n, m * n end
    if code == 1 then return m * k, n * k, m * n end
    return m * k, m * n, k * n
end

-- the product in the result lane (a cdata double array) and its element count
local function host_product(code, a, m, k, b, n)
    for _, d in ipairs({ m, k, n }) do
        if type(d) ~= "number" or d < 0 or d % 1 ~= 0 then
            error(("lanternl_hip: %s dimensions must be non-negative integers, got %s x %s x %s")
                  :format(OPNAME[code], tostring(m), tostring(k), tostring(n)), 3)
        end
    end
    local na, nb, nc = extents(code, m, k, n)
    count_or_fail(a, na, OPNAME[code] .. " operand a", 3)
    count_or_fail(b, nb, OPNAME[code] .. " operand b", 3)
    local A = pack(lanes.f64[LANE_A]:reserve(na), a, na)
    local B = pack(lanes.f64[LANE_B]:reserve(nb), b, nb)
    local R = lanes.f64[LANE_C]:reserve(nc)
    ck(C.lhip_matmul_host(code, A, B, R, m, k, n, 0), OPNAME[code])
    return R, nc
end

--  STRIDE VIEWS AND gemm_ex (luaTL_train.lua:113-172)
--- Explicit stride view: rs = row stride, cs = column stride, bs = batch stride (elements) (:200-203).
function M.view(ptr, rows, cols, rs, cs, bs)
    if type(ptr) == "table" then ptr = is_handle(ptr) and ptr.t.data or ptr.data end
    return { data = ffi.cast("float*", ptr), rows = rows, cols = cols, rs = rs, cs = cs, bs = bs or 0,
             dtype = F32, nelem = rows * cols }
end

local function coerce(x)
    if is_handle(x) then x = x.t end
    if x.rs then return x end
    return { data = x.data, rows = x.rows, cols = x.cols, rs = x.cols, cs = 1, bs = 0, dtype = F32 }
end

local function dptr(x)
    if x == nil then return nil end
    if is_handle(x) then return x.t.data end
    if type(x) == "table" then return x.data end
    return x
end

--- Cc = act(alpha * pre(A) @ B + bias) + beta*Cc on tensors, handles or stride views
--- (luaTL.gemm_ex, luaTL_train.lua:154-172); opts alpha, beta, bias, gamma, rowscale,
--- batch, eps, pre, act.
function M.gemm_ex(A, B, Cc, o)
    o = o or {}
    local a, b, c = coerce(A), coerce(B), coerce(Cc)
    if b.rows ~= a.cols then
        error(("gemm_ex: inner dim mismatch %dx%d @ %dx%d"):format(a.rows, a.cols, b.rows, b.cols), 2)
    end
    ck(C.lhip_gemm_ex(a.data, b.data, c.data, dptr(o.bias), dptr(o.gamma), dptr(o.rowscale),
                      a.rows, b.cols, a.cols, a.rs, a.cs, b.rs, b.cs, c.rs, c.cs, a.bs, b.bs, c.bs,
                      o.batch or 1, o.alpha or 1.0, o.beta or 0.0, o.eps or 1e-5, o.pre or 0, o.act or 0),
       "gemm_ex")
    return Cc
end

local function tview(x)
    if is_handle(x) then x = x.t end
    return M.view(x.data, x.cols, x.rows, 1, x.cols, 0)
end

--  LEGACY-COMPATIBLE ENTRY POINTS (signatures unchanged, luatl_adapter.lua:126-159)

--- a(m x k) . b(k x n): two flat tables -> a new flat table of m*n numbers
--- (the registry's contract, matrix.lua:178-202); two handles -> a new handle;
--- a handle and a table -> a new flat table.
function M.matmul(a, m, k, b, n)
    if not (is_handle(a) or is_handle(b)) then
        return unpack_new(host_product(0, a, m, k, b, n))
    end
    local A, ra = operand(a, m, k, LANE_A)
    local B, rb = operand(b, k, n, LANE_B)
    local resident = ra and rb
    local out = resident and new_tensor(m, n) or dev_lane(LANE_C, m, n)
    M.gemm_ex(A, B, out)
    return deliver(out, m, n, resident)
end

--- a(m x k) . b(n x k)^T -> a new flat table of m*n numbers (matrix.matmul_nt, matrix.lua:597-625)
function M.matmul_nt(a, m, k, b, n) return unpack_new(host_product(1, a, m, k, b, n)) end

--- a(m x k)^T . b(m x n) -> a new flat table of k*n numbers (matrix.matmul_tn, matrix.lua:627-660)
function M.matmul_tn(a, m, k, b, n) return unpack_new(host_product(2, a, m, k, b, n)) end

--- The product `op` ("nn", "nt" or "tn", shapes as in matmul / matmul_nt /
--- matmul_tn) of two flat tables, written into the caller's flat table rd:
--- rd = product when acc is false, rd = rd + product (in double) when acc is
--- true.  This is what matrix.multiply / matmul_nt / matmul_tn call when they
--- are given `out` (the autograd backward's grad_of(x) with acc = true,
--- tensor2.lua:206-211,222-227).  rd is written only after the device call
--- has succeeded, so an error leaves it untouched.  Returns rd.
function M.matmul_into(op, a, m, k, b, n, rd, acc)
    local code = OPCODE[op]
    if code == nil then
        error(("lanternl_hip.matmul_into: op must be \"nn\", \"nt\" or \"tn\", got %s"):format(tostring(op)), 2)
    end
    local nc = select(3, extents(code, m, k, n))
    if type(rd) ~= "table" or #rd < nc then
        error(("lanternl_hip.matmul_into: rd must be a flat table of %d numbers"):format(nc), 2)
    end
    local R = host_product(code, a, m, k, b, n)
    if acc then
        for i = 1, nc do rd[i] = rd[i] + R[i - 1] end
    else
        for i = 1, nc do rd[i] = R[i - 1] end
    end
    return rd
end

function M.rmsnorm(x, rows, cols, w, eps)
    local gain = w and (operand(w, 1, cols, LANE_B)) or nil
    return row_call(x, rows, cols, function(X, O)
        ck(C.lhip_rmsnorm_ex(X.data, gain and gain.data or nil, O.data, rows, cols, eps or 1e-5), "rmsnorm")
    end)
end

function M.softmax(x, rows, cols)
    return row_call(x, rows, cols, function(X, O)
        ck(C.lhip_softmax_ex(X.data, nil, O.data, rows, cols, 1.0, 0, 0, 0), "softmax")
    end)
end

function M.softmax_causal(x, rows, cols, scale, group)
    return row_call(x, rows, cols, function(X, O)
        ck(C.lhip_softmax_ex(X.data, nil, O.data, rows, cols, scale or 1.0, 1, group or 0, 0), "softmax_causal")
    end)
end

--  RESIDENT-MODE PRIMITIVES (luatl_adapter.lua:161-187)

function M.gemm(hA, hB, hC, opts) M.gemm_ex(hA.t, hB.t, hC.t, opts) return hC end
--- dX = dY . W^T + beta*dX (luaTL.matmul_dx, luaTL_train.lua:174-177)
function M.gemm_dx(hdY, hW, hdX, beta) M.gemm_ex(hdY.t, tview(hW), hdX.t, { beta = beta or 0.0 }) return hdX end
--- dW = X^T . dY + beta*dW, beta defaulting to 1 (luaTL.matmul_dw, luaTL_train.lua:179-182)
function M.gemm_dw(hX, hdY, hdW, beta)
    M.gemm_ex(tview(hX), hdY.t, hdW.t, { beta = beta == nil and 1.0 or beta })
    return hdW
end

--- Tensor:add_inplace (luaTL.lua:633-638): the AXPY operator with a = dst,
--- b = src, i.e. dst = alpha*dst + src.
function M.add_inplace(hDst, hSrc, alpha)
    ck(C.lhip_elementwise(hDst.t.data, hSrc.t.data, hDst.t.data, hDst.t.nelem, EW.AXPY, alpha or 1.0, 0.0),
       "add_inplace")
    return hDst
end
function M.silu_inplace(h)
    ck(C.lhip_elementwise(h.t.data, nil, h.t.data, h.t.nelem, EW.SILU, 0.0, 0.0), "silu_inplace")
    return h
end
function M.gelu_inplace(h)
    ck(C.lhip_elementwise(h.t.data, nil, h.t.data, h.t.nelem, EW.GELU, 0.0, 0.0), "gelu_inplace")
    return h
end
function M.scale_inplace(h, a)
    ck(C.lhip_elementwise(h.t.data, nil, h.t.data, h.t.nelem, EW.SCALE, a, 0.0), "scale_inplace")
    return h
end

--  Tensor:rope (luaTL_train.lua:225-234): in place, half-split pairs unless o.interleaved
local function rope_call(x, o)
    o = o or {}
    local heads = o.heads or 1
    local hd = o.head_dim or (x.cols / heads)
    local rs = o.row_stride or x.cols
    ck(C.lhip_rope(x.data, o.pos_ids and ffi.cast("int*", dptr(o.pos_ids)) or nil, x.rows, heads, hd,
                   rs > 0 and rs or heads * hd, o.pos_offset or 0, 0, o.theta or 10000.0,
                   o.interleaved and 1 or 0, o.inverse and 1 or 0), "rope")
end
function M.rope(h, o) rope_call(h.t, o) return h end

--  luaTL.swiglu (luaTL_train.lua:209-215): out = silu(a) * b
local function swiglu_call(a, b, out, o)
    o = o or {}
    ck(C.lhip_swiglu_fwd(a.data, o.lda or a.cols, b.data, o.ldb or b.cols, out.data, o.ldo or out.cols,
                         out.rows, out.cols), "swiglu")
end
function M.swiglu(ha, hb, ho, o) swiglu_call(ha.t, hb.t, ho.t, o) return ho end

function M.rmsnorm_bwd(hx, hg, hdy, hdx, hdg, eps)
    local x = hx.t
    ck(C.lhip_rmsnorm_bwd_ex(x.data, hg and hg.t.data or nil, hdy.t.data, hdx.t.data,
                             hdg and hdg.t.data or nil, x.rows, x.cols, eps or 1e-5), "rmsnorm_bwd")
    return hdx
end

local function softmax_bwd_call(y, dy, dx, o)
    o = o or {}
    ck(C.lhip_softmax_bwd_ex(y.data, dy.data, dx.data, y.rows, y.cols, o.scale or 1.0, o.causal and 1 or 0,
                             o.group or 0, o.mask_offset or 0), "softmax_bwd")
end
function M.softmax_bwd(hy, hdy, hdx, o) softmax_bwd_call(hy.t, hdy.t, hdx.t, o) return hdx end

function M.sync() ck(C.lhip_sync(), "sync") end

--- Memory statistics under the reference pool's keys (luaTL.pool_stats, luaTL.lua:308-325).
--- There is no caching pool: every allocation is a hipMalloc.
local mstats = ffi.new("lhip_mem_stats_t")
function M.stats()
    ck(C.lhip_mem_stats(mstats), "stats")
    local s = mstats
    return {
        reserved = tonumber(s.bytes_in_use + s.workspace_bytes + s.staging_bytes),
        in_use = tonumber(s.bytes_in_use), peak = tonumber(s.peak_in_use), blocks = tonumber(s.live_buffers),
        free_blocks = 0, allocs = tonumber(s.n_alloc), frees = tonumber(s.n_free),
        cuda_malloc = tonumber(s.n_alloc), cuda_free = tonumber(s.n_free), cache_hit = 0,
        cache_miss = tonumber(s.n_alloc), trims = 0,
        workspace = tonumber(s.workspace_bytes), staging = tonumber(s.staging_bytes),
    }
end

local u64a, u64b = ffi.new("unsigned long long[1]"), ffi.new("unsigned long long[1]")
function M.mem()
    ck(C.lhip_mem_info(u64a, u64b), "mem")
    return tonumber(u64a[0]), tonumber(u64b[0])
end

--- Device description under the reference's keys (luaTL.hardware, luaTL.lua:279-305).
function M.hardware()
    ck(C.lhip_device_info(devinfo), "hardware")
    local d = devinfo
    local free, total = M.mem()
    local cus = d.compute_units
    return {
        name = ffi.string(d.name), sm = ffi.string(d.arch):match("^[^:]*"), major = 9, minor = 5,
        multiprocessors = cus, cores_per_sm = 64, cuda_cores = 64 * cus, warp_size = d.wavefront_size,
        max_threads_block = 1024, max_threads_sm = 2048, shared_per_block = tonumber(d.lds_per_block),
        shared_per_sm = 160 * 1024, total_vram = total, free_vram = free, l2_cache = d.l2_bytes,
        bandwidth_gbs = d.peak_hbm_gbps, gflops_fp32 = d.peak_fp32_matrix_tflops * 1000,
        gflops_fp16 = 0, tensor_cores = true, fp16 = false, bf16 = false,
    }
end

--  RESIDENT TENSOR TOOLKIT (luatl_adapter.lua:188-246)

--- Element-offset pointer into a tensor's (or handle's, or view's) f32 storage.
function M.offset(t, elems)
    return ffi.cast("char*", dptr(t)) + elems * 4
end

--- Column slice [col0, col0 + w) keeping the parent's leading dimension.
function M.cols(t, col0, w)
    local base = is_handle(t) and t.t or t
    return M.view(ffi.cast("float*", base.data) + col0, base.rows, w, base.cols, 1, 0)
end

--- Non-owning tensor over a raw device pointer.
function M.wrap(ptr, rows, cols)
    return setmetatable({ data = ffi.cast("float*", ptr), rows = rows, cols = cols, dtype = F32,
                          nelem = rows * cols, nbytes = rows * cols * 4 }, Tensor)
end

--- A zeroed device buffer for n int32 ids: an n x 1 tensor, since ids and
--- fp32 values are both 4 bytes wide.
function M.ids(n) return M.alloc(n, 1) end

function M.upload_i32(t, cbuf, n) ck(C.lhip_upload(dptr(t), cbuf, n * 4), "adapter.upload_i32") end
function M.download_i32(t, cbuf, n) ck(C.lhip_download(cbuf, dptr(t), n * 4), "adapter.download_i32") end
function M.download_f32(ptr, cbuf, n) ck(C.lhip_download(cbuf, dptr(ptr), n * 4), "adapter.download_f32") end

--- The first fp32 value of a device tensor, handle or view (a loss, a norm).
function M.scalar(t) return fetch_f32(dptr(t), 1, LANE_C)[1] end

--  PROGRAM: luaTL.Program's op list (ai/gpu/luaTL_train.lua:332-632) over this
--  library.  Each op method queues one library call; run(keep) issues the
--  queue on the library stream (then, unless async(true), waits and, with
--  timing, reads the elapsed time) and clears it unless keep; capture()
--  records the queue once into a hipGraph (run it first: a recording cannot
--  allocate); replay() launches the graph, or runs the queue when nothing is
--  captured.  barrier() waits for the stream when run and is skipped in a
--  capture, as luaTL_prog_capture skips SYNC ops (luaTL_train.cu:1614-1660).
local Prog = {}
Prog.__index = Prog
M.ProgramClass = Prog

local function new_event()
    local pp = ffi.new("void*[1]")
    ck(C.lhip_event_create(pp), "event")
    return ffi.gc(pp[0], C.lhip_event_destroy)
end

function M.program(cap, timing)
    local p = setmetatable({ ops = {}, capacity = (cap and cap > 0) and cap or 4096, timing = timing and true,
                             flags = 1, last_ms = -1.0, total_runs = 0 }, Prog)
    if p.timing then p.ev0, p.ev1 = new_event(), new_event() end
    return p
end

function Prog:reset() self.ops = {} return self end
function Prog:size() return #self.ops end
function Prog:async(on) self.flags = on and 0 or 1 return self end

function Prog:push(fn, is_sync)
    local n = #self.ops
    if n >= self.capacity then error("luaTL.Program full (" .. self.capacity .. ")", 3) end
    self.ops[n + 1] = { fn = fn, sync = is_sync }
    return self
end

function Prog:gemm(A, B, Cc, o) return self:push(function() M.gemm_ex(A, B, Cc, o) end) end
function Prog:matmul(A, B, Cc, o) return self:gemm(A, B, Cc, o) end
function Prog:dx(dY, W, dX, beta) return self:gemm(dY, tview(W), dX, { beta = beta or 0.0 }) end
function Prog:dw(X, dY, dW, beta) return self:gemm(tview(X), dY, dW, { beta = beta == nil and 1.0 or beta }) end

function Prog:ew(op, A, B, out, alpha, beta)
    return self:push(function()
        ck(C.lhip_elementwise(dptr(A), dptr(B), dptr(out), out.nelem or out.rows * out.cols, op, alpha or 1.0,
                              beta or 0.0), "prog.ew")
    end)
end
function Prog:add(A, B, out) return self:ew(EW.ADD, A, B, out, 1, 1) end
function Prog:axpy(dst, B, a) return self:ew(EW.AXPY, dst, B, dst, a or 1, 0) end
function Prog:scale(dst, a) return self:ew(EW.SCALE, dst, nil, dst, a, 0) end
function Prog:dsilu(x, dy, out) return self:ew(EW.DSILU, x, dy, out, 1, 0) end
function Prog:dgelu(x, dy, out) return self:ew(EW.DGELU, x, dy, out, 1, 0) end

function Prog:rmsnorm(x, w, out, eps)
    return self:push(function()
        ck(C.lhip_rmsnorm_ex(x.data, dptr(w), out.data, x.rows, x.cols, eps or 1e-5), "prog.rmsnorm")
    end)
end

function Prog:rmsnorm_bwd(x, gamma, dy, dx, dgamma, eps)
    return self:push(function()
        ck(C.lhip_rmsnorm_bwd_ex(x.data, dptr(gamma), dy.data, dx.data, dptr(dgamma), x.rows, x.cols, eps or 1e-5),
           "prog.rmsnorm_bwd")
    end)
end

function Prog:softmax(x, out, o)
    o = o or {}
    return self:push(function()
        ck(C.lhip_softmax_ex(x.data, dptr(o.bias), out.data, x.rows, x.cols, o.scale or 1.0, o.causal and 1 or 0,
                             o.group or 0, o.mask_offset or 0), "prog.softmax")
    end)
end

function Prog:softmax_bwd(y, dy, dx, o) return self:push(function() softmax_bwd_call(y, dy, dx, o) end) end
function Prog:swiglu(a, b, out, o) return self:push(function() swiglu_call(a, b, out, o) end) end

function Prog:swiglu_bwd(a, b, dout, da, db, o)
    o = o or {}
    return self:push(function()
        ck(C.lhip_swiglu_bwd_ex(a.data, b.data, dout.data, dptr(da), dptr(db), dout.rows, dout.cols,
                                o.lda or a.cols, o.ldb or b.cols, o.ldo or dout.cols), "prog.swiglu_bwd")
    end)
end

function Prog:rope(x, o) return self:push(function() rope_call(x, o) end) end

function Prog:embed(ids, tbl, out)
    return self:push(function()
        ck(C.lhip_embed_fwd(tbl.data, ffi.cast("int*", dptr(ids)), out.data, out.rows, out.cols, tbl.rows),
           "prog.embed")
    end)
end

function Prog:embed_bwd(ids, dout, dtable, scale)
    return self:push(function()
        ck(C.lhip_embed_bwd(dout.data, ffi.cast("int*", dptr(ids)), dtable.data, dout.rows, dout.cols,
                            dtable.rows, scale or 1.0, 1), "prog.embed_bwd")
    end)
end

function Prog:cross_entropy(logits, targets, losses, dlogits, o)
    o = o or {}
    return self:push(function()
        ck(C.lhip_ce_fused(logits.data, ffi.cast("int*", dptr(targets)), dptr(losses), dptr(dlogits), logits.rows,
                           logits.cols, o.ignore_index or -1, o.grad_scale or (1.0 / logits.rows)),
           "prog.cross_entropy")
    end)
end

function Prog:reduce_cols(x, out, alpha, beta, rs)
    return self:push(function()
        ck(C.lhip_reduce_cols(x.data, dptr(out), x.rows, x.cols, rs or x.cols, alpha or 1.0, beta or 0.0),
           "prog.reduce_cols")
    end)
end

function Prog:l2(x, acc)
    return self:push(function() ck(C.lhip_l2_accum(x.data, x.nelem, dptr(acc)), "prog.l2") end)
end

function Prog:clip(x, nsq, max_norm)
    return self:push(function() ck(C.lhip_clip_by_nsq(x.data, x.nelem, dptr(nsq), max_norm), "prog.clip") end)
end

function Prog:adamw(w, g, m, v, w_lp, o)
    o = o or {}
    return self:push(function()
        ck(C.lhip_adamw_elementwise(w.data, g.data, m.data, v.data, dptr(w_lp), w.nelem, o.step or 1,
                                    o.lr or 1e-3, o.beta1 or 0.9, o.beta2 or 0.999, o.eps or 1e-8, o.wd or 0.0,
                                    o.clip or 0.0), "prog.adamw")
    end)
end

function Prog:zero(t) return self:push(function() ck(C.lhip_zero(t.data, t.nbytes), "prog.zero") end) end
function Prog:copy(src, dst)
    return self:push(function() ck(C.lhip_copy(dst.data, src.data, src.nbytes), "prog.copy") end)
end
function Prog:cast(src, dst)
    if (src.dtype or F32) ~= F32 or (dst.dtype or F32) ~= F32 then
        error("luaTL.Program:cast: this build holds fp32 only", 2)
    end
    return self:copy(src, dst)
end

function Prog:transpose(x, out)
    return self:push(function() ck(C.lhip_transpose(x.data, out.data, x.rows, x.cols), "prog.transpose") end)
end

function Prog:bcast_add(x, vec, out, alpha)
    return self:push(function()
        ck(C.lhip_bcast_add(x.data, dptr(vec), out.data, x.rows, x.cols, alpha or 1.0), "prog.bcast_add")
    end)
end

function Prog:barrier() return self:push(function() ck(C.lhip_sync(), "prog.barrier") end, true) end

function Prog:argmax(x, out)
    return self:push(function()
        ck(C.lhip_argmax_rows(x.data, ffi.cast("int*", dptr(out)), x.rows, x.cols), "prog.argmax")
    end)
end

function Prog:sum(x, acc, scale)
    return self:push(function() ck(C.lhip_sum_accum(x.data, x.nelem, scale or 1.0, dptr(acc)), "prog.sum") end)
end

function Prog:gather(src, idx, dst)
    return self:push(function()
        ck(C.lhip_embed_fwd(src.data, ffi.cast("int*", dptr(idx)), dst.data, dst.rows, dst.cols, src.rows),
           "prog.gather")
    end)
end

function Prog:row_rms(x, out, eps, rs, cs)
    return self:push(function()
        ck(C.lhip_row_rms(x.data, dptr(out), x.rows, x.cols, rs or x.cols, cs or 1, eps or 1e-5), "prog.row_rms")
    end)
end

local ms_buf = ffi.new("float[1]")
function Prog:finish()
    if self.flags == 1 then
        if self.ev1 then
            ck(C.lhip_event_elapsed_ms(self.ev0, self.ev1, ms_buf), "prog.elapsed")
            self.last_ms = ms_buf[0]
        else
            ck(C.lhip_sync(), "prog.sync")
        end
    end
    self.total_runs = self.total_runs + 1
end

function Prog:run(keep)
    if #self.ops == 0 then return self end
    if self.ev0 then ck(C.lhip_event_record(self.ev0), "prog.event") end
    for i = 1, #self.ops do self.ops[i].fn() end
    if self.ev1 then ck(C.lhip_event_record(self.ev1), "prog.event") end
    self:finish()
    if not keep then self.ops = {} end
    return self
end

--- Record the current op list as a hipGraph (barriers skipped).  Run it once first.
function Prog:capture()
    if #self.ops == 0 then error("Program:capture: the op list is empty (ARG)", 2) end
    self:free_graph()
    ck(C.lhip_sync(), "prog.capture")
    ck(C.lhip_program_begin(), "prog.capture")
    local ok, err = pcall(function()
        for i = 1, #self.ops do
            if not self.ops[i].sync then self.ops[i].fn() end
        end
    end)
    if not ok then
        C.lhip_program_end(nil)              -- discard the partial recording
        error(err, 2)
    end
    local h = ffi.new("void*[1]")
    ck(C.lhip_program_end(h), "prog.capture")
    self.graph = ffi.gc(h[0], C.lhip_program_free)
    return self
end

function Prog:replay()
    if not self.graph then return self:run(true) end
    if self.ev0 then ck(C.lhip_event_record(self.ev0), "prog.event") end
    ck(C.lhip_program_replay(self.graph, 1), "prog.replay")
    if self.ev1 then ck(C.lhip_event_record(self.ev1), "prog.event") end
    self:finish()
    return self
end

function Prog:wait()
    ck(C.lhip_sync(), "prog.wait")
    if self.ev1 then
        ck(C.lhip_event_elapsed_ms(self.ev0, self.ev1, ms_buf), "prog.elapsed")
        self.last_ms = ms_buf[0]
    end
    return self
end

function Prog:elapsed_ms() return self.last_ms end
function Prog:is_captured() return self.graph ~= nil end
function Prog:free_graph()
    if self.graph ~= nil then
        C.lhip_program_free(ffi.gc(self.graph, nil))
        self.graph = nil
    end
    return self
end

function M.shutdown()
    for lane, store in pairs(dev_lanes) do
        store:free()
        dev_lanes[lane] = nil
    end
    C.lhip_shutdown()
    M.available = false
    M.reason = "shut down"
    M.error = M.reason
end

return M
