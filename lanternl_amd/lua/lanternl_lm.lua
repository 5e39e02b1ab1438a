--  lanternl_lm.lua -- the CPU LMTrain step run on the GPU (liblanternl_hip.so's
--  lhip_lm_* entry points, MI355X / gfx950), for a LuaJIT host that holds the
--  reference's Transformer and LMTrain.
--
--  One optimizer step of ai/optim/lmtrain.lua:1183-1227 on the device: the
--  forward of ai/nn/transformer.lua:196-257 over a batch of windows, each
--  window's mean CE, the backward, grads scaled by 1/n_in_batch, the global
--  norm skip and clip, and SGD (optim2.lua:48-102) or AdamW (optim2.lua:
--  104-164) -- enqueued with no host round trip.  The weights stay on the
--  device between steps; this module moves them to and from the host's
--  Transformer only when asked (load_model / store_model), for evaluation or
--  checkpoints on the host.
--
--    local lm = require("lanternl_lm")
--    local step = lm.new{ vocab = 2000, dim = 128, layers = 4, heads = 8, ffn = 256,
--                         batch = 8, seq = 64 }
--    step:load_model(model)                      -- Transformer:parameters(), in order
--    step:set_windows(windows, lo, hi)           -- build_windows' { inp, tgt, n }, 1-based ids
--    step:sgd{ lr = lr, momentum = 0.9, weight_decay = 0.01, clip = 1.0 }
--    local st = step:stats()                     -- loss, grad_norm, applied, correct, ...
--    step:store_model(model)                     -- the device weights back into the tensors
--
--  The library is the one luatl_adapter.lua loads (its `C`); when that
--  module is unavailable so is this one, with the same reason.  Errors raise
--  "lanternl_lm[<what>]: <message> (<STATUS>)".

local M = { available = false, reason = "not loaded" }

local okffi, ffi = pcall(require, "ffi")
if not okffi then M.reason = "LuaJIT FFI unavailable" return M end
local okad, adapter = pcall(require, "luatl_adapter")
if not okad then M.reason = "luatl_adapter: " .. tostring(adapter) return M end
if not adapter.available then M.reason = adapter.reason return M end
local C = adapter.C

ffi.cdef[[
typedef struct {
    int vocab, dim, layers, heads, ffn;
    int causal;
    double eps;
    double rope_base;
    int batch;
    int seq;
} lhip_lm_config_t;
typedef struct {
    float loss;
    float grad_norm;
    int applied;
    int correct;
    int steps;
} lhip_lm_stats_t;
typedef struct {
    int format;
    int keep;
    int epoch;
    double loss;
    double best_loss;
    const char* backend;
    const char* extra;
} lhip_ckpt_info_t;
typedef struct {
    int version;
    int format;
    int dtype_bytes;
    int epoch;
    double loss, best_loss;
    int causal, tie, max_seq;
    double rope_base;
} lhip_ckpt_header_t;
long long lhip_lm_num_params(const lhip_lm_config_t* cfg);
int lhip_lm_param_offsets(const lhip_lm_config_t* cfg, long long* offsets, int* rows, int* cols);
int lhip_lm_create(const lhip_lm_config_t* cfg, void** model);
int lhip_lm_destroy(void* model);
int lhip_lm_set_params(void* model, const float* host, long long n);
int lhip_lm_get_params(void* model, float* host, long long n);
int lhip_lm_get_grads(void* model, float* host, long long n);
int lhip_lm_set_velocity(void* model, const float* host, long long n);
int lhip_lm_get_velocity(void* model, float* host, long long n);
int lhip_lm_set_batch_ex(void* model, const int* ids, const int* targets, const int* lengths, int n_windows);
int lhip_lm_use_graph(void* model, int on);
int lhip_lm_step_sgd(void* model, float lr, float momentum, float weight_decay, float clip_norm, int nesterov);
int lhip_lm_step_adamw(void* model, float lr, float beta1, float beta2, float eps, float weight_decay,
                       float clip_norm);
int lhip_lm_set_adam_state(void* model, const float* m, const float* v, long long n, int step);
int lhip_lm_get_adam_state(void* model, float* m, float* v, long long n, int* step);
int lhip_lm_stats(void* model, lhip_lm_stats_t* out, float* window_losses, int nwin);
int lhip_lm_get_argmax(void* model, int* host, int n);
int lhip_lm_save(void* model, const char* path, const lhip_ckpt_info_t* info);
int lhip_lm_load(void* model, const char* path, lhip_ckpt_header_t* header);
]]

local STATUS = { [0] = "OK", [-1] = "NULL", [-2] = "SHAPE", [-3] = "DTYPE", [-4] = "DEVICE",
                 [-5] = "OOM", [-6] = "ARG", [-7] = "CAPACITY", [-8] = "UNSUPPORTED" }

local function check(rc, what)
    if rc ~= 0 then
        error(("lanternl_lm[%s]: %s (%s)"):format(what, ffi.string(C.lhip_last_error()),
                                                  STATUS[rc] or tostring(rc)), 3)
    end
end

local PER_LAYER = { "ln1", "wq", "wk", "wv", "wo", "ln2", "w1", "w3", "w2" }

-- the configuration struct from a table of LMTrain / Transformer options
local function make_config(o)
    local cfg = ffi.new("lhip_lm_config_t")
    for _, k in ipairs({ "vocab", "dim", "layers", "heads", "ffn", "batch", "seq" }) do
        if type(o[k]) ~= "number" or o[k] < 1 or o[k] % 1 ~= 0 then
            error(("lanternl_lm.new: option %s must be a positive integer, got %s"):format(k, tostring(o[k])), 3)
        end
        cfg[k] = o[k]
    end
    cfg.causal = (o.causal == nil or o.causal) and 1 or 0
    cfg.eps = o.eps or 1e-5
    cfg.rope_base = o.rope_base or 10000.0
    return cfg
end

--- The flat parameter layout of a configuration: a list of
--- { name, offset (0-based), rows, cols }, in Transformer:parameters() order
--- (transformer.lua:150-164: emb, then ln1 wq wk wv wo ln2 w1 w3 w2 per layer, lnf).
function M.layout(o)
    local cfg = make_config(o)
    local nt = 2 + 9 * o.layers
    local off, rows, cols = ffi.new("long long[?]", nt), ffi.new("int[?]", nt), ffi.new("int[?]", nt)
    check(C.lhip_lm_param_offsets(cfg, off, rows, cols), "layout")
    local out = {}
    for i = 0, nt - 1 do
        local name
        if i == 0 then name = "emb"
        elseif i == nt - 1 then name = "lnf"
        else
            local l = math.floor((i - 1) / 9)
            name = PER_LAYER[(i - 1) % 9 + 1] .. "." .. (l + 1)
        end
        out[i + 1] = { name = name, offset = tonumber(off[i]), rows = rows[i], cols = cols[i] }
    end
    return out
end

local Step = {}
Step.__index = Step
M.StepClass = Step

--- A device-resident model and its optimizer state for one configuration:
--- o = { vocab, dim, layers, heads, ffn, batch (windows per step), seq
--- (tokens per window), causal = true, eps = 1e-5, rope_base = 10000 }.
function M.new(o)
    local cfg = make_config(o)
    local n = tonumber(C.lhip_lm_num_params(cfg))
    if n < 0 then error("lanternl_lm.new: " .. ffi.string(C.lhip_last_error()), 2) end
    local box = ffi.new("void*[1]")
    check(C.lhip_lm_create(cfg, box), "create")
    local s = setmetatable({ cfg = cfg, n = n, batch = o.batch, seq = o.seq, layers = o.layers,
                             handle = ffi.gc(box[0], C.lhip_lm_destroy) }, Step)
    s.flat = ffi.new("float[?]", n)                   -- host side of params / grads / moments
    s.flat2 = ffi.new("float[?]", n)
    s.ids = ffi.new("int[?]", o.batch * o.seq)
    s.tgt = ffi.new("int[?]", o.batch * o.seq)
    s.lens = ffi.new("int[?]", o.batch)
    s.wloss = ffi.new("float[?]", o.batch)
    s.st = ffi.new("lhip_lm_stats_t")
    s.layout = M.layout(o)
    return s
end

function Step:free()
    if self.handle ~= nil then
        C.lhip_lm_destroy(ffi.gc(self.handle, nil))
        self.handle = nil
    end
end

local function live(self, what)
    if self.handle == nil then error(("lanternl_lm[%s]: the step has been freed"):format(what), 3) end
    return self.handle
end

-- flat vector <-> Lua table
local function put_vector(self, src, what)
    if type(src) ~= "table" or #src ~= self.n then
        error(("lanternl_lm[%s]: expected a table of %d numbers"):format(what, self.n), 3)
    end
    local f = self.flat
    for i = 1, self.n do f[i - 1] = src[i] end
    return f
end

local function get_vector(self, fn, what)
    check(fn(live(self, what), self.flat, self.n), what)
    local out, f = {}, self.flat
    for i = 1, self.n do out[i] = f[i - 1] end
    return out
end

--- Parameters as one flat table of n numbers, in layout order.
function Step:set_params(flat)
    check(C.lhip_lm_set_params(live(self, "set_params"), put_vector(self, flat, "set_params"), self.n), "set_params")
    return self
end
function Step:params() return get_vector(self, C.lhip_lm_get_params, "params") end
--- The last step's gradients (scaled by 1/n_in_batch, before clipping).
function Step:grads() return get_vector(self, C.lhip_lm_get_grads, "grads") end
function Step:set_velocity(flat)
    check(C.lhip_lm_set_velocity(live(self, "set_velocity"), put_vector(self, flat, "set_velocity"), self.n),
          "set_velocity")
    return self
end
function Step:velocity() return get_vector(self, C.lhip_lm_get_velocity, "velocity") end

-- each tensor of Transformer:parameters(): a Tensor (its .data a matrix
-- { rows, cols, data }) or the matrix itself
local function tensor_matrix(p)
    if type(p) == "table" and type(p.data) == "table" and p.data.rows ~= nil then return p.data end
    return p
end

local function check_model(self, params, what)
    if type(params) ~= "table" or #params ~= #self.layout then
        error(("lanternl_lm[%s]: the model has %d parameter tensors, this configuration %d (a Transformer "
               .. "with a learned position table or an untied head has no counterpart here)")
              :format(what, type(params) == "table" and #params or 0, #self.layout), 3)
    end
    for i, L in ipairs(self.layout) do
        local mtx = tensor_matrix(params[i])
        if mtx.rows ~= L.rows or mtx.cols ~= L.cols then
            error(("lanternl_lm[%s]: tensor %d (%s) is %sx%s, the configuration needs %dx%d")
                  :format(what, i, L.name, tostring(mtx.rows), tostring(mtx.cols), L.rows, L.cols), 3)
        end
        if type(mtx.data) ~= "table" or #mtx.data ~= L.rows * L.cols then
            error(("lanternl_lm[%s]: tensor %d (%s) holds %s values, its %dx%d shape needs %d")
                  :format(what, i, L.name, type(mtx.data) == "table" and tostring(#mtx.data) or "no",
                          L.rows, L.cols, L.rows * L.cols), 3)
        end
    end
end

--- Copy a Transformer's parameters (model:parameters(), or that list itself)
--- into the device model.
function Step:load_model(model)
    local params = type(model.parameters) == "function" and model:parameters() or model
    check_model(self, params, "load_model")
    local f = self.flat
    for i, L in ipairs(self.layout) do
        local d = tensor_matrix(params[i]).data
        local base = L.offset
        for j = 1, L.rows * L.cols do f[base + j - 1] = d[j] end
    end
    check(C.lhip_lm_set_params(live(self, "load_model"), f, self.n), "load_model")
    return self
end

--- Copy the device weights back into a Transformer's parameter tensors.
function Step:store_model(model)
    local params = type(model.parameters) == "function" and model:parameters() or model
    check_model(self, params, "store_model")
    check(C.lhip_lm_get_params(live(self, "store_model"), self.flat, self.n), "store_model")
    local f = self.flat
    for i, L in ipairs(self.layout) do
        local d = tensor_matrix(params[i]).data
        local base = L.offset
        for j = 1, L.rows * L.cols do d[j] = f[base + j - 1] end
    end
    return self
end

--- The batch: windows[lo..hi] (default all), each build_windows' { inp, tgt,
--- n } with 1-based token ids (lmtrain.lua:535-558).  At most `batch`
--- windows of at most `seq` tokens; a short window or a short batch is
--- handled as LMTrain does (per-window mean CE, grads scaled by 1/n_in_batch).
function Step:set_windows(windows, lo, hi)
    lo = lo or 1
    hi = hi or #windows
    local nw = hi - lo + 1
    if nw < 1 or nw > self.batch then
        error(("lanternl_lm[set_windows]: %d windows for a batch of %d"):format(nw, self.batch), 2)
    end
    local ids, tgt, lens, T, V = self.ids, self.tgt, self.lens, self.seq, self.cfg.vocab
    for b = 0, self.batch - 1 do
        local w = windows[lo + b]
        local n = 0
        if b < nw then
            if type(w) ~= "table" or type(w[1]) ~= "table" or type(w[2]) ~= "table" then
                error(("lanternl_lm[set_windows]: window %d is not an { inp, tgt, n } table"):format(lo + b), 2)
            end
            n = w[3] or #w[1]
            if type(n) ~= "number" or n % 1 ~= 0 or n < 1 or n > T or #w[1] < n or #w[2] < n then
                error(("lanternl_lm[set_windows]: window %d holds %s tokens (1..%d, with as many targets)")
                      :format(lo + b, tostring(n), T), 2)
            end
        end
        lens[b] = n
        for t = 0, T - 1 do
            local id, tg = 0, 0
            if t < n then
                id, tg = w[1][t + 1] - 1, w[2][t + 1] - 1
                if id < 0 or id >= V or tg < 0 or tg >= V then
                    error(("lanternl_lm[set_windows]: window %d token %d: id %s / target %s outside 1..%d")
                          :format(lo + b, t + 1, tostring(id + 1), tostring(tg + 1), V), 2)
                end
            end
            ids[b * T + t], tgt[b * T + t] = id, tg
        end
    end
    check(C.lhip_lm_set_batch_ex(live(self, "set_windows"), ids, tgt, lens, nw), "set_windows")
    self.n_windows = nw
    return self
end

--- Capture the step into a hipGraph on the next call and replay it afterwards.
function Step:use_graph(on)
    check(C.lhip_lm_use_graph(live(self, "use_graph"), on and 1 or 0), "use_graph")
    return self
end

--- One SGD step (LMTrain's optimizer "sgd"; asynchronous, stats() waits):
--- o = { lr, momentum = 0.9, weight_decay = 0.01, clip = 1.0, nesterov = false }.
function Step:sgd(o)
    if type(o) ~= "table" or type(o.lr) ~= "number" then error("lanternl_lm.sgd: o.lr is required", 2) end
    check(C.lhip_lm_step_sgd(live(self, "sgd"), o.lr, o.momentum or 0.9, o.weight_decay or 0.01, o.clip or 1.0,
                             o.nesterov and 1 or 0), "sgd")
    return self
end

--- One AdamW step (LMTrain's default optimizer, lmtrain.lua:25-26):
--- o = { lr = 1e-3, beta1 = 0.9, beta2 = 0.95, eps = 1e-8, weight_decay = 0.01, clip = 1.0 }.
function Step:adamw(o)
    o = o or {}
    check(C.lhip_lm_step_adamw(live(self, "adamw"), o.lr or 1e-3, o.beta1 or 0.9, o.beta2 or 0.95, o.eps or 1e-8,
                               o.weight_decay or 0.01, o.clip or 1.0), "adamw")
    return self
end

--- AdamW moments (flat tables, either may be nil) and step count.
function Step:set_adam_state(m, v, t)
    local pm = m and put_vector(self, m, "set_adam_state") or nil
    local pv = nil
    if v then
        if type(v) ~= "table" or #v ~= self.n then
            error(("lanternl_lm[set_adam_state]: expected a table of %d numbers"):format(self.n), 2)
        end
        pv = self.flat2
        for i = 1, self.n do pv[i - 1] = v[i] end
    end
    check(C.lhip_lm_set_adam_state(live(self, "set_adam_state"), pm, pv, self.n, t or 0), "set_adam_state")
    return self
end

function Step:adam_state()
    local t = ffi.new("int[1]")
    check(C.lhip_lm_get_adam_state(live(self, "adam_state"), self.flat, self.flat2, self.n, t), "adam_state")
    local m, v = {}, {}
    for i = 1, self.n do m[i], v[i] = self.flat[i - 1], self.flat2[i - 1] end
    return m, v, t[0]
end

--- Wait for the last step and report it: loss (token-weighted over the
--- batch's windows, as LMTrain's batch_loss / batch_tokens), grad_norm
--- (before clipping), applied (false when the norm was not finite and the
--- update was skipped), correct (argmax hits), steps, window_losses.
function Step:stats()
    check(C.lhip_lm_stats(live(self, "stats"), self.st, self.wloss, self.batch), "stats")
    local wl = {}
    for i = 1, self.batch do wl[i] = self.wloss[i - 1] end
    local st = self.st
    return { loss = st.loss, grad_norm = st.grad_norm, applied = st.applied ~= 0, correct = st.correct,
             steps = st.steps, window_losses = wl }
end

--- Row argmax of the last step's logits, 1-based ids, batch*seq of them
--- (the accuracy loop's best_id, lmtrain.lua:1200-1209).
function Step:argmax()
    local n = self.batch * self.seq
    check(C.lhip_lm_get_argmax(live(self, "argmax"), self.ids, n), "argmax")
    local out = {}
    for i = 1, n do out[i] = self.ids[i - 1] + 1 end
    return out
end

--- An lmio v3 checkpoint of the device weights (lmio.lua:226-368):
--- info = { format = "bin" | "text", keep = 1, epoch = 0, loss, best_loss, backend, extra }.
function Step:save(path, info)
    info = info or {}
    local ci = ffi.new("lhip_ckpt_info_t")
    ci.format = info.format == "text" and 1 or 0
    ci.keep = info.keep or 1
    ci.epoch = info.epoch or 0
    ci.loss = info.loss or (0 / 0)
    ci.best_loss = info.best_loss or (0 / 0)
    ci.backend = info.backend        -- info keeps both strings alive through the call
    ci.extra = info.extra
    check(C.lhip_lm_save(live(self, "save"), path, ci), "save")
    return self
end

--- Load a checkpoint (v1-v3, bin or text) into the device weights; returns its header.
function Step:load(path)
    local h = ffi.new("lhip_ckpt_header_t")
    check(C.lhip_lm_load(live(self, "load"), path, h), "load")
    return { version = h.version, format = h.format == 1 and "text" or "bin", dtype_bytes = h.dtype_bytes,
             epoch = h.epoch, loss = h.loss, best_loss = h.best_loss, causal = h.causal, tie = h.tie,
             max_seq = h.max_seq, rope_base = h.rope_base }
end

M.available = true
M.reason = "ready"
M.device = adapter.device
return M
