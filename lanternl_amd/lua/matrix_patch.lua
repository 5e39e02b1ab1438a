--  matrix_patch.lua -- the change ai/core/matrix.lua takes so that a backend
--  serves every product, the autograd backward's included.
--
--  matrix.multiply / matmul_nt / matmul_tn offload only calls without `out`
--  (matrix.lua:571), and the backward passes `out = grad_of(x)` with
--  `acc = true` on every product (tensor2.lua:206-211,222-227).  With this
--  patch a call with `out` goes to the backend's matmul_into(op, a, m, k, b,
--  n, rd, acc), which writes the product into rd, or adds it in double with
--  acc; a call without `out` goes to matmul / matmul_nt / matmul_tn as before.
--  A backend without the entry a call needs is skipped, not counted as a
--  failure.  The threshold, `force`, strict checking and failure counting are
--  matrix.lua's own (:19-20, :169-202).
--
--  Two parts.  The helper is a local function of matrix.lua, placed after
--  backend_failed (:169-176); it uses matrix.lua's locals `matrix`,
--  `backends`, `backend_failed` and `sformat`.  The call sites go into the
--  three products where each comment says.

-- [helper]
-- Offload one product.  `fname` is the backend entry for a call without `out`
-- (matmul / matmul_nt / matmul_tn); a call with `out` goes to matmul_into,
-- which writes into result.data.  Returns true when a backend served it.
local INTO_OP = { matmul = "nn", matmul_nt = "nt", matmul_tn = "tn" }
local function try_offload(fname, who, ad, m, k, bd, n, last, result, out, acc)
    local force = matrix.accel.force
    if not matrix.accel.enabled or force == "lua" then return false end
    if force == nil and m * k * n < (matrix.accel.threshold or 0) then return false end
    local entry_name = (out == nil) and fname or "matmul_into"
    for i = 1, #backends do
        local e = backends[i]
        local fn = e.module and e.module[entry_name]
        if e.available and (force == nil or force == e.name) and type(fn) == "function" then
            local ok, res
            if out == nil then
                ok, res = pcall(fn, ad, m, k, bd, n)
            else
                ok, res = pcall(fn, INTO_OP[fname], ad, m, k, bd, n, result.data, acc and true or false)
            end
            local bad = not ok and (tostring(res):match("^[^\n]*"))
            if ok and type(res) ~= "table" then bad = entry_name .. " returned " .. type(res) .. ", expected flat table" end
            if not bad then
                for j = 1, (matrix.strict and last or 0) do
                    if type(res[j]) ~= "number" then bad = sformat("%s result index %d is %s", entry_name, j, type(res[j])) break end
                end
                if not bad and (type(res[1]) ~= "number" or type(res[last]) ~= "number") then
                    bad = sformat("%s returned a malformed result (expected %d numbers)", entry_name, last)
                end
            end
            if bad then
                backend_failed(e, bad)
            else
                matrix.last_backend = e.name
                result.data = res
                return true
            end
        end
    end
    if force ~= nil then
        error(sformat("matrix.%s: backend '%s' was forced via matrix.use() but is unavailable", who, force), 3)
    end
    return false
end

-- [call sites]
-- matrix.multiply: replace the block `if out == nil and not acc and matrix.accel.enabled ...`
-- (matrix.lua:571-590) by
    if try_offload("matmul", "multiply", ad, m, k, bd, n, m * n, result, out, acc) then return result end

-- matrix.matmul_nt: after `if m == 0 or n == 0 then return result end`
    if k > 0 and try_offload("matmul_nt", "matmul_nt", a.data, m, k, b.data, n, m * n, result, out, acc) then
        return result
    end

-- matrix.matmul_tn: after `if m == 0 or k == 0 or n == 0 then return result end`
    if try_offload("matmul_tn", "matmul_tn", a.data, m, k, b.data, n, k * n, result, out, acc) then
        return result
    end
