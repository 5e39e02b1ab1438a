"""lanternl_amd -- MI355X (gfx950) backend for lanternl's ai.Matrix registry.

The product is the C-ABI library ``liblanternl_hip.so`` (HIP kernels under
``csrc/``, ABI in ``include/lanternl_hip.h``).  This package holds its build
script, a ctypes binding and host-side restatements of the reference's Lua
interface for this path:

  build    -- compiles csrc/*.hip for gfx950 into liblanternl_hip.so
  _lib     -- ctypes declarations, status -> exception
  device   -- init/shutdown, device Buffers, event Timer
  kernels  -- wrappers of the device entry points
  backend  -- the `luatl_adapter` module contract (flat-table matmul family)
  matrix   -- ai.Matrix's backend registry and GEMM entry points
  lua/     -- the LuaJIT FFI module that a lanternl checkout loads instead of
              ai/gpu/luatl_adapter.lua

Importing the package does not touch the GPU; ``device.init`` (or importing
``backend``) does.
"""
__version__ = "0.1.0"
