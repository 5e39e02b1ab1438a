"""ctypes binding of liblanternl_hip.so (the C ABI declared in include/lanternl_hip.h).

There is no fallback: if the library is missing or the GPU cannot be
initialised, every call raises.  Status codes become ``LanternlHipError`` with
the library's last-error text, the way the reference's Lua ``ck()`` turns a
luaTL status into a Lua error (ai/gpu/luaTL.lua:240-246).
"""
import ctypes
import os

from .build import LIB_PATH

STATUS = {
    0: "OK", -1: "NULL", -2: "SHAPE", -3: "DTYPE", -4: "DEVICE",
    -5: "OOM", -6: "ARG", -7: "CAPACITY", -8: "UNSUPPORTED",
}


class LanternlHipError(RuntimeError):
    def __init__(self, what, code, msg):
        self.code = code
        super().__init__(f"lanternl_hip[{what}]: {msg} ({STATUS.get(code, code)})")


class DevInfo(ctypes.Structure):
    """lhip_devinfo_t"""
    _fields_ = [
        ("name", ctypes.c_char * 256), ("arch", ctypes.c_char * 64), ("device", ctypes.c_int),
        ("compute_units", ctypes.c_int), ("clock_khz", ctypes.c_int), ("wavefront_size", ctypes.c_int),
        ("total_mem", ctypes.c_longlong), ("lds_per_block", ctypes.c_longlong), ("l2_bytes", ctypes.c_int),
        ("peak_fp32_matrix_tflops", ctypes.c_double), ("peak_hbm_gbps", ctypes.c_double),
    ]


class MemStats(ctypes.Structure):
    """lhip_mem_stats_t"""
    _fields_ = [(n, ctypes.c_ulonglong) for n in ("bytes_in_use", "peak_in_use", "live_buffers", "n_alloc",
                                                  "n_free", "workspace_bytes", "staging_bytes")]


_i, _f, _d, _ll, _sz = ctypes.c_int, ctypes.c_float, ctypes.c_double, ctypes.c_longlong, ctypes.c_size_t
_p = ctypes.c_void_p
_pp = ctypes.POINTER(ctypes.c_void_p)

# name -> (restype, argtypes); every function of include/lanternl_hip.h.
SIGNATURES = {
    "lhip_init": (_i, [_i]),
    "lhip_shutdown": (_i, []),
    "lhip_is_ready": (_i, []),
    "lhip_last_error": (ctypes.c_char_p, []),
    "lhip_clear_error": (None, []),
    "lhip_device_info": (_i, [ctypes.POINTER(DevInfo)]),
    "lhip_version": (ctypes.c_char_p, []),
    "lhip_malloc": (_i, [_pp, _sz]),
    "lhip_free": (_i, [_p]),
    "lhip_mem_info": (_i, [ctypes.POINTER(ctypes.c_ulonglong), ctypes.POINTER(ctypes.c_ulonglong)]),
    "lhip_mem_stats": (_i, [ctypes.POINTER(MemStats)]),
    "lhip_upload": (_i, [_p, _p, _sz]),
    "lhip_download": (_i, [_p, _p, _sz]),
    "lhip_copy": (_i, [_p, _p, _sz]),
    "lhip_zero": (_i, [_p, _sz]),
    "lhip_sync": (_i, []),
    "lhip_stream": (_p, []),
    "lhip_event_create": (_i, [_pp]),
    "lhip_event_destroy": (_i, [_p]),
    "lhip_event_record": (_i, [_p]),
    "lhip_event_elapsed_ms": (_i, [_p, _p, ctypes.POINTER(_f)]),
    "lhip_program_begin": (_i, []),
    "lhip_program_end": (_i, [_pp]),
    "lhip_program_replay": (_i, [_p, _i]),
    "lhip_program_free": (_i, [_p]),
    "lhip_is_recording": (_i, []),
    "lhip_ktimer_start": (_i, [_i]),
    "lhip_ktimer_stop": (_i, [ctypes.POINTER(_f), _i, ctypes.POINTER(_i)]),
    "lhip_sgemm": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i]),
    "lhip_sgemm_strided_batched": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _ll, _p, _i, _ll, _f,
                                        _p, _i, _ll, _i]),
    "lhip_sgemm_batched_reduce": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _ll, _p, _i, _ll, _f, _p, _i, _i]),
    "lhip_sgemm_noalloc": (_i, [_i, _i, _i, _i, _i, _f, _p, _i, _p, _i, _f, _p, _i]),
    "lhip_matmul_host": (_i, [_i, _p, _p, _p, _i, _i, _i, _i]),
    "lhip_set_host_spin": (_i, [_i, ctypes.POINTER(_i)]),
    "lhip_rmsnorm_fwd": (_i, [_p, _p, _p, _p, _i, _i, _f]),
    "lhip_rmsnorm_bwd": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i]),
    "lhip_softmax_fwd": (_i, [_p, _p, _i, _i, _f, _i, _i, _i]),
    "lhip_softmax_bwd": (_i, [_p, _p, _p, _i, _i, _f, _i, _i, _i, _i]),
    "lhip_swiglu_fwd": (_i, [_p, _i, _p, _i, _p, _i, _i, _i]),
    "lhip_swiglu_bwd": (_i, [_p, _i, _p, _i, _p, _i, _p, _i, _p, _i, _i, _i, _i]),
    "lhip_rope": (_i, [_p, _p, _i, _i, _i, _i, _i, _i, _d, _i, _i]),
    "lhip_ce_fused": (_i, [_p, _p, _p, _p, _i, _i, _i, _f]),
    "lhip_argmax_rows": (_i, [_p, _p, _i, _i]),
    "lhip_embed_fwd": (_i, [_p, _p, _p, _i, _i, _i]),
    "lhip_embed_bwd": (_i, [_p, _p, _p, _i, _i, _i, _f, _i]),
    "lhip_fill": (_i, [_p, _ll, _f]),
    "lhip_add": (_i, [_p, _p, _p, _ll]),
    "lhip_silu": (_i, [_p, _p, _ll]),
    "lhip_sumsq": (_i, [_p, _ll, _p]),
    "lhip_sum": (_i, [_p, _i, _f, _p]),
    "lhip_sgd_step": (_i, [_p, _p, _p, _ll, _p, _f, _f, _f, _f, _f, _i, _p, _p]),
    "lhip_adamw_step": (_i, [_p, _p, _p, _p, _ll, _p, _f, _f, _f, _f, _f, _f, _f, _i, _p, _p]),
    # the luaTL operation set
    "lhip_gemm_ex": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _ll, _ll, _ll, _ll, _ll, _ll, _ll, _ll, _ll,
                          _i, _f, _f, _f, _i, _i]),
    "lhip_elementwise": (_i, [_p, _p, _p, _ll, _i, _f, _f]),
    "lhip_rmsnorm_ex": (_i, [_p, _p, _p, _i, _i, _f]),
    "lhip_rmsnorm_bwd_ex": (_i, [_p, _p, _p, _p, _p, _i, _i, _f]),
    "lhip_row_rms": (_i, [_p, _p, _i, _i, _ll, _ll, _f]),
    "lhip_softmax_ex": (_i, [_p, _p, _p, _i, _i, _f, _i, _i, _i]),
    "lhip_softmax_bwd_ex": (_i, [_p, _p, _p, _i, _i, _f, _i, _i, _i]),
    "lhip_swiglu_bwd_ex": (_i, [_p, _p, _p, _p, _p, _i, _i, _i, _i, _i]),
    "lhip_reduce_cols": (_i, [_p, _p, _i, _i, _ll, _f, _f]),
    "lhip_l2_accum": (_i, [_p, _ll, _p]),
    "lhip_clip_by_nsq": (_i, [_p, _ll, _p, _f]),
    "lhip_sum_accum": (_i, [_p, _ll, _f, _p]),
    "lhip_transpose": (_i, [_p, _p, _i, _i]),
    "lhip_bcast_add": (_i, [_p, _p, _p, _i, _i, _f]),
    "lhip_adamw_elementwise": (_i, [_p, _p, _p, _p, _p, _ll, _i, _f, _f, _f, _f, _f, _f]),
}

class LmConfig(ctypes.Structure):
    """lhip_lm_config_t"""
    _fields_ = [("vocab", ctypes.c_int), ("dim", ctypes.c_int), ("layers", ctypes.c_int),
                ("heads", ctypes.c_int), ("ffn", ctypes.c_int), ("causal", ctypes.c_int),
                ("eps", ctypes.c_double), ("rope_base", ctypes.c_double),
                ("batch", ctypes.c_int), ("seq", ctypes.c_int)]


class LmStats(ctypes.Structure):
    """lhip_lm_stats_t"""
    _fields_ = [("loss", ctypes.c_float), ("grad_norm", ctypes.c_float), ("applied", ctypes.c_int),
                ("correct", ctypes.c_int), ("steps", ctypes.c_int)]


class CkptInfo(ctypes.Structure):
    """lhip_ckpt_info_t"""
    _fields_ = [("format", ctypes.c_int), ("keep", ctypes.c_int), ("epoch", ctypes.c_int),
                ("loss", ctypes.c_double), ("best_loss", ctypes.c_double),
                ("backend", ctypes.c_char_p), ("extra", ctypes.c_char_p)]


class CkptHeader(ctypes.Structure):
    """lhip_ckpt_header_t"""
    _fields_ = [("version", ctypes.c_int), ("format", ctypes.c_int), ("dtype_bytes", ctypes.c_int),
                ("epoch", ctypes.c_int), ("loss", ctypes.c_double), ("best_loss", ctypes.c_double),
                ("causal", ctypes.c_int), ("tie", ctypes.c_int), ("max_seq", ctypes.c_int),
                ("rope_base", ctypes.c_double)]


_cfgp = ctypes.POINTER(LmConfig)
SIGNATURES.update({
    "lhip_lm_num_params": (_ll, [_cfgp]),
    "lhip_lm_param_offsets": (_i, [_cfgp, _p, _p, _p]),
    "lhip_lm_create": (_i, [_cfgp, _pp]),
    "lhip_lm_destroy": (_i, [_p]),
    "lhip_lm_set_params": (_i, [_p, _p, _ll]),
    "lhip_lm_get_params": (_i, [_p, _p, _ll]),
    "lhip_lm_get_grads": (_i, [_p, _p, _ll]),
    "lhip_lm_set_velocity": (_i, [_p, _p, _ll]),
    "lhip_lm_get_velocity": (_i, [_p, _p, _ll]),
    "lhip_lm_set_batch": (_i, [_p, _p, _p]),
    "lhip_lm_set_batch_ex": (_i, [_p, _p, _p, _p, _i]),
    "lhip_lm_use_graph": (_i, [_p, _i]),
    "lhip_lm_step_sgd": (_i, [_p, _f, _f, _f, _f, _i]),
    "lhip_lm_step_adamw": (_i, [_p, _f, _f, _f, _f, _f, _f]),
    "lhip_lm_set_adam_state": (_i, [_p, _p, _p, _ll, _i]),
    "lhip_lm_get_adam_state": (_i, [_p, _p, _p, _ll, _p]),
    "lhip_lm_stats": (_i, [_p, ctypes.POINTER(LmStats), _p, _i]),
    "lhip_lm_get_argmax": (_i, [_p, _p, _i]),
    "lhip_ckpt_save_host": (_i, [ctypes.c_char_p, _cfgp, ctypes.POINTER(CkptInfo), _p, _ll]),
    "lhip_ckpt_load_host": (_i, [ctypes.c_char_p, _cfgp, _p, _ll, ctypes.POINTER(CkptHeader)]),
    "lhip_lm_save": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(CkptInfo)]),
    "lhip_lm_load": (_i, [_p, ctypes.c_char_p, ctypes.POINTER(CkptHeader)]),
})

_lib = None


def lib():
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python -m lanternl_amd.build` "
                               "(or __graft_entry__.build()); there is no CPU fallback")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error():
    msg = lib().lhip_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc, what):
    if rc != 0:
        raise LanternlHipError(what, rc, last_error())
    return rc


def call(name, *args):
    """Call `name` and raise LanternlHipError on a non-zero status."""
    return check(getattr(lib(), name)(*args), name)
