"""ctypes binding of ``libadafactor8bit_amd.so`` (the HIP C ABI).

The library is built in-tree by ``adafactor-8bit_amd/build.py`` for gfx950 and
declared in ``include/adafactor8bit_amd.h``.  There is no fallback: every
optimizer step runs through this library, and a missing or unloadable library
raises immediately.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libadafactor8bit_amd.so")

F32, BF16, F16, F64 = 0, 1, 2, 3
MODE_NOCLIP, MODE_NORM, MODE_APPLY, MODE_LAG, MODE_MNORM = 0, 1, 2, 3, 4
AL_KERNEL_RULE = 0x100   # A8_AL_KERNEL_RULE: OR'd into v_bits of the 1-D quantised steps

_c_vp = ctypes.c_void_p
_c_i = ctypes.c_int
_c_i64 = ctypes.c_int64
_c_u64 = ctypes.c_uint64
_c_f = ctypes.c_float
_c_d = ctypes.c_double


class StepSpec(ctypes.Structure):
    """Mirror of ``a8_step_spec``."""
    _fields_ = [("beta1", _c_d), ("beta2", _c_d), ("beta2_decay", _c_d), ("eps1", _c_d), ("lr", _c_d),
                ("wd", _c_f), ("v_mode", _c_i), ("relative_step", _c_i), ("bias_mode", _c_i), ("adam_denom", _c_i),
                ("wd_mode", _c_i), ("fact_bias_mode", _c_i), ("apollo_bias_mode", _c_i), ("lr_dev", _c_vp)]


STEP_SCALARS_BYTES = 40   # sizeof(a8_step_scalars)


class Tensor1D(ctypes.Structure):
    """Mirror of ``a8_tensor1d``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("m_q", _c_vp), ("m_scale", _c_vp),
                ("v_q", _c_vp), ("v_scale", _c_vp), ("v_min_log", _c_vp), ("v_buf", _c_vp),
                ("norm_buf", _c_vp), ("alpha", _c_vp), ("prev_norm", _c_vp), ("decay", _c_vp),
                ("numel", _c_i64), ("sr_seed", _c_u64), ("fira_scale", _c_vp), ("norm_parts", _c_vp)]


class TensorFull(ctypes.Structure):
    """Mirror of ``a8_tensor_full``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("variance", _c_vp), ("m", _c_vp),
                ("norm_buf", _c_vp), ("alpha", _c_vp), ("prev_norm", _c_vp), ("decay", _c_vp),
                ("numel", _c_i64), ("sr_seed", _c_u64), ("psq", _c_vp), ("fira_scale", _c_vp),
                ("norm_parts", _c_vp)]


class TensorSgd(ctypes.Structure):
    """Mirror of ``a8_tensor_sgd``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("m_q", _c_vp), ("m_scale", _c_vp), ("m", _c_vp),
                ("norm_buf", _c_vp), ("fira", _c_vp), ("alpha", _c_vp), ("decay", _c_vp),
                ("numel", _c_i64), ("sr_seed", _c_u64), ("norm_parts", _c_vp), ("fira_sum", _c_vp)]


class FactoredPrimArgs(ctypes.Structure):
    """Mirror of ``a8_factored_prim_args``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("m_q", _c_vp), ("m_scale", _c_vp), ("m", _c_vp),
                ("row", _c_vp), ("col", _c_vp), ("row_mean", _c_vp), ("conf_row", _c_vp), ("conf_col", _c_vp),
                ("conf_row_mean", _c_vp), ("row_sum", _c_vp), ("col_sum", _c_vp), ("norm_buf", _c_vp),
                ("alpha", _c_vp), ("prev_norm", _c_vp), ("decay", _c_vp), ("clip", _c_vp), ("rows", _c_i64),
                ("cols", _c_i64), ("numel", _c_i64), ("beta1", _c_d), ("eps_came", _c_f), ("d", _c_f),
                ("m_bits", _c_i), ("m_mode", _c_i), ("m_block_size", _c_i), ("sr_seed", _c_u64),
                ("sr_step", _c_u64)]


class Tensor2D(ctypes.Structure):
    """Mirror of ``a8_tensor2d``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("m_q", _c_vp), ("m_scale", _c_vp),
                ("row_q", _c_vp), ("row_scale", _c_vp), ("row_min_log", _c_vp), ("row_var", _c_vp),
                ("col_q", _c_vp), ("col_scale", _c_vp), ("col_min_log", _c_vp), ("col_var", _c_vp),
                ("conf_row_q", _c_vp), ("conf_row_scale", _c_vp), ("conf_row_min_log", _c_vp),
                ("conf_row", _c_vp), ("conf_col_q", _c_vp), ("conf_col_scale", _c_vp),
                ("conf_col_min_log", _c_vp), ("conf_col", _c_vp), ("workspace", _c_vp),
                ("lr", _c_vp), ("fira_prev_norm", _c_vp), ("has_fira_prev", _c_i),
                ("batch", _c_i64), ("rows", _c_i64), ("cols", _c_i64), ("sr_seed", _c_u64), ("m", _c_vp)]


class ApolloTensor(ctypes.Structure):
    """Mirror of ``a8_apollo_tensor``."""
    _fields_ = [("param", _c_vp), ("grad", _c_vp), ("rows", _c_i64), ("cols", _c_i64),
                ("proj_t", _c_vp), ("rank", _c_i64), ("v_q", _c_vp), ("v_scale", _c_vp),
                ("v_min_log", _c_vp), ("v_fp32", _c_vp), ("m_q", _c_vp), ("m_scale", _c_vp),
                ("m_fp32", _c_vp), ("fira_prev", _c_vp), ("has_fira_prev", _c_i), ("lr", _c_vp),
                ("workspace", _c_vp), ("sr_seed", _c_u64), ("first_step", _c_i), ("proj_fresh", _c_i),
                ("step", _c_u64), ("bias_factor", _c_f), ("proj_state", _c_vp), ("proj_gap", _c_i)]


class ApolloXArgs(ctypes.Structure):
    """Mirror of ``a8_apollo_x_args``."""
    _fields_ = [("g_low", _c_vp), ("u", _c_vp), ("xws", _c_vp), ("rows_low", _c_i64), ("cols_low", _c_i64),
                ("factorize", _c_i), ("came", _c_i), ("has_m", _c_i), ("first_step", _c_i),
                ("v_q", _c_vp), ("v_scale", _c_vp), ("v_min_log", _c_vp), ("v_fp32", _c_vp), ("v_bits", _c_i),
                ("block_size", _c_i), ("row_var", _c_vp), ("col_var", _c_vp),
                ("m_q", _c_vp), ("m_scale", _c_vp), ("m_fp32", _c_vp), ("m_bits", _c_i), ("m_mode", _c_i),
                ("m_block_size", _c_i),
                ("res_q", _c_vp), ("res_scale", _c_vp), ("res_min_log", _c_vp), ("res_fp32", _c_vp),
                ("crow_q", _c_vp), ("crow_scale", _c_vp), ("crow_min_log", _c_vp), ("crow_fp32", _c_vp),
                ("ccol_q", _c_vp), ("ccol_scale", _c_vp), ("ccol_min_log", _c_vp), ("ccol_fp32", _c_vp),
                ("c_bits", _c_i), ("beta_v", _c_d), ("beta1", _c_d), ("beta3", _c_d),
                ("apollo_eps", _c_f), ("eps_sq", _c_f), ("log_floor", _c_f), ("eps_came", _c_f), ("d", _c_f),
                ("u_rowsums", _c_i)]


_SIGS = {
    "a8_last_error": (ctypes.c_char_p, []),
    "a8_version": (ctypes.c_char_p, []),
    "a8_set_qmap": (_c_i, [_c_vp, _c_vp]),
    "a8_fused_update_1d": (_c_i, [_c_i, _c_i, _c_i, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                  _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_u64, _c_u64, _c_d, _c_d,
                                  _c_f, _c_i, _c_f, _c_f, _c_f, _c_i64, _c_i, _c_i, _c_i, _c_i,
                                  _c_f, _c_i, _c_i, _c_f, _c_f, _c_i, _c_vp]),
    "a8_fused_update_1d_multi": (_c_i, [_c_i, _c_i, _c_i, ctypes.POINTER(Tensor1D), _c_i, _c_vp,
                                        _c_i64, _c_d, _c_d, _c_f, _c_i, _c_f, _c_f, _c_f, _c_i, _c_i,
                                        _c_i, _c_i, _c_f, _c_i, _c_i, _c_u64, _c_f, _c_f, _c_i, _c_i,
                                        _c_vp, _c_vp]),
    "a8_fused_update_1d_multi_noalloc": (_c_i, [_c_i, _c_i, _c_i, ctypes.POINTER(Tensor1D), _c_i, _c_d, _c_d,
                                                _c_f, _c_i, _c_f, _c_f, _c_f, _c_i, _c_i, _c_i, _c_i, _c_f,
                                                _c_i, _c_i, _c_u64, _c_f, _c_f, _c_i, _c_i, _c_vp, _c_vp]),
    "a8_noalloc_max_tensors_1d": (_c_i, []),
    "a8_step_advance": (_c_i, [ctypes.POINTER(StepSpec), _c_vp, _c_vp, _c_vp]),
    "a8_table_bytes_1d": (_c_i64, [_c_i]),
    "a8_norm_parts_1d": (_c_i64, [_c_i64, _c_i, _c_i]),
    "a8_norm_parts_full": (_c_i64, [_c_i64]),
    "a8_norm_parts_sgd": (_c_i64, [_c_i64, _c_i]),
    "a8_fused_update_1d_full": (_c_i, [_c_i, _c_i, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                                       _c_vp, _c_vp, _c_d, _c_d, _c_f, _c_f, _c_i, _c_f, _c_i64, _c_f, _c_i,
                                       _c_f, _c_f, _c_i, _c_i, _c_u64, _c_u64, _c_i, _c_vp]),
    "a8_fused_update_1d_full_multi": (_c_i, [_c_i, _c_i, ctypes.POINTER(TensorFull), _c_i, _c_vp,
                                             _c_i64, _c_d, _c_d, _c_f, _c_f, _c_i, _c_f, _c_f, _c_i,
                                             _c_f, _c_f, _c_i, _c_i, _c_u64, _c_i, _c_f, _c_i, _c_f,
                                             _c_i, _c_i, _c_vp, _c_vp]),
    "a8_table_bytes_full": (_c_i64, [_c_i]),
    "a8_fira_scalar": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i, _c_i, _c_f, _c_vp]),
    "a8_factored_step": (_c_i, [_c_i, _c_i, ctypes.POINTER(Tensor2D), _c_i, _c_vp, _c_i64, _c_i, _c_d,
                                _c_f, _c_f, _c_f, _c_i, _c_i, _c_f, _c_f, _c_i, _c_f, _c_i, _c_f, _c_f,
                                _c_i, _c_i, _c_d, _c_i, _c_i, _c_i, _c_u64, _c_i, _c_d, _c_f, _c_i,
                                _c_vp, _c_vp]),
    "a8_factored_workspace_floats": (_c_i64, [_c_i64, _c_i64, _c_i64]),
    "a8_table_bytes_2d": (_c_i64, [_c_i]),
    "a8_apollo_step": (_c_i, [_c_i, _c_i, ctypes.POINTER(ApolloTensor), _c_i, _c_i, _c_d, _c_d, _c_i, _c_f,
                              _c_f, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_i, _c_i, _c_f, _c_f,
                              _c_f, _c_f, _c_i, _c_i, _c_f, _c_f, _c_i, _c_u64, _c_vp]),
    "a8_apollo_workspace_floats": (_c_i64, [_c_i64, _c_i64, _c_i64, _c_i]),
    "a8_apollo_step_multi": (_c_i, [_c_i, _c_i, ctypes.POINTER(ApolloTensor), _c_i, _c_vp, _c_i64, _c_d, _c_d,
                                    _c_i, _c_f, _c_f, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i, _c_f, _c_i, _c_i,
                                    _c_f, _c_f, _c_f, _c_f, _c_i, _c_i, _c_f, _c_i, _c_i, _c_vp, _c_vp]),
    "a8_apollo_proj_gen": (_c_i, [_c_vp, _c_i64, _c_i64, _c_i64, _c_u64, _c_vp]),
    "a8_apollo_next_seed": (_c_i, [_c_vp, _c_vp, _c_i64, _c_vp]),
    "a8_apollo_table_bytes": (_c_i64, [_c_i]),
    "a8_apollo_step_multi_phase": (_c_i, [_c_i, _c_i, _c_i, ctypes.POINTER(ApolloTensor), _c_i, _c_vp, _c_i64,
                                          _c_d, _c_d, _c_i, _c_f, _c_f, _c_i, _c_i, _c_i, _c_i, _c_i, _c_i,
                                          _c_i, _c_f, _c_i, _c_i, _c_f, _c_f, _c_f, _c_f, _c_i, _c_i, _c_f,
                                          _c_i, _c_i, _c_vp, _c_vp]),
    "a8_apollo_lowrank_x": (_c_i, [ctypes.POINTER(ApolloXArgs), _c_vp]),
    "a8_vema_fp32": (_c_i, [_c_vp, _c_vp, _c_i, _c_d, _c_f, _c_i64, _c_vp]),
    "a8_apollo_x_workspace_floats": (_c_i64, [_c_i64, _c_i64]),
    "a8_apollo_lowrank_x_multi": (_c_i, [ctypes.POINTER(ApolloXArgs), _c_i, _c_vp, _c_i64, _c_i, _c_vp, _c_vp]),
    "a8_apollo_x_table_bytes": (_c_i64, [_c_i]),
    "a8_dequantize_log_nonneg": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i, _c_i, _c_vp]),
    "a8_dequantize_dynamic": (_c_i, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i, _c_i, _c_vp]),
    "a8_dequantize_momentum": (_c_i, [_c_vp, _c_vp, _c_vp, _c_i64, _c_i, _c_i, _c_i, _c_vp]),
    "a8_al_encode": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i, _c_i, _c_f, _c_vp]),
    "a8_sgd_step": (_c_i, [_c_i, _c_i, _c_i, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp,
                           _c_vp, _c_i64, _c_d, _c_i, _c_i, _c_i, _c_f, _c_f, _c_f, _c_i, _c_u64, _c_u64, _c_vp]),
    "a8_sgd_step_multi": (_c_i, [_c_i, _c_i, _c_i, ctypes.POINTER(TensorSgd), _c_i, _c_vp, _c_i64, _c_d, _c_i,
                                 _c_i, _c_i, _c_i, _c_f, _c_f, _c_f, _c_i, _c_u64, _c_i, _c_vp, _c_vp]),
    "a8_table_bytes_sgd": (_c_i64, [_c_i]),
    "a8_m_quantize_lerp": (_c_i, [_c_vp, _c_vp, _c_vp, _c_i, _c_vp, _c_d, _c_i, _c_i64, _c_i, _c_i, _c_vp]),
    "a8_log_quantize_lerp": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_i, _c_vp, _c_d, _c_i, _c_i, _c_f, _c_i64, _c_f,
                                    _c_i, _c_vp]),
    "a8_factored_prim": (_c_i, [_c_i, _c_i, _c_i, ctypes.POINTER(FactoredPrimArgs), _c_vp]),
    "a8_apollo_norms": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_f,
                               _c_i, _c_vp]),
    "a8_apollo_came_rms": (_c_i, [_c_vp, _c_vp, _c_vp, _c_f, _c_i64, _c_vp]),
    "a8_apollo_came_m_res": (_c_i, [_c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_d, _c_d, _c_f, _c_f,
                                    _c_i, _c_i64, _c_i, _c_i, _c_vp]),
    "a8_apollo_writeback": (_c_i, [_c_i, _c_i, _c_i, _c_vp, _c_vp, _c_vp, _c_vp, _c_vp, _c_i, _c_i, _c_i, _c_u64,
                                   _c_u64, _c_i64, _c_i64, _c_vp]),
}

_LIB = None


def lib():
    """Load the library once; raise if it is missing (no CPU fallback exists)."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"adafactor8bit: HIP library not found at {LIB_PATH}; build it with "
                "`python adafactor-8bit_amd/build.py` (there is no CPU fallback)")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def check(rc: int, what: str = ""):
    if rc != 0:
        msg = lib().a8_last_error().decode(errors="replace")
        raise RuntimeError(f"adafactor8bit HIP call {what} failed ({rc}): {msg}")


def ptr(t):
    """Device address of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_of(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dt) -> int:
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    if dt == torch.float16:
        return F16
    if dt == torch.float64:
        return F64
    raise TypeError(f"adafactor8bit: unsupported parameter dtype {dt}")


_ROCTX = None


def roctx():
    """The ROCm tracing-marker library (rocprofiler-sdk roctx), or False when the
    runtime has none: optimizer steps push named ranges onto it, which
    ``rocprofv3 --marker-trace`` records around each step's kernels."""
    global _ROCTX
    if _ROCTX is None:
        _ROCTX = False
        for name in ("librocprofiler-sdk-roctx.so.1", "librocprofiler-sdk-roctx.so", "/opt/rocm/lib/librocprofiler-sdk-roctx.so"):
            try:
                r = ctypes.CDLL(name)
                r.roctxRangePushA.argtypes = [ctypes.c_char_p]
                r.roctxRangePushA.restype = ctypes.c_int
                r.roctxRangePop.argtypes = []
                r.roctxRangePop.restype = ctypes.c_int
                _ROCTX = r
                break
            except (OSError, AttributeError):
                continue
    return _ROCTX


class range_marker:
    """``with range_marker(b"name"):`` -- a roctx range (no-op without roctx)."""
    __slots__ = ("msg",)

    def __init__(self, msg: bytes):
        self.msg = msg

    def __enter__(self):
        r = roctx()
        if r:
            r.roctxRangePushA(self.msg)
        return self

    def __exit__(self, *exc):
        r = roctx()
        if r:
            r.roctxRangePop()
        return False


def exported_symbols():
    return sorted(_SIGS)
