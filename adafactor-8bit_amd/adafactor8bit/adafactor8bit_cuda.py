"""Drop-in for the reference's compiled module ``adafactor8bit_cuda``.

The reference JIT-builds ``adafactor8bit/kernels.cu`` into a pybind11 module of
that name (optimizer.py:85-98; bindings kernels.cu:3089-3150) and calls it as
``_CUDA_MODULE.<name>(...)``.  This module exposes the same names with the same
positional signatures, converts tensors to device pointers and launches the
HIP kernels of ``libadafactor8bit_amd.so`` on the current stream.

Numerics follow the reference's PyTorch path (optimizer.py:299-353, 504-532) by
default: the AL floor of the 1-D kernels is the CPU quantiser's -126, so the
``log_eps_sq`` argument only supplies eps1 for the Adam denominator's momentum clamp.
``set_refit_rule("kernel")`` switches the fused 1-D functions (fused_update_1d_*,
fused_update_1d_vonly_*) to the refit rule of the reference's own CUDA kernels
(kernels.cu:686-687, 772-791): the block minimum includes zeros and is floored at
``log_eps_sq``, l_max is capped at 126 (A8_AL_KERNEL_RULE).

Every one of the reference module's 61 functions is provided.
"""
import torch

from . import _native as nat
from ._state import dynamic_map

__all__ = [
    "set_qmap", "fira_scalar",
    "fused_update_1d_noclip", "fused_update_1d_norm", "fused_update_1d_apply", "fused_update_1d_lag",
    "fused_update_1d_noclip_sr", "fused_update_1d_apply_sr", "fused_update_1d_lag_sr",
    "fused_update_1d_vonly_noclip", "fused_update_1d_vonly_norm", "fused_update_1d_vonly_apply",
    "fused_update_1d_vonly_lag", "fused_update_1d_vonly_noclip_sr", "fused_update_1d_vonly_apply_sr",
    "fused_update_1d_vonly_lag_sr",
    "fused_update_1d_full_noclip", "fused_update_1d_full_norm", "fused_update_1d_full_apply",
    "fused_update_1d_full_lag", "fused_update_1d_full_noclip_sr", "fused_update_1d_full_apply_sr",
    "fused_update_1d_full_lag_sr",
    "fused_m_quantize_lerp", "dequantize_log_nonneg", "dequantize_dynamic",
    "fused_log_quantize_lerp",
    "fused_update_2d_noclip", "fused_update_2d_norm", "fused_update_2d_apply", "fused_update_2d_lag",
    "fused_update_2d_noclip_sr", "fused_update_2d_apply_sr", "fused_update_2d_lag_sr",
    "fused_update_2d_full_noclip", "fused_update_2d_full_norm", "fused_update_2d_full_apply",
    "fused_update_2d_full_lag", "fused_update_2d_full_noclip_sr", "fused_update_2d_full_apply_sr",
    "fused_update_2d_full_lag_sr", "compute_factored_sums", "compute_ut_rms",
    "fused_came_pass1", "fused_came_pass2_norm", "fused_came_pass2", "fused_came_pass2_sr",
    "fused_came_full_pass1", "fused_came_full_pass2", "fused_came_full_pass2_sr",
    "compute_apollo_norms", "compute_apollo_came_rms", "apollo_came_compute_m_res",
    "apollo_came_compute_update_norms", "apollo_apply_bf16_det", "apollo_apply_bf16_sr", "apollo_apply_fp16_sr",
    "apollo_apply_bf16_det_native", "apollo_apply_fp16_det_native", "apollo_apply_bf16_sr_native",
    "apollo_apply_fp16_sr_native",
]

_AL_FLOOR = -126.0
_EPS_FLOOR = 1.17549435e-38
_RULE = {"kernel": False}


def set_refit_rule(rule):
    """The V refit rule of the fused 1-D functions: "fallback" (the reference's CPU
    quantiser, optimizer.py:299-325; the default) or "kernel" (the reference's fused
    CUDA kernels, kernels.cu:686-687, 772-791, whose floor is the log_eps_sq argument).
    Process-wide for this module; the optimizer's own switch is al_refit_rule."""
    if rule not in ("fallback", "kernel"):
        raise ValueError(f"refit rule must be 'fallback' or 'kernel', got {rule!r}")
    _RULE["kernel"] = rule == "kernel"


def refit_rule():
    return "kernel" if _RULE["kernel"] else "fallback"


def _stream(t):
    return nat.stream_of(t.device)


def _vbits_check(v_q, v_bits):
    want = torch.uint8 if v_bits == 8 else torch.int16
    if v_q.dtype != want:
        raise RuntimeError(f"v_bits={v_bits} requires v_q to be {want}")


def set_qmap(qmap_8, qmap_4):
    """kernels.cu:32-37: upload the 256/16-entry dynamic codebooks."""
    q8 = qmap_8.detach().to("cpu", torch.float32).contiguous()
    q4 = qmap_4.detach().to("cpu", torch.float32).contiguous()
    if q8.numel() != 256 or q4.numel() != 16:
        raise RuntimeError("set_qmap expects 256 and 16 fp32 entries")
    with torch.cuda.device(qmap_8.device):
        nat.check(nat.lib().a8_set_qmap(q8.data_ptr(), q4.data_ptr()), "set_qmap")


def _parts(device, n):
    """Workspace for a norm pass's per-workgroup partial sums (the library adds them
    in a fixed order, where the reference adds into norm_buf with float atomics)."""
    return torch.empty(max(int(n), 1), dtype=torch.float64, device=device)


def _u1d(mode, sr, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha,
         prev_norm, decay, sr_seed, sr_step, beta1, beta_val, eps_for_denom, use_adam_denom,
         log_eps_sq, eps_for_grad_sq, numel, block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only):
    _vbits_check(v_q, v_bits)
    ref = grad
    if sr and (param is None or param.dtype not in (torch.bfloat16, torch.float16)
               or grad.dtype != param.dtype):
        raise RuntimeError("SR writeback requires matching FP16/BF16 param and grad")
    dec = decay if (decay is not None and decay.numel()) else None
    # optimizer.py:1961-1967: eps_sq = max(eps1^2, floor); eps1 is eps_for_grad_sq on the
    # non-Adam denominator, and only recoverable from log_eps_sq on the Adam one (where the
    # clamp is used by momentum-only clipping alone).
    if use_adam_denom:
        eps_sq = max(2.0 ** float(log_eps_sq), _EPS_FLOOR)
    else:
        eps_sq = max(float(eps_for_grad_sq) ** 2, _EPS_FLOOR)
    parts = None
    if mode in (1, 3):
        parts = _parts(ref.device, nat.lib().a8_norm_parts_1d(int(numel), int(block_size), int(m_block_size)))
    rc = nat.lib().a8_fused_update_1d(
        mode, int(sr), nat.dtype_code(ref.dtype), nat.ptr(param), nat.ptr(grad), nat.ptr(m_q),
        nat.ptr(m_scale), nat.ptr(v_q), nat.ptr(v_scale), nat.ptr(v_min_log), nat.ptr(v_buf),
        nat.ptr(norm_buf), nat.ptr(parts), nat.ptr(alpha), nat.ptr(prev_norm), nat.ptr(dec), int(sr_seed), int(sr_step),
        float(beta1), float(beta_val), float(eps_for_denom), int(bool(use_adam_denom)),
        float(log_eps_sq) if _RULE["kernel"] else _AL_FLOOR,
        float(eps_for_grad_sq), eps_sq, int(numel),
        int(block_size), int(m_block_size), int(m_bits), int(m_mode), float(d),
        int(v_bits) | (nat.AL_KERNEL_RULE if _RULE["kernel"] else 0),
        int(bool(momentum_only)), 0.0, 1.0, 0, _stream(ref))
    nat.check(rc, "fused_update_1d")


# ---- fused_update_1d_* (kernels.cu:826-990)
def fused_update_1d_noclip(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, alpha, beta1, beta_val,
                           eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
                           block_size, m_block_size, m_bits, m_mode, v_bits, momentum_only):
    _u1d(0, False, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, None, None, alpha, None, None,
         0, 0, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         m_block_size, m_bits, m_mode, 0.0, v_bits, momentum_only)


def fused_update_1d_norm(grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, beta1, beta_val,
                         eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
                         m_block_size, m_bits, m_mode, v_bits, momentum_only):
    _u1d(1, False, None, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, None, None, None,
         0, 0, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         m_block_size, m_bits, m_mode, 0.0, v_bits, momentum_only)


def fused_update_1d_apply(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha,
                          beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq,
                          numel, block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only):
    _u1d(2, False, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, None,
         None, 0, 0, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         m_block_size, m_bits, m_mode, d, v_bits, momentum_only)


def fused_update_1d_lag(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, norm_buf, alpha, prev_norm,
                        beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq,
                        numel, block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only):
    _u1d(3, False, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, None, norm_buf, alpha, prev_norm,
         None, 0, 0, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         m_block_size, m_bits, m_mode, d, v_bits, momentum_only)


def fused_update_1d_noclip_sr(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, alpha, decay, sr_seed,
                              sr_step, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq,
                              eps_for_grad_sq, numel, block_size, m_block_size, m_bits, m_mode, v_bits,
                              momentum_only):
    _u1d(0, True, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, None, None, alpha, None, decay,
         sr_seed, sr_step, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, m_block_size, m_bits, m_mode, 0.0, v_bits, momentum_only)


def fused_update_1d_apply_sr(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha,
                             decay, sr_seed, sr_step, beta1, beta_val, eps_for_denom, use_adam_denom,
                             log_eps_sq, eps_for_grad_sq, numel, block_size, m_block_size, m_bits, m_mode,
                             d, v_bits, momentum_only):
    _u1d(2, True, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, None,
         decay, sr_seed, sr_step, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only)


def fused_update_1d_lag_sr(param, grad, m_q, m_scale, v_q, v_scale, v_min_log, norm_buf, alpha,
                           prev_norm, decay, sr_seed, sr_step, beta1, beta_val, eps_for_denom,
                           use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size, m_block_size,
                           m_bits, m_mode, d, v_bits, momentum_only):
    _u1d(3, True, param, grad, m_q, m_scale, v_q, v_scale, v_min_log, None, norm_buf, alpha, prev_norm,
         decay, sr_seed, sr_step, beta1, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, m_block_size, m_bits, m_mode, d, v_bits, momentum_only)


# ---- fused_update_1d_vonly_* (kernels.cu:1100-1255): no momentum
def fused_update_1d_vonly_noclip(param, grad, v_q, v_scale, v_min_log, alpha, beta_val, eps_for_denom,
                                 use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size, v_bits):
    _u1d(0, False, param, grad, None, None, v_q, v_scale, v_min_log, None, None, alpha, None, None, 0, 0,
         0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size, block_size, 0,
         0, 0.0, v_bits, False)


def fused_update_1d_vonly_norm(grad, v_q, v_scale, v_min_log, v_buf, norm_buf, beta_val, eps_for_denom,
                               use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size, v_bits):
    _u1d(1, False, None, grad, None, None, v_q, v_scale, v_min_log, v_buf, norm_buf, None, None, None, 0,
         0, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size, block_size,
         0, 0, 0.0, v_bits, False)


def fused_update_1d_vonly_apply(param, grad, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, beta_val,
                                eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
                                block_size, d, v_bits):
    _u1d(2, False, param, grad, None, None, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, None, None,
         0, 0, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         block_size, 0, 0, d, v_bits, False)


def fused_update_1d_vonly_lag(param, grad, v_q, v_scale, v_min_log, norm_buf, alpha, prev_norm, beta_val,
                              eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
                              block_size, d, v_bits):
    _u1d(3, False, param, grad, None, None, v_q, v_scale, v_min_log, None, norm_buf, alpha, prev_norm,
         None, 0, 0, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel, block_size,
         block_size, 0, 0, d, v_bits, False)


def fused_update_1d_vonly_noclip_sr(param, grad, v_q, v_scale, v_min_log, alpha, decay, sr_seed, sr_step,
                                    beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq,
                                    numel, block_size, v_bits):
    _u1d(0, True, param, grad, None, None, v_q, v_scale, v_min_log, None, None, alpha, None, decay,
         sr_seed, sr_step, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, block_size, 0, 0, 0.0, v_bits, False)


def fused_update_1d_vonly_apply_sr(param, grad, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, decay,
                                   sr_seed, sr_step, beta_val, eps_for_denom, use_adam_denom, log_eps_sq,
                                   eps_for_grad_sq, numel, block_size, d, v_bits):
    _u1d(2, True, param, grad, None, None, v_q, v_scale, v_min_log, v_buf, norm_buf, alpha, None, decay,
         sr_seed, sr_step, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, block_size, 0, 0, d, v_bits, False)


def fused_update_1d_vonly_lag_sr(param, grad, v_q, v_scale, v_min_log, norm_buf, alpha, prev_norm, decay,
                                 sr_seed, sr_step, beta_val, eps_for_denom, use_adam_denom, log_eps_sq,
                                 eps_for_grad_sq, numel, block_size, d, v_bits):
    _u1d(3, True, param, grad, None, None, v_q, v_scale, v_min_log, None, norm_buf, alpha, prev_norm,
         decay, sr_seed, sr_step, 0.0, beta_val, eps_for_denom, use_adam_denom, log_eps_sq, eps_for_grad_sq, numel,
         block_size, block_size, 0, 0, d, v_bits, False)


# ---- fused_update_1d_full_*[_sr] (kernels.cu:1374-1515): fp32 state
def _full(mode, param, grad, variance, m, norm_buf, alpha, prev_norm, beta1, beta_val, eps_sq,
          eps_for_denom, use_adam_denom, eps_for_grad_sq, numel, d, momentum_only, decay=None, sr_seed=None,
          sr_step=0):
    sr = sr_seed is not None and param is not None and param.dtype in (torch.bfloat16, torch.float16)
    parts = _parts(grad.device, nat.lib().a8_norm_parts_full(int(numel))) if mode in (1, 3) else None
    rc = nat.lib().a8_fused_update_1d_full(
        mode, nat.dtype_code(grad.dtype), nat.ptr(param), nat.ptr(grad), nat.ptr(variance), nat.ptr(m),
        nat.ptr(norm_buf), nat.ptr(parts), nat.ptr(alpha), nat.ptr(prev_norm), nat.ptr(decay), float(beta1), float(beta_val),
        float(eps_sq), float(eps_for_denom), int(bool(use_adam_denom)), float(eps_for_grad_sq),
        int(numel), float(d), int(bool(momentum_only)), 0.0, 1.0, 0, int(sr), int(sr_seed or 0), int(sr_step), 0,
        _stream(grad))
    nat.check(rc, "fused_update_1d_full")


def fused_update_1d_full_noclip(param, grad, variance, m, alpha, beta1, beta_val, eps_sq, eps_for_denom,
                                use_adam_denom, eps_for_grad_sq, numel, momentum_only):
    _full(0, param, grad, variance, m, None, alpha, None, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, 0.0, momentum_only)


def fused_update_1d_full_norm(grad, variance, m, norm_buf, beta1, beta_val, eps_sq, eps_for_denom,
                              use_adam_denom, eps_for_grad_sq, numel, momentum_only):
    _full(1, None, grad, variance, m, norm_buf, None, None, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, 0.0, momentum_only)


def fused_update_1d_full_apply(param, grad, variance, m, norm_buf, alpha, beta1, beta_val, eps_sq,
                               eps_for_denom, use_adam_denom, eps_for_grad_sq, numel, d, momentum_only):
    _full(2, param, grad, variance, m, norm_buf, alpha, None, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, d, momentum_only)


def fused_update_1d_full_lag(param, grad, variance, m, norm_buf, alpha, prev_norm, beta1, beta_val,
                             eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, numel, d,
                             momentum_only):
    _full(3, param, grad, variance, m, norm_buf, alpha, prev_norm, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, d, momentum_only)


def fused_update_1d_full_noclip_sr(param, grad, variance, m, alpha, decay, sr_seed, sr_step, beta1, beta_val,
                                   eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, numel, momentum_only):
    _full(0, param, grad, variance, m, None, alpha, None, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, 0.0, momentum_only, decay, sr_seed, sr_step)


def fused_update_1d_full_apply_sr(param, grad, variance, m, norm_buf, alpha, decay, sr_seed, sr_step, beta1,
                                  beta_val, eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, numel, d,
                                  momentum_only):
    _full(2, param, grad, variance, m, norm_buf, alpha, None, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, d, momentum_only, decay, sr_seed, sr_step)


def fused_update_1d_full_lag_sr(param, grad, variance, m, norm_buf, alpha, prev_norm, decay, sr_seed, sr_step,
                                beta1, beta_val, eps_sq, eps_for_denom, use_adam_denom, eps_for_grad_sq, numel,
                                d, momentum_only):
    _full(3, param, grad, variance, m, norm_buf, alpha, prev_norm, beta1, beta_val, eps_sq, eps_for_denom,
          use_adam_denom, eps_for_grad_sq, numel, d, momentum_only, decay, sr_seed, sr_step)


# ---- decode utilities (kernels.cu:2571-2632)
def dequantize_log_nonneg(output, q, scale, min_log, numel, block_size, v_bits):
    if int(v_bits) == 8 and q.dtype != torch.uint8:
        raise RuntimeError("v_bits=8 requires q to be torch.uint8")
    if int(v_bits) == 16 and q.dtype != torch.int16:
        raise RuntimeError("v_bits=16 requires q to be torch.int16")
    if scale.dtype != torch.float32 or min_log.dtype != torch.float32:
        raise RuntimeError("scale and min_log must be torch.float32")
    rc = nat.lib().a8_dequantize_log_nonneg(nat.ptr(output), nat.ptr(q), nat.ptr(scale), nat.ptr(min_log),
                                            int(numel), int(block_size), int(v_bits), _stream(output))
    nat.check(rc, "dequantize_log_nonneg")


def dequantize_dynamic(output, q, scale, numel, block_size, m_bits):
    rc = nat.lib().a8_dequantize_dynamic(nat.ptr(output), nat.ptr(q), nat.ptr(scale), int(numel),
                                         int(block_size), int(m_bits), _stream(output))
    nat.check(rc, "dequantize_dynamic")


# ---- fused_m_quantize_lerp (kernels.cu:574-588)
def fused_m_quantize_lerp(q, scale, new_val, fp32_out, beta, block_size, N, m_bits, m_mode):
    """Momentum EMA in place: m' = lerp(deq(q, scale), new_val, 1 - beta), requantised
    per block; fp32_out (optional) receives m'."""
    if q.dtype != torch.uint8 or scale.dtype != torch.float32:
        raise RuntimeError("q must be torch.uint8 and scale torch.float32")
    if fp32_out is not None and fp32_out.dtype != torch.float32:
        raise RuntimeError("fp32_out must be torch.float32")
    rc = nat.lib().a8_m_quantize_lerp(nat.ptr(q), nat.ptr(scale), nat.ptr(new_val), nat.dtype_code(new_val.dtype),
                                      nat.ptr(fp32_out), float(beta), int(block_size), int(N), int(m_bits),
                                      int(m_mode), _stream(new_val))
    nat.check(rc, "fused_m_quantize_lerp")


# ---- fused_log_quantize_lerp (kernels.cu:332-368)
def fused_log_quantize_lerp(q, scale, min_log_out, new_val, fp32_out, beta, block_size, square_input, eps1, N,
                            log_floor, v_bits):
    """V EMA in place: v' = lerp(deq(q), x, beta) with x = new_val (squared + eps1
    when square_input), AL-requantised per block; fp32_out (optional) receives v'."""
    _vbits_check(q, v_bits)
    if scale.dtype != torch.float32 or min_log_out.dtype != torch.float32:
        raise RuntimeError("scale and min_log_out must be torch.float32")
    rc = nat.lib().a8_log_quantize_lerp(nat.ptr(q), nat.ptr(scale), nat.ptr(min_log_out), nat.ptr(new_val),
                                        nat.dtype_code(new_val.dtype), nat.ptr(fp32_out), float(beta),
                                        int(block_size), int(bool(square_input)), float(eps1), int(N),
                                        float(log_floor), int(v_bits), _stream(new_val))
    nat.check(rc, "fused_log_quantize_lerp")


# ---- factored element primitives (kernels.cu:1523-2400)
_F_NOCLIP, _F_NORM, _F_APPLY, _F_LAG, _F_SUMS, _F_CAME1, _F_CAME2N, _F_CAME2 = range(8)


def _fprim(op, ref, stochastic=False, **kw):
    """One a8_factored_prim call; ``ref`` is the tensor whose dtype and device
    select the kernel (the gradient, or the parameter)."""
    a = nat.FactoredPrimArgs()
    for k, v in kw.items():
        if torch.is_tensor(v):
            setattr(a, k, v.data_ptr())
        elif v is None:
            setattr(a, k, None)
        else:
            setattr(a, k, v)
    rc = nat.lib().a8_factored_prim(op, nat.dtype_code(ref.dtype), int(bool(stochastic)), a, _stream(ref))
    nat.check(rc, "factored primitive")


def _sr_check(param, grad):
    if param.dtype not in (torch.bfloat16, torch.float16) or (grad is not None and grad.dtype != param.dtype):
        raise RuntimeError("SR writeback requires matching FP16/BF16 param and grad")


def _u2d(op, param, grad, m_q, m_scale, m, row, col, rm, norm_buf, alpha, prev_norm, decay, sr_seed, sr_step,
         beta1, R, C, numel, m_block_size, m_bits, m_mode, d, sr):
    if sr:
        _sr_check(param, grad)
    _fprim(op, grad, sr, param=param, grad=grad, m_q=m_q, m_scale=m_scale, m=m, row=row, col=col,
           row_mean=rm, norm_buf=norm_buf, alpha=alpha, prev_norm=prev_norm, decay=decay, rows=int(R),
           cols=int(C), numel=int(numel), beta1=float(beta1), d=float(d), m_bits=int(m_bits), m_mode=int(m_mode),
           m_block_size=int(m_block_size), sr_seed=int(sr_seed), sr_step=int(sr_step))


def fused_update_2d_noclip(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, alpha, beta1, R, C, numel,
                           m_block_size, m_bits, m_mode):
    _u2d(_F_NOCLIP, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, None, alpha, None, None, 0, 0,
         beta1, R, C, numel, m_block_size, m_bits, m_mode, 0.0, False)


def fused_update_2d_norm(grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, norm_buf, beta1, R, C, numel,
                         m_block_size, m_bits, m_mode):
    _u2d(_F_NORM, None, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, norm_buf, None, None, None, 0, 0,
         beta1, R, C, numel, m_block_size, m_bits, m_mode, 0.0, False)


def fused_update_2d_apply(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, beta1, R, C,
                          numel, m_block_size, m_bits, m_mode, d):
    _u2d(_F_APPLY, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, None, None, 0,
         0, beta1, R, C, numel, m_block_size, m_bits, m_mode, d, False)


def fused_update_2d_lag(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm,
                        beta1, R, C, numel, m_block_size, m_bits, m_mode, d):
    _u2d(_F_LAG, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, None,
         0, 0, beta1, R, C, numel, m_block_size, m_bits, m_mode, d, False)


def fused_update_2d_noclip_sr(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, alpha, decay, sr_seed,
                              sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode):
    _u2d(_F_NOCLIP, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, None, alpha, None, decay,
         sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, 0.0, True)


def fused_update_2d_apply_sr(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, decay,
                             sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, d):
    _u2d(_F_APPLY, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, None, decay,
         sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, d, True)


def fused_update_2d_lag_sr(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm,
                           decay, sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, d):
    _u2d(_F_LAG, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, decay,
         sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, d, True)


def fused_update_2d_full_noclip(param, grad, m, row_fp32, col_fp32, row_mean_val, alpha, beta1, R, C, numel,
                                m_block_size):
    _u2d(_F_NOCLIP, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, None, alpha, None, None, 0, 0,
         beta1, R, C, numel, m_block_size, 8, 0, 0.0, False)


def fused_update_2d_full_norm(grad, m, row_fp32, col_fp32, row_mean_val, norm_buf, beta1, R, C, numel, m_block_size):
    _u2d(_F_NORM, None, grad, None, None, m, row_fp32, col_fp32, row_mean_val, norm_buf, None, None, None, 0, 0,
         beta1, R, C, numel, m_block_size, 8, 0, 0.0, False)


def fused_update_2d_full_apply(param, grad, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, beta1, R, C,
                               numel, m_block_size, d):
    _u2d(_F_APPLY, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, None, None, 0, 0,
         beta1, R, C, numel, m_block_size, 8, 0, d, False)


def fused_update_2d_full_lag(param, grad, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, beta1, R,
                             C, numel, m_block_size, d):
    _u2d(_F_LAG, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, None, 0, 0,
         beta1, R, C, numel, m_block_size, 8, 0, d, False)


def fused_update_2d_full_noclip_sr(param, grad, m, row_fp32, col_fp32, row_mean_val, alpha, decay, sr_seed, sr_step,
                                   beta1, R, C, numel, m_block_size):
    _u2d(_F_NOCLIP, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, None, alpha, None, decay, sr_seed,
         sr_step, beta1, R, C, numel, m_block_size, 8, 0, 0.0, True)


def fused_update_2d_full_apply_sr(param, grad, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, decay, sr_seed,
                                  sr_step, beta1, R, C, numel, m_block_size, d):
    _u2d(_F_APPLY, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, None, decay,
         sr_seed, sr_step, beta1, R, C, numel, m_block_size, 8, 0, d, True)


def fused_update_2d_full_lag_sr(param, grad, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, decay,
                                sr_seed, sr_step, beta1, R, C, numel, m_block_size, d):
    _u2d(_F_LAG, param, grad, None, None, m, row_fp32, col_fp32, row_mean_val, norm_buf, alpha, prev_norm, decay,
         sr_seed, sr_step, beta1, R, C, numel, m_block_size, 8, 0, d, True)


def compute_factored_sums(grad, row_sum, col_sum, R, C, numel):
    _fprim(_F_SUMS, grad, grad=grad, row_sum=row_sum, col_sum=col_sum, rows=int(R), cols=int(C), numel=int(numel))


def compute_ut_rms(grad, row_fp32, col_fp32, row_mean_val, ut_sq_sum, R, C, numel):
    _fprim(_F_NORM, grad, grad=grad, row=row_fp32, col=col_fp32, row_mean=row_mean_val, norm_buf=ut_sq_sum,
           rows=int(R), cols=int(C), numel=int(numel))


def fused_came_pass1(grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, res_row_sum, res_col_sum, clip_factor,
                     beta1, eps_came, R, C, numel, m_block_size, m_bits, m_mode):
    _fprim(_F_CAME1, grad, grad=grad, m_q=m_q, m_scale=m_scale, row=row_fp32, col=col_fp32, row_mean=row_mean_val,
           row_sum=res_row_sum, col_sum=res_col_sum, clip=clip_factor, beta1=float(beta1), eps_came=float(eps_came),
           rows=int(R), cols=int(C), numel=int(numel), m_block_size=int(m_block_size), m_bits=int(m_bits),
           m_mode=int(m_mode))


def _came2(op, param, grad, m_q, m_scale, m, row, col, rm, crow, ccol, crm, clip, norm_buf, alpha, decay, sr_seed,
           sr_step, beta1, R, C, numel, m_block_size, m_bits, m_mode, sr):
    ref = grad if grad is not None else m
    if sr:
        _sr_check(param, grad)
    _fprim(op, param if (param is not None and op == _F_CAME2) else ref, sr, param=param, grad=grad, m_q=m_q,
           m_scale=m_scale, m=m, row=row, col=col, row_mean=rm, conf_row=crow, conf_col=ccol, conf_row_mean=crm,
           clip=clip, norm_buf=norm_buf, alpha=alpha, decay=decay, sr_seed=int(sr_seed), sr_step=int(sr_step),
           beta1=float(beta1), rows=int(R), cols=int(C), numel=int(numel), m_block_size=int(m_block_size),
           m_bits=int(m_bits), m_mode=int(m_mode))


def fused_came_pass2_norm(grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
                          conf_row_mean, clip_factor, norm_buf, beta1, R, C, numel, m_block_size, m_bits, m_mode):
    _came2(_F_CAME2N, None, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
           conf_row_mean, clip_factor, norm_buf, None, None, 0, 0, beta1, R, C, numel, m_block_size, m_bits, m_mode,
           False)


def fused_came_pass2(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
                     conf_row_mean, clip_factor, alpha, beta1, R, C, numel, m_block_size, m_bits, m_mode):
    _came2(_F_CAME2, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
           conf_row_mean, clip_factor, None, alpha, None, 0, 0, beta1, R, C, numel, m_block_size, m_bits, m_mode,
           False)


def fused_came_pass2_sr(param, grad, m_q, m_scale, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
                        conf_row_mean, clip_factor, alpha, decay, sr_seed, sr_step, beta1, R, C, numel, m_block_size,
                        m_bits, m_mode):
    _came2(_F_CAME2, param, grad, m_q, m_scale, None, row_fp32, col_fp32, row_mean_val, conf_row_fp32, conf_col_fp32,
           conf_row_mean, clip_factor, None, alpha, decay, sr_seed, sr_step, beta1, R, C, numel, m_block_size, m_bits,
           m_mode, True)


def fused_came_full_pass1(grad, m, row_fp32, col_fp32, row_mean_val, res_row_sum, res_col_sum, clip_factor, beta1,
                          eps_came, R, C, numel, m_block_size):
    _fprim(_F_CAME1, grad, grad=grad, m=m, row=row_fp32, col=col_fp32, row_mean=row_mean_val, row_sum=res_row_sum,
           col_sum=res_col_sum, clip=clip_factor, beta1=float(beta1), eps_came=float(eps_came), rows=int(R),
           cols=int(C), numel=int(numel), m_block_size=int(m_block_size))


def fused_came_full_pass2(param, m, conf_row_fp32, conf_col_fp32, conf_row_mean, norm_buf, alpha, R, C, numel,
                          m_block_size, norm_only):
    op = _F_CAME2N if norm_only else _F_CAME2
    if norm_only and norm_buf is None:
        raise RuntimeError("fused_came_full_pass2: norm_only needs norm_buf")
    _fprim(op, param, param=None if norm_only else param, m=m, conf_row=conf_row_fp32, conf_col=conf_col_fp32,
           conf_row_mean=conf_row_mean, norm_buf=norm_buf, alpha=alpha, rows=int(R), cols=int(C), numel=int(numel),
           m_block_size=int(m_block_size))


def fused_came_full_pass2_sr(param, m, conf_row_fp32, conf_col_fp32, conf_row_mean, alpha, decay, sr_seed, sr_step,
                             R, C, numel, m_block_size):
    _sr_check(param, None)
    _fprim(_F_CAME2, param, True, param=param, m=m, conf_row=conf_row_fp32, conf_col=conf_col_fp32,
           conf_row_mean=conf_row_mean, alpha=alpha, decay=decay, sr_seed=int(sr_seed), sr_step=int(sr_step),
           rows=int(R), cols=int(C), numel=int(numel), m_block_size=int(m_block_size))


# ---- APOLLO primitives (kernels.cu:2410-2570, 2638-3000)
def compute_apollo_norms(m_fp32, v_fp32, grad_low, norm_update, norm_grad, N, D, stride_N, stride_D, apollo_eps):
    rc = nat.lib().a8_apollo_norms(nat.ptr(m_fp32), nat.ptr(v_fp32), nat.ptr(grad_low), nat.ptr(norm_update),
                                   nat.ptr(norm_grad), int(N), int(D), int(stride_N), int(stride_D),
                                   int(m_fp32.numel()), float(apollo_eps), 0, _stream(m_fp32))
    nat.check(rc, "compute_apollo_norms")


def compute_apollo_came_rms(grad_low, v_fp32, sum_u2, eps_sq, numel):
    rc = nat.lib().a8_apollo_came_rms(nat.ptr(grad_low), nat.ptr(v_fp32), nat.ptr(sum_u2), float(eps_sq),
                                      int(numel), _stream(grad_low))
    nat.check(rc, "compute_apollo_came_rms")


def apollo_came_compute_m_res(grad_low, v_fp32, m_q_old, m_scale_old, res_fp32_old, m_temp, res_temp, clip_factor,
                              beta1, beta3, eps_came, eps_sq, m_block_size, numel, m_bits, m_mode):
    rc = nat.lib().a8_apollo_came_m_res(nat.ptr(grad_low), nat.ptr(v_fp32), nat.ptr(m_q_old), nat.ptr(m_scale_old),
                                        nat.ptr(res_fp32_old), nat.ptr(m_temp), nat.ptr(res_temp),
                                        nat.ptr(clip_factor), float(beta1), float(beta3), float(eps_came),
                                        float(eps_sq), int(m_block_size), int(numel), int(m_bits), int(m_mode),
                                        _stream(grad_low))
    nat.check(rc, "apollo_came_compute_m_res")


def apollo_came_compute_update_norms(m_fp32_new, res_fp32_new, grad_low, norm_update, norm_grad, eps_sq, N, D,
                                     stride_N, stride_D, numel):
    rc = nat.lib().a8_apollo_norms(nat.ptr(m_fp32_new), nat.ptr(res_fp32_new), nat.ptr(grad_low),
                                   nat.ptr(norm_update), nat.ptr(norm_grad), int(N), int(D), int(stride_N),
                                   int(stride_D), int(numel), float(eps_sq), 1, _stream(m_fp32_new))
    nat.check(rc, "apollo_came_compute_update_norms")


def _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, native, sr, maximize=False,
          sr_seed=0, sr_step=0, want=None):
    if want is not None and param.dtype != want:
        raise RuntimeError(f"param must be {want}")
    if param.dim() != 2 or not param.is_contiguous() or not grad.is_contiguous():
        raise RuntimeError("param must be 2D; param and grad must be contiguous")
    if native and grad.dtype != param.dtype:
        raise RuntimeError("param and grad dtypes must match")
    if not native and grad.dtype != torch.float32:
        raise RuntimeError("grad must be float32")
    if final_scale.dtype != torch.float32:
        raise RuntimeError("final_scale must be float32")
    dec = decay if (decay is not None and decay.numel()) else None
    rc = nat.lib().a8_apollo_writeback(nat.dtype_code(param.dtype), int(native), int(sr), nat.ptr(param),
                                       nat.ptr(grad), nat.ptr(final_scale), nat.ptr(dec), nat.ptr(update_scale),
                                       int(bool(side_right)), int(bool(is_channel)), int(bool(maximize)),
                                       int(sr_seed), int(sr_step), param.shape[0], param.shape[1], _stream(param))
    nat.check(rc, "apollo_apply")


def apollo_apply_bf16_det(param, grad, final_scale, decay, update_scale, side_right, is_channel):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, False, False, want=torch.bfloat16)


def apollo_apply_bf16_sr(param, grad, final_scale, decay, update_scale, side_right, is_channel, sr_seed, sr_step):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, False, True, sr_seed=sr_seed,
          sr_step=sr_step, want=torch.bfloat16)


def apollo_apply_fp16_sr(param, grad, final_scale, decay, update_scale, side_right, is_channel, sr_seed, sr_step):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, False, True, sr_seed=sr_seed,
          sr_step=sr_step, want=torch.float16)


def apollo_apply_bf16_det_native(param, grad, final_scale, decay, update_scale, side_right, is_channel, maximize):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, True, False, maximize,
          want=torch.bfloat16)


def apollo_apply_fp16_det_native(param, grad, final_scale, decay, update_scale, side_right, is_channel, maximize):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, True, False, maximize,
          want=torch.float16)


def apollo_apply_bf16_sr_native(param, grad, final_scale, decay, update_scale, side_right, is_channel, maximize,
                                sr_seed, sr_step):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, True, True, maximize, sr_seed,
          sr_step, want=torch.bfloat16)


def apollo_apply_fp16_sr_native(param, grad, final_scale, decay, update_scale, side_right, is_channel, maximize,
                                sr_seed, sr_step):
    _apwb(param, grad, final_scale, decay, update_scale, side_right, is_channel, True, True, maximize, sr_seed,
          sr_step, want=torch.float16)


# ---- fira_scalar (kernels.cu:3055-3084)
def fira_scalar(x, prev, alpha, has_prev, apply, margin, inv_margin):
    """Returns [3n] fp32: scale (or alpha*scale), next previous norm, cleaned input."""
    n = x.numel()
    out = torch.empty(3 * n, dtype=torch.float32, device=x.device)
    rc = nat.lib().a8_fira_scalar(nat.ptr(x), nat.ptr(prev) if has_prev else None,
                                  nat.ptr(alpha) if apply else None, nat.ptr(out), n, int(bool(has_prev)),
                                  int(bool(apply)), float(margin), _stream(x))
    nat.check(rc, "fira_scalar")
    return out


def qmaps():
    """The codebooks set_qmap expects (dynamic_map(8), dynamic_map(4))."""
    return dynamic_map(8), dynamic_map(4)
