"""Drop-in for the reference's compiled module ``adafactor8bit_cuda``.

The reference JIT-builds ``adafactor8bit/kernels.cu`` into a pybind11 module of
that name (optimizer.py:85-98; bindings kernels.cu:3089-3150) and calls it as
``_CUDA_MODULE.<name>(...)``.  This module exposes the same names with the same
positional signatures, converts tensors to device pointers and launches the
HIP kernels of ``libadafactor8bit_amd.so`` on the current stream.

Numerics follow the reference's PyTorch path (optimizer.py:299-353, 504-532):
the AL floor of the 1-D kernels is the CPU quantiser's -126, so the
``log_eps_sq`` argument only supplies eps1 for the Adam denominator's momentum clamp.

Names of the reference module not listed in ``__all__`` are not provided yet;
looking one up raises ``AttributeError``, which the reference's own
``hasattr`` probes (optimizer.py:738, 2621-2628) treat as "absent".
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
]

_AL_FLOOR = -126.0
_EPS_FLOOR = 1.17549435e-38


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
    rc = nat.lib().a8_fused_update_1d(
        mode, int(sr), nat.dtype_code(ref.dtype), nat.ptr(param), nat.ptr(grad), nat.ptr(m_q),
        nat.ptr(m_scale), nat.ptr(v_q), nat.ptr(v_scale), nat.ptr(v_min_log), nat.ptr(v_buf),
        nat.ptr(norm_buf), nat.ptr(alpha), nat.ptr(prev_norm), nat.ptr(dec), int(sr_seed), int(sr_step),
        float(beta1), float(beta_val), float(eps_for_denom), int(bool(use_adam_denom)), _AL_FLOOR,
        float(eps_for_grad_sq), eps_sq, int(numel),
        int(block_size), int(m_block_size), int(m_bits), int(m_mode), float(d), int(v_bits),
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
    rc = nat.lib().a8_fused_update_1d_full(
        mode, nat.dtype_code(grad.dtype), nat.ptr(param), nat.ptr(grad), nat.ptr(variance), nat.ptr(m),
        nat.ptr(norm_buf), nat.ptr(alpha), nat.ptr(prev_norm), nat.ptr(decay), float(beta1), float(beta_val),
        float(eps_sq), float(eps_for_denom), int(bool(use_adam_denom)), float(eps_for_grad_sq),
        int(numel), float(d), int(bool(momentum_only)), 0.0, 1.0, 0, int(sr), int(sr_seed or 0), int(sr_step),
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
