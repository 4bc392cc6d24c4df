"""CPU oracle: a restatement of adafactor8bit's pure-PyTorch optimizer step.

TEST INFRASTRUCTURE ONLY.  Nothing in the product imports this module: only
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and only as the checker (or, for ``cpu_baseline``, as the
CPU restatement that is timed).  The product path is the HIP library and fails
loudly without it.

Every function states the reference file:line it follows.  The arithmetic runs
in float32 torch ATen CPU kernels, op for op in the reference's order, because
the reference's own fallback is built from those same kernels
(``torch.lerp`` = fma(w, e-s, s) for w < 0.5, ``add_(x, alpha=a)`` = fma(a, x, p),
``torch.round`` = half-to-even, int16 storage wraps).

Pinning (see tests/test_oracle_*.py):
  * codecs (AL8/AL16, UF8/UF4, D8/D4, dynamic map): closed forms, brute force
    over every code, invariants (q=0 <=> v=0, half-step decode error bound,
    monotonicity), plus the golden trajectories;
  * step functions: the golden fixtures written by tests/golden/gen_golden.py
    from the reference itself, bit-exact;
  * Fira scalar: truth table over first step / reset / growth / non-finite;
  * the fused 1-D CUDA kernels' AL rule (al_quantize_kernel, al_refit_rule
    "kernel"): kernels.cu cannot run here, so it is pinned by closed forms read
    from kernels.cu:686-687, 772-791, 318-326 (tests/test_oracle_kernel_rule.py).
"""
import math
from typing import Any, Dict, Optional

import numpy as np
import torch

LOG_QUANT_FLOOR = 1.17549435e-38  # optimizer.py:22

# Reduction order.  The reference reduces in float32, in torch's CPU order
# (``mean``, ``vector_norm``, ``norm``, ``sum``); that is what the golden fixtures
# pin.  With EXACT_REDUCTIONS set, every such reduction accumulates in float64 and
# rounds once to float32: the value any fixed summation order approximates.  The
# large-shape GPU tests set it, because over millions of terms torch's float32
# order drifts from that value by up to ~1e-4 relative (a CAME clip factor over a
# 2304 x 2080 matrix), far more than the reduction error of the HIP kernels.
EXACT_REDUCTIONS = False


def set_exact_reductions(on: bool) -> bool:
    """Switch the reduction mode; returns the previous one."""
    global EXACT_REDUCTIONS
    old, EXACT_REDUCTIONS = EXACT_REDUCTIONS, bool(on)
    return old


def _mean(x, dim):
    """``x.mean(dim, keepdim=True)``.  On the CPU torch forms a float32 mean as the
    float32 sum divided by the count (ReduceOps.cpp, mean_out: sum_out then div_);
    the exact form keeps that structure with an exactly accumulated sum."""
    if EXACT_REDUCTIONS:
        return x.double().sum(dim=dim, keepdim=True).float() / x.shape[dim]
    return x.mean(dim=dim, keepdim=True)


def _vnorm(x, dim=None, f32=False):
    """``torch.linalg.vector_norm(x)`` (``dtype=torch.float32`` when ``f32``), or
    along ``dim`` with keepdim (``x.norm(dim=dim, keepdim=True)``).  Exact form: the
    sum of squares accumulated exactly, rounded to float32, then a float32 sqrt."""
    kd = dim is not None
    if EXACT_REDUCTIONS:
        return x.double().square().sum(dim=dim, keepdim=kd).float().sqrt()
    if f32:
        return torch.linalg.vector_norm(x, ord=2, dim=dim, keepdim=kd, dtype=torch.float32)
    if kd:
        return x.norm(dim=dim, keepdim=True)
    return torch.linalg.vector_norm(x)


def _sum(x):
    """``x.sum()``."""
    if EXACT_REDUCTIONS:
        return x.double().sum().float()
    return x.sum()


# --------------------------------------------------------------------------
# AL (adaptive log-space) codec            optimizer.py:299-353
# --------------------------------------------------------------------------
def al_quantize(v: torch.Tensor, block_size: int, floor: float = -126.0, levels: int = 256):
    """Block-wise log-space quantisation with a reserved zero code.

    Follows ``_log_quantize_nonneg`` (optimizer.py:299-325): zero-pad to the
    block size, log2 of max(v, 1e-38), l_min = min over non-zero entries clamped
    at ``floor``, l_max = max over all entries, l_min := l_max-1 when
    l_min >= l_max, scale = max(l_max-l_min, 1e-12),
    q = clamp(round((l-l_min)/scale*(levels-2))+1, 1, levels-1), q=0 for v=0.
    Returns (codes, scale[nb], min_log[nb], pad).  AL16 codes are int16 (wrapping).
    """
    shape = v.shape
    flat = v.reshape(-1)
    pad = (block_size - flat.numel() % block_size) % block_size
    if pad:
        flat = torch.nn.functional.pad(flat, (0, pad))
    blocks = flat.view(-1, block_size)
    zero = blocks == 0
    logs = torch.log2(blocks.clamp(min=1e-38))
    lmin = logs.masked_fill(zero, float("inf")).min(dim=1, keepdim=True).values
    lmax = logs.amax(dim=1, keepdim=True)
    lmin = lmin.clamp(min=floor)
    lmin = torch.where(lmin >= lmax, lmax - 1.0, lmin)
    scale = (lmax - lmin).clamp(min=1e-12)
    top = levels - 1
    q = (torch.round((logs - lmin) / scale * (top - 1.0)) + 1.0).clamp(1, top)
    q[zero] = 0.0
    dt = torch.uint8 if levels <= 256 else torch.int16
    del shape
    return q.to(dt), scale.squeeze(-1), lmin.squeeze(-1), pad


def al_dequantize(q: torch.Tensor, scale: torch.Tensor, min_log: torch.Tensor, numel: int):
    """Inverse of :func:`al_quantize` (optimizer.py:341-353, CPU branch).

    v = 0 for q = 0, else 2^(((q-1)*scale)/(levels-2) + min_log), computed in that
    order in float32; int16 codes below zero get 65536 added back.
    Returns the first ``numel`` decoded values (flat).
    """
    qf = q.reshape(-1)
    levels = 256 if qf.dtype == torch.uint8 else 65536
    bs = qf.numel() // scale.numel()
    q2 = qf.view(-1, bs)
    zero = q2 == 0
    x = q2.float()
    if q2.dtype == torch.int16:
        x = torch.where(x < 0, x + 65536.0, x)
    logs = (x - 1.0) * scale.unsqueeze(-1) / (levels - 2.0) + min_log.unsqueeze(-1)
    out = torch.pow(2.0, logs)
    out[zero] = 0.0
    return out.reshape(-1)[:numel]


# --------------------------------------------------------------------------
# AL codec, the reference's fused 1-D CUDA kernels' rule   kernels.cu:318-326, 686-687, 772-791
# --------------------------------------------------------------------------
FLT_MIN = 1.17549435e-38
LOG_ZERO, LOG_MAX, MIN_SCALE = -1e30, 126.0, 1e-12     # kernels.cu:15-17


def kernel_floor(eps1: float) -> float:
    """The kernels' floor: log_eps_sq = log2(max(eps1^2, FLT_MIN)) (optimizer.py:1961-1962)."""
    return float(np.float32(math.log2(max(eps1 * eps1, FLT_MIN))))


def al_quantize_kernel(v: torch.Tensor, block_size: int, floor: float, levels: int = 256):
    """The fused 1-D kernels' refit and codes (kernels.cu:686-687, 772-791, 322-326).

    Per block of the tensor's elements (no padding enters the statistics):
    l = log2(v), log2(0) = -inf; lmax = min(max(-1e30, max l), 126); lmin =
    max(min(126, min l), floor) with zeros in the minimum; lmin := lmax - 1 if
    lmin >= lmax; s = max(lmax - lmin, 1e-12); code 0 for v == 0, else
    clamp(rint((l - lmin) * fp32((levels-2)/s)) + 1, 1, levels-1), every operation
    rounded to fp32.  log2 is correctly rounded here (CUDA's log2f is within an ulp
    or two).  Returns (codes, scale, min_log, pad) as :func:`al_quantize`.
    """
    flat = v.reshape(-1).to(torch.float32).numpy().astype(np.float32)
    n = flat.size
    pad = (block_size - n % block_size) % block_size
    nb = (n + pad) // block_size
    lm2 = np.float32(levels - 2)
    codes = np.zeros(n + pad, dtype=np.int64)
    scale = np.zeros(nb, dtype=np.float32)
    minlog = np.zeros(nb, dtype=np.float32)
    with np.errstate(divide="ignore"):
        logs = np.where(flat > 0, np.log2(flat.astype(np.float64)), -np.inf).astype(np.float32)
    f32 = np.float32
    for b in range(nb):
        lo, hi = b * block_size, min((b + 1) * block_size, n)
        lb = logs[lo:hi]
        lmax = min(max(f32(LOG_ZERO), lb.max()), f32(LOG_MAX))
        lmin = max(min(f32(LOG_MAX), lb.min()), f32(floor))
        if lmin >= lmax:
            lmin = f32(lmax - f32(1.0))
        s = max(f32(lmax - lmin), f32(MIN_SCALE))
        inv = f32(lm2 / s)
        x = np.rint((lb - lmin).astype(np.float32) * inv).astype(np.float64) + 1.0
        q = np.clip(x, 1.0, levels - 1.0)
        q[flat[lo:hi] == 0] = 0.0
        codes[lo:hi] = q.astype(np.int64)
        scale[b], minlog[b] = s, lmin
    dt = torch.uint8 if levels <= 256 else torch.int16
    out = codes.astype(np.uint8) if levels <= 256 else codes.astype(np.uint16).view(np.int16)
    return torch.from_numpy(out.copy()).to(dt), torch.from_numpy(scale), torch.from_numpy(minlog), pad


def al_dequantize_kernel(q: torch.Tensor, scale: torch.Tensor, min_log: torch.Tensor, numel: int):
    """dequant_v (kernels.cu:318-320; AL16 kernels.cu:442): 0 for q = 0, else
    2^(((q-1) * fp32(1/(levels-2))) * s + min_log) rounded to fp32 at each step; the
    power correctly rounded."""
    qf = q.reshape(-1)
    levels = 256 if qf.dtype == torch.uint8 else 65536
    x = qf.numpy().astype(np.int64)
    if levels == 65536:
        x = np.where(x < 0, x + 65536, x)
    bs = x.size // scale.numel()
    s = np.repeat(scale.numpy().astype(np.float32), bs)
    lm = np.repeat(min_log.numpy().astype(np.float32), bs)
    inv = np.float32(1.0) / np.float32(levels - 2)
    arg = ((np.float32(x - 1).astype(np.float32) * inv).astype(np.float32) * s).astype(np.float32) + lm
    out = np.exp2(arg.astype(np.float64)).astype(np.float32)
    out[x == 0] = 0.0
    return torch.from_numpy(out[:numel].copy())


# --------------------------------------------------------------------------
# Momentum codecs                           optimizer.py:416-532
# --------------------------------------------------------------------------
def dynamic_map(total_bits: int) -> torch.Tensor:
    """Signed dynamic (Dettmers) codebook, optimizer.py:416-441.

    8-bit: 7 exponent levels; 4-bit: 3 exponent levels.  For exponent level i the
    entries are +/-10^(i-(E-1)) * midpoints of linspace(0.1, 1, 2^(i+N-E)+1)
    (N = total_bits-1), then the extra +/-midpoints of linspace(0.1,1,2^(N-E)+1)
    when N > E, then 0 and 1.0, sorted ascending.
    """
    e_bits = 7 if total_bits == 8 else 3
    n_bits = total_bits - 1
    vals = []
    for i in range(e_bits):
        k = int(2 ** (i + n_bits - e_bits) + 1)
        b = torch.linspace(0.1, 1, k, dtype=torch.float32)
        mids = ((b[:-1] + b[1:]) / 2.0)
        mag = 10 ** (-(e_bits - 1) + i)
        vals += (mag * mids).tolist()
        vals += (-mag * mids).tolist()
    extra = 2 ** (n_bits - e_bits) - 1
    if extra > 0:
        b = torch.linspace(0.1, 1, extra + 1, dtype=torch.float32)
        mids = (b[:-1] + b[1:]) / 2.0
        vals += mids.tolist()
        vals += (-mids).tolist()
    vals += [0, 1.0]
    assert len(vals) == 2 ** total_bits
    vals.sort()
    return torch.tensor(vals, dtype=torch.float32)


def _pad_blocks(m: torch.Tensor, block_size: int):
    flat = m.reshape(-1)
    pad = (block_size - flat.numel() % block_size) % block_size
    if pad:
        flat = torch.nn.functional.pad(flat, (0, pad))
    return flat.view(-1, block_size)


def _pack_nibbles(codes2d: torch.Tensor) -> torch.Tensor:
    """Even element in the high nibble (optimizer.py:477-479, 513-515)."""
    hi = codes2d[:, 0::2].to(torch.uint8)
    lo = codes2d[:, 1::2].to(torch.uint8)
    return ((hi << 4) | lo).reshape(-1)


def _unpack_nibbles(q: torch.Tensor) -> torch.Tensor:
    hi = (q >> 4) & 0x0F
    lo = q & 0x0F
    return torch.stack((hi, lo), dim=-1).reshape(-1)


def uf_quantize(m: torch.Tensor, block_size: int, bits: int):
    """UF8/UF4 absmax codec, optimizer.py:504-519.

    absmax = max(|m|, 1e-12) per block; UF8 q = clamp(round(m/absmax*128),-128,127)+128;
    UF4 q = clamp(round(m/absmax*8),-8,7)+8 packed two per byte.
    """
    blocks = _pad_blocks(m, block_size)
    amax = blocks.abs().amax(dim=1, keepdim=True).clamp(min=1e-12)
    if bits == 4:
        q = (torch.round(blocks / amax * 8.0).clamp(-8, 7) + 8).to(torch.uint8)
        return _pack_nibbles(q), amax.squeeze(-1)
    q = (torch.round(blocks / amax * 128.0).clamp(-128, 127) + 128).to(torch.uint8)
    return q.reshape(-1), amax.squeeze(-1)


def uf_dequantize(q: torch.Tensor, scale: torch.Tensor, numel: int, block_size: int, bits: int):
    """optimizer.py:522-532: (q-zero) * (scale/divisor), divisor 8 (UF4) or 128 (UF8)."""
    if bits == 4:
        x = _unpack_nibbles(q).to(torch.float32) - 8.0
        div = 8.0
    else:
        x = q.to(torch.float32) - 128.0
        div = 128.0
    out = (x.view(-1, block_size) * (scale.unsqueeze(-1) / div)).reshape(-1)
    return out[:numel]


def d_quantize(m: torch.Tensor, block_size: int, bits: int):
    """Dynamic-map codec, optimizer.py:454-480.

    Normalise by block absmax, take the nearest codebook entry (searchsorted,
    ties keep the upper index), then step one index toward the value's sign when
    the chosen entry has the opposite sign.
    """
    qmap = dynamic_map(bits)
    blocks = _pad_blocks(m, block_size)
    amax = blocks.abs().amax(dim=1, keepdim=True).clamp(min=1e-12)
    x = (blocks / amax).reshape(-1)
    idx = torch.searchsorted(qmap, x).clamp(0, len(qmap) - 1)
    prev = (idx - 1).clamp(0)
    d_cur = (x - qmap[idx]).abs()
    d_prev = (x - qmap[prev]).abs()
    idx = torch.where(d_prev < d_cur, prev, idx)
    s_x = x.sign()
    s_q = qmap[idx].sign()
    wrong = (s_x != s_q) & (s_x != 0)
    idx = torch.where(wrong & (s_x > 0) & (idx < len(qmap) - 1), idx + 1, idx)
    idx = torch.where(wrong & (s_x < 0) & (idx > 0), idx - 1, idx)
    if bits == 8:
        return idx.to(torch.uint8), amax.squeeze(-1)
    return _pack_nibbles(idx.view(-1, block_size)), amax.squeeze(-1)


def d_dequantize(q: torch.Tensor, scale: torch.Tensor, numel: int, block_size: int, bits: int):
    """optimizer.py:483-499 (CPU branch): qmap[q] * scale."""
    qmap = dynamic_map(bits)
    ids = q.long() if bits == 8 else _unpack_nibbles(q).long()
    vals = qmap[ids].view(-1, block_size)
    return (vals * scale.unsqueeze(-1)).reshape(-1)[:numel]


def m_bits_of(mqt: str) -> int:
    return 4 if mqt in ("uf4", "d4") else 8


def m_quantize(m, mqt, block_size):
    if mqt in ("uf4", "uf8"):
        return uf_quantize(m, block_size, m_bits_of(mqt))
    return d_quantize(m, block_size, m_bits_of(mqt))


def m_dequantize(q, scale, numel, block_size, mqt):
    if mqt in ("uf4", "uf8"):
        return uf_dequantize(q, scale, numel, block_size, m_bits_of(mqt))
    return d_dequantize(q, scale, numel, block_size, m_bits_of(mqt))


# --------------------------------------------------------------------------
# State layout                              optimizer.py:389-401, 574-590
# --------------------------------------------------------------------------
def init_v(st, prefix, shape, block_size, vqt, quantize):
    numel = math.prod(shape)
    if not quantize or vqt == "fp32":
        st[prefix] = torch.zeros(shape, dtype=torch.float32)
        return
    pad = (block_size - numel % block_size) % block_size
    nb = (numel + pad) // block_size
    st[f"{prefix}_q"] = torch.zeros(numel + pad, dtype=torch.uint8 if vqt == "al8" else torch.int16)
    st[f"{prefix}_scale"] = torch.ones(nb, dtype=torch.float32)
    st[f"{prefix}_min_log"] = torch.zeros(nb, dtype=torch.float32)
    st[f"{prefix}_shape"] = tuple(shape)
    st[f"{prefix}_pad"] = pad


def init_m(st, numel, shape, m_block, mqt, quantize):
    if not quantize or mqt == "fp32":
        st["m"] = torch.zeros(shape, dtype=torch.float32)
        st["m_quant_type"] = "fp32"
        return
    padded = ((numel + m_block - 1) // m_block) * m_block
    if m_bits_of(mqt) == 4:
        st["m_q"] = torch.full((padded // 2,), 0x88 if mqt == "uf4" else 0x77, dtype=torch.uint8)
    else:
        st["m_q"] = torch.full((padded,), 128 if mqt == "uf8" else 127, dtype=torch.uint8)
    st["m_scale"] = torch.ones(padded // m_block, dtype=torch.float32)
    st["m_block_size"] = m_block
    st["m_quant_type"] = mqt


def deq_v(st, prefix, krule=False):
    q = st[f"{prefix}_q"]
    shape = st[f"{prefix}_shape"]
    numel = math.prod(shape)
    deq = al_dequantize_kernel if krule else al_dequantize
    return deq(q, st[f"{prefix}_scale"], st[f"{prefix}_min_log"], numel).view(shape)


def quant_v(st, prefix, v, block_size, vqt, floor=-126.0, krule=False):
    qfn = al_quantize_kernel if krule else al_quantize
    q, s, ml, pad = qfn(v, block_size, floor, 256 if vqt == "al8" else 65536)
    st[f"{prefix}_q"], st[f"{prefix}_scale"], st[f"{prefix}_min_log"] = q, s, ml
    st[f"{prefix}_shape"], st[f"{prefix}_pad"] = tuple(v.shape), pad


# --------------------------------------------------------------------------
# Update helpers                            optimizer.py:690-881
# --------------------------------------------------------------------------
def m_ema(st, x, beta1, mqt, m_block, quantize):
    """``_get_updated_m`` / ``_m_ema_pytorch`` (optimizer.py:690-711)."""
    if quantize and mqt != "fp32":
        if "m_q" in st:
            m = m_dequantize(st["m_q"], st["m_scale"], x.numel(), m_block, mqt).view(x.shape)
        else:
            m = torch.zeros_like(x)
        m.lerp_(x, 1.0 - beta1)
        st["m_q"], st["m_scale"] = m_quantize(m, mqt, m_block)
        return m
    if "m" not in st:
        st["m"] = torch.zeros_like(x)
    st["m"].lerp_(x, 1.0 - beta1)
    return st["m"]


def fira_scale(st, curr_norm, margin, key="fira_prev_norm"):
    """Norm-growth limiter, optimizer.py:760-782 (PyTorch branch)."""
    curr = torch.where(torch.isfinite(curr_norm), curr_norm, torch.zeros_like(curr_norm))
    prev = st.get(key)
    if prev is None:
        st[key] = curr
        return torch.tensor(1.0, dtype=torch.float32)
    if not torch.is_tensor(prev):
        prev = torch.tensor(prev, dtype=torch.float32)
    reset = prev < 1e-6
    ratio = curr / (prev + 1e-8)
    lim = torch.clamp_min(ratio, 1.0 + margin) / (1.0 + margin)
    fs = torch.where(reset, torch.ones_like(curr), 1.0 / lim)
    st[key] = torch.where(reset, curr, curr * fs)
    return fs


def _one():
    return torch.tensor(1.0)


def apply_update(p, u, alpha, st, d, fira, margin):
    """``_apply_update_pytorch`` without SR (optimizer.py:866-875) incl. Fira
    (optimizer.py:796-810) and the RMS clip denominator (optimizer.py:859-863)."""
    if fira:
        norm = _vnorm(u)
        if not torch.isfinite(norm):
            u.zero_()
            norm.zero_()
        fs = fira_scale(st, norm, margin)
        u = u * fs
        denom = torch.clamp(norm / (math.sqrt(u.numel()) * d), min=1.0) if d > 0 else _one()
    elif d > 0:
        denom = torch.clamp(_vnorm(u) / (math.sqrt(u.numel()) * d), min=1.0)
    else:
        denom = _one()
    p.add_(u, alpha=-alpha / denom)


def compute_alpha(p, lr, step, relative_step, scale_parameter, eps2):
    """optimizer.py:832-856 for a float learning rate."""
    if relative_step:
        rho = torch.tensor(min(lr, 1.0 / math.sqrt(step)), dtype=torch.float32)
    else:
        rho = torch.tensor(lr, dtype=torch.float32)
    if scale_parameter:
        rms = _vnorm(p, f32=True) / math.sqrt(p.numel())
        return torch.clamp(rms, min=eps2) * rho, rho
    return rho, rho


# --------------------------------------------------------------------------
# The optimizer step (fallback branches)    optimizer.py:1618-2552
# --------------------------------------------------------------------------
DEFAULTS = dict(lr=1e-2, beta1=None, beta2=None, beta2_decay=-0.8, beta3=None, eps_came=1e-16,
                eps=(1e-30, 1e-3), weight_decay=0.0, d=1.0, maximize=False, relative_step=True,
                scale_parameter=True, factored=True, quantize=True, block_size=2048,
                m_block_size=256, m_quant_type="uf8", v_quant_type="al8", c_quant_type=None,
                min_8bit_size=4096, scale_weight_decay=True, enable_fira_for_adafactor=False,
                fira_margin=0.01, lag_norm=False, momentum_only_1d=None, bias_correction=None,
                apollo_rank=0, apollo_update_proj_gap=200, apollo_scale_type="channel",
                apollo_scale=1.0, apollo_scale_front=False, apollo_eps=1e-6, apollo_factorize=False,
                apollo_cache_proj=False, enable_fira_for_apollo=True,
                stochastic_round_writeback=False, al_refit_rule="fallback")

ADV_DEFAULT = 0xF   # optimizer.py:26


def stable_randn(shape, seed, device=None, dtype=torch.float32):
    """optimizer.py:139-149 (the tests install inputs.make_proj in its place)."""
    dev = device if device is not None else torch.device("cpu")
    gen = torch.Generator(device=dev).manual_seed(seed)
    return torch.randn(shape, generator=gen, device=dev, dtype=dtype)


def next_seed(seed: int, adv: int = ADV_DEFAULT) -> int:
    """optimizer.py:152-155."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, torch.iinfo(torch.int64).max, (adv,), generator=gen).tolist()[-1]


def apollo_proj_T(st, shape, step, cache):
    """_get_apollo_proj_matrix, optimizer.py:2557-2584."""
    rank, gap = int(st["apollo_rank"]), int(st["apollo_update_proj_gap"])
    last = int(st.get("last_proj_step", -gap))
    refresh = (step - last) >= gap
    if not refresh and cache and st.get("apollo_proj_matrix_T") is not None:
        return st["apollo_proj_matrix_T"]
    if refresh:
        st["current_proj_seed"] = int(st["apollo_seed"])
        st["apollo_seed"] = next_seed(st["current_proj_seed"])
        st["last_proj_step"] = step
    R, C = shape[-2], shape[-1]
    m_shape = (rank, C) if R >= C else (R, rank)
    seed = st.get("current_proj_seed", st["apollo_seed"])
    proj = stable_randn(m_shape, seed=seed, device=torch.device("cpu"), dtype=torch.float32) / math.sqrt(rank)
    proj_T = proj.T.to(torch.float32).contiguous()
    if cache:
        st["apollo_proj_matrix_T"] = proj_T
    return proj_T


class OracleOptimizer:
    """Single-group restatement of ``Adafactor8Bit.step`` on the CPU path.

    Covers SGD, the full-rank 1-D path (quantised and fp32 state) and the
    factored 2-D path including CAME, with Fira, RMS clipping, weight decay and
    bias correction.  State keys and dtypes are the reference's.
    """

    def __init__(self, params, **kw):
        self.params = list(params)
        self.hp = dict(DEFAULTS)
        for k, v in kw.items():
            if k not in self.hp:
                raise KeyError(k)
            self.hp[k] = v
        self.state: Dict[Any, Dict[str, Any]] = {id(p): {} for p in self.params}
        self.apollo_seed_counter = 1

    # optimizer.py:1618-1743 (fresh-state branch only)
    def _init_state(self, p, st):
        h = self.hp
        use_quant = h["quantize"] and p.numel() >= h["min_8bit_size"]
        vqt, mqt = h["v_quant_type"], h["m_quant_type"]
        cqt = h["c_quant_type"] or vqt
        st["step"] = 0
        st["is_quantized"] = use_quant
        st["block_size"] = h["block_size"]
        st["v_quant_type"] = vqt
        st["c_quant_type"] = cqt
        sgd = h["beta2"] is None and h["beta2_decay"] is None
        if sgd:
            if h["beta1"] is not None:
                init_m(st, p.numel(), p.shape, h["m_block_size"], mqt, use_quant)
            return
        if h["apollo_rank"] > 0 and p.dim() >= 2:   # optimizer.py:1725-1745
            gap = h["apollo_update_proj_gap"]
            st["apollo_seed"] = self.apollo_seed_counter
            self.apollo_seed_counter += 1
            st["apollo_rank"] = h["apollo_rank"]
            st["apollo_factorize"] = h["apollo_factorize"]
            st["beta3"] = h["beta3"]
            st["apollo_update_proj_gap"] = gap
            st["last_proj_step"] = -gap
            st["apollo_proj_matrix_T"] = None
            st["m_quant_type"] = mqt
            for k in ("v_low_q", "v_low_scale", "v_low_min_log", "v_low_shape", "v_low_pad", "v_low"):
                st[k] = None
            if h["beta3"] is not None:   # optimizer.py:1740-1748
                names = ("conf_row_low", "conf_col_low") if h["apollo_factorize"] else ("res_low",)
                for nm in names:
                    for suf in ("_q", "_scale", "_min_log", "_shape", "_pad"):
                        st[nm + suf] = None
                for nm in names:
                    st[nm] = None
            return
        if p.dim() >= 2 and h["factored"]:
            R, C = p.shape[-2], p.shape[-1]
            rs = list(p.shape[:-2]) + [R, 1]
            cs = list(p.shape[:-2]) + [1, C]
            init_v(st, "row_var", rs, h["block_size"], vqt, use_quant)
            init_v(st, "col_var", cs, h["block_size"], vqt, use_quant)
            if h["beta1"] is not None:
                init_m(st, p.numel(), p.shape, h["m_block_size"], mqt, use_quant)
            if h["beta3"] is not None:
                init_v(st, "conf_row", rs, h["block_size"], cqt, use_quant)
                init_v(st, "conf_col", cs, h["block_size"], cqt, use_quant)
        else:
            init_v(st, "variance", p.shape, h["block_size"], vqt, use_quant)
            if h["beta1"] is not None:
                init_m(st, p.numel(), p.shape, h["m_block_size"], mqt, use_quant)

    def _update_apollo(self, p, grad, st):
        apollo_update(self, p, grad, st)

    @torch.no_grad()
    def step(self):
        for p in self.params:
            if p.grad is None:
                continue
            st = self.state[id(p)]
            if not st:
                self._init_state(p, st)
            if self.hp["apollo_rank"] > 0 and "apollo_seed" in st:
                self._update_apollo(p, p.grad, st)
            else:
                self._update(p, p.grad, st)

    def _update(self, p, grad, st):  # optimizer.py:1944-2552, CPU branches
        h = self.hp
        beta1, beta2, beta2_decay, beta3 = h["beta1"], h["beta2"], h["beta2_decay"], h["beta3"]
        d, lr = h["d"], h["lr"]
        eps1, eps2 = h["eps"]
        eps1 = 1e-30 if eps1 is None else eps1
        fira, margin = h["enable_fira_for_adafactor"], h["fira_margin"]
        sgd = beta2 is None and beta2_decay is None
        full_rank = grad.dim() < 2 or not h["factored"] or sgd
        eps_sq = max(eps1 * eps1, LOG_QUANT_FLOOR)
        adam_denom = (not h["factored"]) and beta2 is not None and beta3 is None
        eps_d = eps1 if adam_denom else 0.0
        eps_g = eps1 if not adam_denom else 0.0
        mom_only = h["momentum_only_1d"]
        if mom_only is None:
            mom_only = not adam_denom
        g = grad.contiguous()
        if h["maximize"]:
            g = g.neg()
        quant = st.get("is_quantized", False)
        vqt = st.get("v_quant_type", "al8")
        cqt = st.get("c_quant_type", vqt)
        bs = st.get("block_size", h["block_size"])
        mqt = st.get("m_quant_type", "uf8") if beta1 is not None else "uf8"
        mbs = st.get("m_block_size", h["m_block_size"]) if beta1 is not None else 0
        g32 = g.float()
        if g32.data_ptr() == g.data_ptr():
            g32 = g32.clone()

        step = st["step"] + 1
        st["step"] = step
        if sgd:
            bv = 0.0
        elif beta2 is not None:
            bv = 1.0 - beta2
        else:
            bv = math.pow(step, beta2_decay)
        alpha, rho = compute_alpha(p, lr, step, h["relative_step"], h["scale_parameter"], eps2)
        if beta1 is not None and not h["relative_step"] and not sgd:
            bc_on = adam_denom if h["bias_correction"] is None else h["bias_correction"]
            if bc_on:
                bc1 = 1.0 - beta1 ** step
                if beta2 is not None:
                    bc2 = 1.0 - beta2 ** step
                    alpha = alpha * (math.sqrt(bc2) / bc1)
                    if adam_denom:
                        eps_d = eps1 * math.sqrt(bc2)
                else:
                    alpha = alpha / bc1
        if h["weight_decay"] != 0:
            mult = alpha if h["scale_weight_decay"] else rho
            p.mul_(1.0 - (mult * h["weight_decay"]))

        if sgd:  # optimizer.py:2052-2077
            if beta1 is not None:
                upd = m_ema(st, g32, beta1, mqt, mbs, quant)
                upd = upd / (1.0 - beta1)
            else:
                upd = g32
            apply_update(p, upd, alpha, st, d, fira, margin)
            return

        if full_rank:  # optimizer.py:2082-2190
            if quant and vqt != "fp32":
                # al_refit_rule "kernel": the V refit and codes of the fused 1-D CUDA
                # kernels (floor log_eps_sq, kernels.cu:772-774); "fallback": the CPU rule
                kr = h.get("al_refit_rule", "fallback") == "kernel" and not sgd
                gsq = g32.square().add_(eps_g)
                var = deq_v(st, "variance", kr)
                var.lerp_(gsq, bv)
                if kr:
                    quant_v(st, "variance", var, bs, vqt, floor=kernel_floor(eps1), krule=True)
                else:
                    quant_v(st, "variance", var, bs, vqt)
            else:
                var = st["variance"]
                var.mul_(1.0 - bv).addcmul_(g32, g32, value=bv)
                if eps_g > 0.0:
                    var.add_(bv * eps_g)
            self._update_1d(p, g32, var, st, alpha, d, fira, margin, beta1, mqt, mbs, quant,
                            mom_only, adam_denom, eps_d, eps_sq)
            return

        # factored 2-D path, optimizer.py:2198-2552 (fallback branches)
        gsq = g32.square()
        row_mean = _mean(gsq, -1).add_(eps1)
        col_mean = _mean(gsq, -2).add_(eps1)
        if quant and vqt != "fp32":
            row_var = deq_v(st, "row_var")
            col_var = deq_v(st, "col_var")
            row_var.lerp_(row_mean, bv)
            col_var.lerp_(col_mean, bv)
            rmv = _mean(row_var, -2).clamp(min=eps1)
            quant_v(st, "row_var", row_var, bs, vqt)
            quant_v(st, "col_var", col_var, bs, vqt)
        else:
            row_var, col_var = st["row_var"], st["col_var"]
            row_var.lerp_(row_mean, bv)
            col_var.lerp_(col_mean, bv)
            rmv = _mean(row_var, -2).clamp(min=eps1)
        inv_row = (row_var / rmv).rsqrt_()
        inv_col = col_var.rsqrt()
        self._update_2d(p, g32, st, alpha, d, fira, margin, beta1, beta3, h["eps_came"], eps1,
                        mqt, mbs, quant, inv_row, inv_col, bs, vqt, cqt)

    @staticmethod
    def _update_1d(p, g32, var, st, alpha, d, fira, margin, beta1, mqt, mbs, quant, mom_only,
                   adam_denom, eps_d, eps_sq):  # optimizer.py:886-917
        temp_m = quant and mqt != "fp32"
        if beta1 is not None:
            if mom_only:
                u = g32 * var.clamp(min=eps_sq).rsqrt()
                if d > 0:
                    rms = _vnorm(u) / math.sqrt(u.numel())
                    u.div_(torch.clamp(rms / d, min=1.0))
                m = m_ema(st, u, beta1, mqt, mbs, quant)
                apply_update(p, m, alpha, st, 0, fira, margin)
            else:
                m = m_ema(st, g32, beta1, mqt, mbs, quant)
                if adam_denom:
                    inv = 1.0 / (var.sqrt() + eps_d)
                else:
                    inv = var.clamp(min=eps_sq).rsqrt()
                u = m.mul_(inv) if temp_m else m * inv
                apply_update(p, u, alpha, st, d, fira, margin)
        else:
            if adam_denom:
                u = g32 / (var.sqrt() + eps_d)
            else:
                u = g32 * var.clamp(min=eps_sq).rsqrt()
            apply_update(p, u, alpha, st, d, fira, margin)

    @staticmethod
    def _update_2d(p, g32, st, alpha, d, fira, margin, beta1, beta3, eps_came, eps1, mqt, mbs,
                   quant, inv_row, inv_col, bs, vqt, cqt):  # optimizer.py:920-970
        cqt = cqt or vqt
        temp_m = quant and mqt != "fp32"
        if beta3 is not None and beta1 is not None:
            u = g32.mul_(inv_row).mul_(inv_col)
            if d > 0:
                rms = _vnorm(u) / math.sqrt(u.numel())
                u.div_(torch.clamp(rms / d, min=1.0))
            m = m_ema(st, u, beta1, mqt, mbs, quant)
            res = u.sub_(m).square_().add_(eps_came)
            res_row = _mean(res, -1)
            res_col = _mean(res, -2)
            if quant and cqt != "fp32":
                c_row = deq_v(st, "conf_row")
                c_col = deq_v(st, "conf_col")
            else:
                c_row, c_col = st["conf_row"], st["conf_col"]
            c_row.lerp_(res_row, 1.0 - beta3)
            c_col.lerp_(res_col, 1.0 - beta3)
            if quant and cqt != "fp32":
                quant_v(st, "conf_row", c_row, bs, cqt)
                quant_v(st, "conf_col", c_col, bs, cqt)
            crm = _mean(c_row, -2).clamp(min=eps1)
            icr = (c_row / crm).rsqrt_()
            icc = c_col.rsqrt()
            if temp_m:
                m.mul_(icr).mul_(icc)
                apply_update(p, m, alpha, st, 0, fira, margin)
            else:
                apply_update(p, m.mul(icr).mul_(icc), alpha, st, 0, fira, margin)
        elif beta1 is not None:
            m = m_ema(st, g32, beta1, mqt, mbs, quant)
            if temp_m:
                m.mul_(inv_row).mul_(inv_col)
                apply_update(p, m, alpha, st, d, fira, margin)
            else:
                apply_update(p, m.mul(inv_row).mul_(inv_col), alpha, st, d, fira, margin)
        else:
            u = g32 * inv_row
            u.mul_(inv_col)
            apply_update(p, u, alpha, st, d, fira, margin)


def m_ema_prefix(st, x, beta1, mqt, m_block, prefix):
    """``_m_ema_pytorch`` with a state prefix (optimizer.py:690-700)."""
    qk, sk = f"{prefix}_q", f"{prefix}_scale"
    if qk in st and st[qk] is not None:
        m = m_dequantize(st[qk], st[sk], x.numel(), m_block, mqt).view(x.shape)
    else:
        m = torch.zeros_like(x)
    m.lerp_(x, 1.0 - beta1)
    st[qk], st[sk] = m_quantize(m, mqt, m_block)
    return m


def init_m_prefix(st, numel, m_block, mqt, prefix):
    """``_m_init_state`` with a prefix (optimizer.py:574-590), quantised codecs."""
    padded = ((numel + m_block - 1) // m_block) * m_block
    if m_bits_of(mqt) == 4:
        st[f"{prefix}_q"] = torch.full((padded // 2,), 0x88 if mqt == "uf4" else 0x77, dtype=torch.uint8)
    else:
        st[f"{prefix}_q"] = torch.full((padded,), 128 if mqt == "uf8" else 127, dtype=torch.uint8)
    st[f"{prefix}_scale"] = torch.ones(padded // m_block, dtype=torch.float32)
    st["m_block_size"] = m_block
    st["m_quant_type"] = mqt


@torch.no_grad()
def apollo_update(opt, p, grad, st):
    """``_update_param_apollo`` (optimizer.py:2587-3084), CPU branches (the
    reference with no CUDA module), deterministic writeback: plain, factorised
    (apollo_factorize) and CAME (beta3) low-rank updates."""
    h = opt.hp
    beta1, beta2, beta2_decay = h["beta1"], h["beta2"], h["beta2_decay"]
    if h["stochastic_round_writeback"] and p.dtype in (torch.bfloat16, torch.float16):
        raise NotImplementedError("oracle: SR writeback (its CPU RNG stream is not the GPU's)")
    d, lr = h["d"], h["lr"]
    eps2 = h["eps"][1]
    gw = grad.float()
    if gw.data_ptr() == grad.data_ptr():
        gw = gw.clone()
    if h["maximize"]:
        gw.neg_()
    torch.nan_to_num_(gw, nan=0.0, posinf=0.0, neginf=0.0)
    pw = p.data
    if pw.dim() > 2:
        pw = pw.reshape(pw.shape[0], -1)
        gw = gw.reshape(gw.shape[0], -1)
    step = st["step"] + 1
    st["step"] = step
    vqt = st.get("v_quant_type", "al8")
    mqt = st.get("m_quant_type", "uf8") if beta1 is not None else "uf8"
    bv = 1.0 - beta2 if beta2 is not None else math.pow(step, beta2_decay)
    alpha, rho = compute_alpha(pw, lr, step, h["relative_step"], h["scale_parameter"], eps2)
    projT = apollo_proj_T(st, gw.shape, step, h["apollo_cache_proj"])
    R, C = gw.shape[-2], gw.shape[-1]
    right = R >= C
    fira = h["enable_fira_for_apollo"]
    need_norm = fira or d > 0
    hook = getattr(opt, "glow_hook", None)
    if hook is not None:   # a test injects the projection output of the implementation under test
        glow = hook(p, gw, projT).float()
    else:
        glow = (torch.matmul(gw, projT) if right else torch.matmul(projT, gw)).float()

    first = st.get("v_low_q") is None and st.get("v_low") is None
    quant = st.get("is_quantized", False)
    bs = st.get("block_size", h["block_size"])
    aeps = h["apollo_eps"]
    eps_sq = max(aeps * aeps, LOG_QUANT_FLOOR)
    lf = math.log2(eps_sq)
    if h["apollo_factorize"]:
        upd = apollo_low_factorised(st, glow, h, bv, beta1, mqt, quant)
    else:
        upd = _apollo_low_plain(st, glow, h, bv, beta1, mqt, quant, first, bs, eps_sq, lf)
    _apollo_finish(opt, st, pw, gw, glow, upd, alpha, rho, step, right, need_norm)


def _apollo_low_plain(st, glow, h, bv, beta1, mqt, quant, first, bs, eps_sq, lf):
    """Non-factorised low-rank V EMA and update (optimizer.py:2759-2951, CPU
    branches); with beta3 the CAME residual path of optimizer.py:2800-2896."""
    vqt = st.get("v_quant_type", "al8")
    aeps = h["apollo_eps"]
    if first:
        vinit = glow.flatten().square() * bv
        if quant and vqt != "fp32":
            quant_v(st, "v_low", vinit, bs, vqt)
        else:
            st["v_low"] = vinit
        vdeq = vinit
    elif quant and vqt != "fp32":
        vd = deq_v(st, "v_low")
        vd.lerp_(glow.flatten().square(), bv)
        quant_v(st, "v_low", vd, bs, vqt, floor=lf)
        vdeq = vd
    else:
        st["v_low"].lerp_(glow.flatten().square(), bv)
        vdeq = st["v_low"]

    if h["beta3"] is not None and beta1 is not None:
        return _apollo_came_low(st, glow, vdeq, h, beta1, mqt, quant, bs, eps_sq)
    if beta1 is not None:
        if not quant or mqt == "fp32":
            if st.get("m_low") is None:
                st["m_low"] = torch.zeros_like(glow)
            st["m_low"].lerp_(glow, 1.0 - beta1)
            mdeq = st["m_low"]
        else:
            mbs = st.get("m_block_size", h["m_block_size"])
            if st.get("m_low_q") is None:
                init_m_prefix(st, glow.numel(), mbs, mqt, "m_low")
            mdeq = m_ema_prefix(st, glow, beta1, mqt, mbs, "m_low")
        return mdeq / (torch.sqrt(vdeq.view_as(glow)) + aeps)
    return glow / (torch.sqrt(vdeq).view_as(glow) + aeps)


def apollo_m_ema(st, x, beta1, mqt, mbs, quant, prefix="m_low"):
    """``_apollo_m_ema`` (optimizer.py:714-729) without the CUDA module: fp32 m
    through lerp_, codes through ``_m_ema_pytorch``."""
    if not quant or mqt == "fp32":
        if st.get(prefix) is None:
            st[prefix] = torch.zeros_like(x)
        st[prefix].lerp_(x, 1.0 - beta1)
        return st[prefix]
    if st.get(f"{prefix}_q") is None:
        init_m_prefix(st, x.numel(), mbs, mqt, prefix)
    return m_ema_prefix(st, x, beta1, mqt, mbs, prefix)


def _clip_rms(u, d):
    """``U.div_(clamp(rms(U) / d, min=1))`` (optimizer.py:2715-2717, 2869-2871)."""
    if d > 0:
        rms = _vnorm(u) / math.sqrt(u.numel())
        u.div_(torch.clamp(rms / d, min=1.0))
    return u


def _apollo_came_low(st, glow, vdeq, h, beta1, mqt, quant, bs, eps_sq):
    """CAME on the low-rank gradient, non-factorised (optimizer.py:2800-2896, the
    branch taken without the CUDA module): U = g / sqrt(max(v, eps^2)) with RMS
    clipping, m EMA of U, residual EMA (beta3) of (U - m)^2 + eps_came in fp32 or
    AL codes (read back decoded), u = m / sqrt(max(res, eps^2))."""
    beta3 = h["beta3"]
    cqt = st.get("c_quant_type", st.get("v_quant_type", "al8"))
    mbs = st.get("m_block_size", h["m_block_size"])
    if st.get("res_low_q") is None and st.get("res_low") is None:
        if quant and cqt != "fp32":
            init_v(st, "res_low", tuple(glow.shape), bs, cqt, True)
        else:
            st["res_low"] = torch.zeros_like(glow)
    u = glow * vdeq.view_as(glow).clamp(min=eps_sq).rsqrt()
    _clip_rms(u, h["d"])
    m = apollo_m_ema(st, u, beta1, mqt, mbs, quant)
    res = u.sub(m).square_().add_(h["eps_came"])
    del u
    if quant and cqt != "fp32":
        rd = deq_v(st, "res_low")
        rd.lerp_(res, 1.0 - beta3)
        quant_v(st, "res_low", rd, bs, cqt)
        rd = deq_v(st, "res_low")
    else:
        st["res_low"].lerp_(res, 1.0 - beta3)
        rd = st["res_low"]
    return m * rd.view_as(glow).clamp(min=eps_sq).rsqrt()


def apollo_low_factorised(st, glow, h, bv, beta1, mqt, quant):
    """Factorised low-rank second moment (optimizer.py:2689-2758): row / column
    means of g^2 (+ FLT_MIN) into fp32 EMAs, v = r c / max(mean r, eps);
    u = x / (sqrt(v) + eps) with x = g or its momentum; with beta3 the CAME form
    with row / column confidence EMAs of the residual."""
    aeps, beta3 = h["apollo_eps"], h["beta3"]
    gsq = glow.square()
    row_mean = _mean(gsq, -1).add_(LOG_QUANT_FLOOR)
    col_mean = _mean(gsq, -2).add_(LOG_QUANT_FLOOR)
    del gsq
    if "row_var_low" not in st:
        st["row_var_low"] = row_mean * bv
        st["col_var_low"] = col_mean * bv
    else:
        st["row_var_low"].mul_(1.0 - bv).add_(row_mean, alpha=bv)
        st["col_var_low"].mul_(1.0 - bv).add_(col_mean, alpha=bv)
    rv, cv = st["row_var_low"], st["col_var_low"]
    v_est = rv.mul(cv).div_(_mean(rv, -2).clamp_(min=aeps))
    mbs = st.get("m_block_size", h["m_block_size"])
    if beta1 is None:
        return glow / (torch.sqrt(v_est) + aeps)
    if beta3 is None:
        m = apollo_m_ema(st, glow, beta1, mqt, mbs, quant)
        return m / (torch.sqrt(v_est) + aeps)
    rmv = _mean(rv, -2).clamp(min=LOG_QUANT_FLOOR)
    inv_row = (rv / rmv).rsqrt_()
    inv_col = cv.rsqrt()
    u = glow.mul(inv_row).mul_(inv_col)
    _clip_rms(u, h["d"])
    m = apollo_m_ema(st, u, beta1, mqt, mbs, quant)
    res = u.sub(m).square_().add_(h["eps_came"])
    del u
    res_row = _mean(res, -1)
    res_col = _mean(res, -2)
    bs = st.get("block_size", h["block_size"])
    cqt = st.get("c_quant_type", st.get("v_quant_type", "al8"))
    if quant and cqt != "fp32":
        if st.get("conf_row_low_q") is None:
            init_v(st, "conf_row_low", tuple(res_row.shape), bs, cqt, True)
            init_v(st, "conf_col_low", tuple(res_col.shape), bs, cqt, True)
        c_row = deq_v(st, "conf_row_low")
        c_col = deq_v(st, "conf_col_low")
        c_row.lerp_(res_row, 1.0 - beta3)
        c_col.lerp_(res_col, 1.0 - beta3)
        quant_v(st, "conf_row_low", c_row, bs, cqt)
        quant_v(st, "conf_col_low", c_col, bs, cqt)
    else:
        if st.get("conf_row_low") is None:
            st["conf_row_low"] = torch.zeros_like(res_row)
            st["conf_col_low"] = torch.zeros_like(res_col)
        st["conf_row_low"].lerp_(res_row, 1.0 - beta3)
        st["conf_col_low"].lerp_(res_col, 1.0 - beta3)
        c_row, c_col = st["conf_row_low"], st["conf_col_low"]
    crm = _mean(c_row, -2).clamp(min=LOG_QUANT_FLOOR)
    icr = (c_row / crm).rsqrt_()
    icc = c_col.rsqrt()
    return m * icr * icc


def _apollo_finish(opt, st, pw, gw, glow, upd, alpha, rho, step, right, need_norm):
    """Channel / tensor scale, Fira, RMS denominator, bias correction and the
    deterministic writeback of _update_param_apollo (optimizer.py:2995-3084)."""
    h = opt.hp
    beta1, beta2 = h["beta1"], h["beta2"]
    d = h["d"]
    fira = h["enable_fira_for_apollo"]
    channel = h["apollo_scale_type"] == "channel"
    nd = -1 if right else -2
    if channel:
        s = _vnorm(upd, dim=nd) / (_vnorm(glow, dim=nd) + 1e-8)
    else:
        s = _vnorm(upd) / (_vnorm(glow) + 1e-8)
    sv = math.sqrt(h["apollo_scale"])
    if h["apollo_scale_front"]:
        s = s * sv
    if need_norm:
        if channel:
            ngsq = _vnorm(gw, dim=nd, f32=True).square()
            nun = torch.sqrt(_sum(ngsq * s.square()))
        else:
            nun = _vnorm(gw, f32=True) * s
    if fira:
        final = s * fira_scale(st, nun, h["fira_margin"], key="scaled_grad_norm_prev")
    else:
        final = s
    if not h["apollo_scale_front"]:
        final = final * sv
    denom = torch.clamp_min(nun / (math.sqrt(pw.numel()) * d), 1.0) if d > 0 else _one()
    wd = h["weight_decay"]
    decay = (1.0 - ((alpha if h["scale_weight_decay"] else rho) * wd)) if wd != 0 else None
    us = -alpha / denom
    if beta1 is not None and not h["relative_step"]:
        bc_on = True if h["bias_correction"] is None else h["bias_correction"]
        if bc_on:
            bc1 = 1.0 - beta1 ** step
            if beta2 is not None:
                us = us * (math.sqrt(1.0 - beta2 ** step) / bc1)
            else:
                us = us / bc1
    if decay is not None:
        pw.mul_(decay)
    if channel:
        pw.addcmul_(gw, final.to(gw.dtype), value=us)
    else:
        pw.add_(gw, alpha=us * final)


def reference_adamw_block_bytes(numel: int, block_size: int = 2048, m_block: int = 256) -> float:
    """Algorithmic HBM bytes of one fused AdamW UF8/AL8 step over ``numel`` fp32
    params: p r+w, g r, m code r+w, v code r+w, plus per-block metadata r+w."""
    nv = -(-numel // block_size)
    nm = -(-numel // m_block)
    return numel * 16.0 + nv * 16.0 + nm * 8.0
