"""Adafactor8Bit for MI355X: host side of the fused block-quantised optimizer step.

Mirrors the reference optimizer's public interface (adafactor8bit/optimizer.py:
``Adafactor8Bit.__init__`` 1313-1461, ``state_dict``/``load_state_dict``
1463-1553, ``_init_group`` 1618-1864, ``step`` 1866-1938): the same keyword
arguments and validation, the same per-parameter state keys, dtypes, shapes
and padding, the same scalar preparation (bias correction, epsilon, alpha,
weight decay).  The arithmetic of every step runs in the hand-written HIP
library ``libadafactor8bit_amd.so`` (see ``_native.py``); there is no CPU or
PyTorch fallback.  Quantised codes follow the reference's PyTorch numerics
(optimizer.py:299-353, 504-532), so a run matches the reference's CPU results.

Parameters that share a step counter and hyper-parameters are updated by one
multi-tensor launch per group instead of one launch per parameter.
"""
import ctypes
import gc
import logging
import math
from typing import Any, Dict, Iterable, Optional, Tuple, Union

import numpy as np
import torch
from torch import Tensor
from torch.optim import Optimizer

from . import _native as nat
from . import _state as S

__all__ = ["Adafactor8Bit"]

logger = logging.getLogger(__name__)

_LOG_QUANT_FLOOR = 1.17549435e-38
_VALID_M_QUANT_TYPES = ("uf4", "uf8", "d4", "d8", "fp32")
_VALID_V_QUANT_TYPES = ("al8", "al16", "fp32")
_AL_FLOOR = -126.0   # min_log floor of the reference's AL quantiser (optimizer.py:299)

_F32 = np.float32


def _f32(x) -> float:
    return float(_F32(x))


_ADV_DEFAULT = 0xF   # optimizer.py:26


def stable_randn(shape, seed: int, device=None, dtype=torch.float32) -> Tensor:
    """optimizer.py:139-149: a reproducible N(0, 1) tensor from a torch generator
    seeded on ``device`` (the projection matrices of APOLLO)."""
    if device is None:
        device = torch.device("cuda" if torch.cuda.is_available() else "cpu")
    gen = torch.Generator(device=device).manual_seed(seed)
    return torch.randn(shape, generator=gen, device=device, dtype=dtype)


def next_seed(seed: int, adv: int = _ADV_DEFAULT) -> int:
    """optimizer.py:152-155: advance a seed by consuming ``adv`` random integers."""
    gen = torch.Generator().manual_seed(seed)
    return torch.randint(0, torch.iinfo(torch.int64).max, (adv,), generator=gen).tolist()[-1]


class Adafactor8Bit(Optimizer):
    """8-bit Adafactor / AdamW / CAME / RMSprop / SGD with block-quantised states.

    Keyword arguments, defaults and semantics are those of the reference
    ``Adafactor8Bit`` (adafactor8bit/optimizer.py:1176-1360).  ``use_cuda_kernel``
    is accepted for compatibility; the step always runs on the HIP library and
    parameters must live on a ROCm device.

    ``capturable`` (not in the reference; default False) keeps each group's step
    count on the device.  A step then derives its scalars there (a8_step_advance)
    and launches only multi-tensor kernels that read them, so ``step()`` can be
    captured in a CUDA/HIP graph after one eager step and replayed; eager and
    replayed steps run the same kernels on the same inputs, so they give the same
    bits.  APOLLO schedules its projection refreshes on the device (it needs
    apollo_update_proj_gap > 0), and a tensor learning rate is read on the device
    at every replay.  Parameters that need a per-tensor launch raise in this mode.
    ``state_dict()`` reads the device counts and schedules back.  A graph holds the
    addresses of the state and buffers it was captured with: after
    ``load_state_dict()``, ``add_param_group()`` or a parameter's first step, run
    one eager step and capture again instead of replaying the old graph.
    """

    def __init__(
        self,
        params: Iterable[Union[Tensor, Dict[str, Any]]],
        lr: float = 1e-2,
        beta1: Optional[float] = None,
        beta2: Optional[float] = None,
        beta2_decay: Optional[float] = -0.8,
        beta3: Optional[float] = None,
        eps_came: float = 1e-16,
        eps: Tuple[Optional[float], float] = (1e-30, 1e-3),
        weight_decay: float = 0.0,
        d: float = 1.0,
        maximize: bool = False,
        relative_step: bool = True,
        scale_parameter: bool = True,
        factored: bool = True,
        quantize: bool = True,
        block_size: int = 2048,
        m_block_size: int = 256,
        m_quant_type: str = "uf8",
        v_quant_type: str = "al8",
        c_quant_type: Optional[str] = None,
        min_8bit_size: int = 4096,
        use_cuda_kernel: bool = True,
        stochastic_round_writeback: bool = False,
        apollo_rank: int = 0,
        apollo_update_proj_gap: int = 200,
        apollo_scale_type: str = "channel",
        apollo_scale: float = 1.0,
        apollo_scale_front: bool = False,
        apollo_eps: float = 1e-6,
        apollo_factorize: bool = False,
        apollo_cache_proj: bool = False,
        enable_fira_for_apollo: bool = True,
        scale_weight_decay: bool = True,
        enable_fira_for_adafactor: bool = False,
        fira_margin: float = 0.01,
        lag_norm: bool = False,
        momentum_only_1d: Optional[bool] = None,
        bias_correction: Optional[bool] = None,
        warmup_multiplier: float = 0.0,
        capturable: bool = False,
        al_refit_rule: str = "fallback",
    ):
        # argument validation: optimizer.py:1362-1432 (same conditions and messages)
        if lr < 0.0:
            raise ValueError(f"Invalid lr: {lr}, must be >= 0.0")
        if beta1 is not None and (beta1 < 0.0 or beta1 >= 1.0):
            raise ValueError(f"Invalid beta1: {beta1}, must be in [0.0, 1.0)")
        if beta2_decay is not None and beta2_decay > 0.0:
            raise ValueError(f"Invalid beta2_decay: {beta2_decay}, must be <= 0.0")
        if beta2 is None and beta2_decay is None:
            if relative_step:
                raise ValueError(
                    "When `beta2` and `beta2_decay` are both None, `relative_step` must be False. "
                    "Please set `relative_step=False` for standard SGD, or specify `beta2`/`beta2_decay` "
                    "to use adaptive optimizers.")
            if apollo_rank > 0:
                raise ValueError("APOLLO requires a second-moment estimate (`beta2` or `beta2_decay`), "
                                 "but both are currently None.")
            if beta3 is not None:
                raise ValueError("CAME (`beta3`) requires both `beta1` and `beta2`, but `beta2` is "
                                 "currently None.")
        eps1, eps2 = eps
        if eps1 is None:
            eps1 = 1e-30
        if eps1 < 0.0:
            raise ValueError(f"Invalid eps1: {eps1}, must be >= 0.0")
        if eps2 < 0.0:
            raise ValueError(f"Invalid eps2: {eps2}, must be >= 0.0")
        if d < 0.0:
            raise ValueError(f"Invalid d: {d}, must be >= 0.0. d=0 disables RMS clipping.")
        if weight_decay < 0.0:
            raise ValueError(f"Invalid weight_decay: {weight_decay}, must be >= 0.0")
        if beta2 is not None and (beta2 < 0.0 or beta2 >= 1.0):
            raise ValueError(f"Invalid beta2: {beta2}, must be in [0.0, 1.0)")
        if quantize and (block_size < 128 or block_size % 128 != 0):
            raise ValueError(f"block_size must be >= 128 and a multiple of 128, but got {block_size}.")
        if m_block_size < 32 or m_block_size % 4 != 0:
            raise ValueError(f"m_block_size must be a multiple of 4 and >= 32, but got {m_block_size}.")
        if m_quant_type not in _VALID_M_QUANT_TYPES:
            raise ValueError(f"m_quant_type must be one of {_VALID_M_QUANT_TYPES}, got '{m_quant_type}'.")
        if v_quant_type not in _VALID_V_QUANT_TYPES:
            raise ValueError(f"v_quant_type must be one of {_VALID_V_QUANT_TYPES}, got '{v_quant_type}'.")
        if c_quant_type is not None and c_quant_type not in _VALID_V_QUANT_TYPES:
            raise ValueError(f"c_quant_type must be one of {_VALID_V_QUANT_TYPES} or None, "
                             f"got '{c_quant_type}'.")
        if quantize and beta1 is not None and m_quant_type != "fp32" and block_size % m_block_size != 0:
            raise ValueError(
                f"For the fused 1D kernel, block_size must be a multiple of m_block_size "
                f"(got block_size={block_size}, m_block_size={m_block_size}).")
        if apollo_rank > 0 and apollo_scale_type not in ("channel", "tensor"):
            raise ValueError(f"apollo_scale_type must be 'channel' or 'tensor', got {apollo_scale_type}.")
        if apollo_scale < 0.0:
            raise ValueError(f"Invalid apollo_scale: {apollo_scale}, must be >= 0.0")
        if fira_margin < 0.0:
            raise ValueError(f"Invalid fira_margin: {fira_margin}, must be >= 0.0")
        if beta3 is not None:
            if beta3 < 0.0 or beta3 >= 1.0:
                raise ValueError(f"Invalid beta3: {beta3}, must be in [0.0, 1.0)")
            if beta1 is None:
                raise ValueError("CAME (beta3) strictly requires momentum (beta1) to compute update "
                                 "instability.")
            if apollo_rank == 0 and not factored:
                raise ValueError("CAME (beta3) requires factored=True (2D row/col factorization). It is "
                                 "not supported for 1D full-rank paths.")

        if al_refit_rule not in ("fallback", "kernel"):
            raise ValueError(f"al_refit_rule must be 'fallback' or 'kernel', got {al_refit_rule!r}")
        defaults = dict(
            lr=lr, beta1=beta1, beta2=beta2, beta2_decay=beta2_decay, beta3=beta3, eps_came=eps_came,
            eps=eps, weight_decay=weight_decay, d=d, maximize=maximize,
            relative_step=relative_step, scale_parameter=scale_parameter, factored=factored,
            quantize=quantize, block_size=block_size, m_block_size=m_block_size,
            m_quant_type=m_quant_type, v_quant_type=v_quant_type, c_quant_type=c_quant_type,
            min_8bit_size=min_8bit_size, use_cuda_kernel=use_cuda_kernel,
            stochastic_round_writeback=stochastic_round_writeback,
            apollo_rank=apollo_rank, apollo_update_proj_gap=apollo_update_proj_gap,
            apollo_scale_type=apollo_scale_type, apollo_scale=apollo_scale,
            apollo_scale_front=apollo_scale_front, apollo_eps=apollo_eps,
            apollo_factorize=apollo_factorize, apollo_cache_proj=apollo_cache_proj,
            enable_fira_for_apollo=enable_fira_for_apollo,
            scale_weight_decay=scale_weight_decay,
            enable_fira_for_adafactor=enable_fira_for_adafactor, fira_margin=fira_margin,
            lag_norm=lag_norm, momentum_only_1d=momentum_only_1d, bias_correction=bias_correction,
            warmup_multiplier=warmup_multiplier, capturable=capturable, al_refit_rule=al_refit_rule,
        )
        super().__init__(params, defaults)
        self._apollo_seed_counter = 1
        self._sr_seed_counter = 1
        self._ws = {}   # device workspaces (tensor tables, norm buffers, v_buf)

    def add_param_group(self, param_group):
        """``Optimizer.add_param_group`` plus a check that every parameter's route
        can run with the group's block sizes, so an unsupported size fails here
        and not halfway through a step."""
        super().add_param_group(param_group)
        try:
            _check_block_sizes(self.param_groups[-1])
        except ValueError:
            self.param_groups.pop()
            raise

    # ------------------------------------------------------------------ checkpoint
    def state_dict(self):
        for key, ent in list(self._ws.items()):
            if isinstance(key, tuple) and len(key) == 3 and key[1] == "devstep":
                t = int(ent["ctr"].item())   # graph replays advance only the device count
                for p in ent["group"]["params"]:
                    if p in self.state and "step" in self.state[p]:
                        self.state[p]["step"] = t
        _sync_apollo_schedule(self)
        sd = super().state_dict()
        sd["_apollo_seed_counter"] = self._apollo_seed_counter
        sd["_sr_seed_counter"] = self._sr_seed_counter
        return sd

    def load_state_dict(self, state_dict):
        """optimizer.py:1467-1553: the base loader maps saved parameters to these
        ones; state tensors keep their stored dtype (fp32 or codes, whatever the
        parameter's dtype), the codec tags, seed counters and SR policy come from
        the checkpoint, and the loaded state is then compacted (optimizer.py:1555-1590)."""
        ckpt = S.Checkpoint(state_dict, self.param_groups)
        super().load_state_dict(ckpt.skeleton)
        ckpt.restore(self)
        S.compact(self)
        self._ws.clear()

    def _warmup_allocator(self):
        """optimizer.py:1592-1616: optional allocate-and-free of a large block."""
        mult = self.param_groups[0].get("warmup_multiplier", 0.0)
        if mult <= 0.0 or not torch.cuda.is_available():
            return
        biggest = {}
        for g in self.param_groups:
            for p in g["params"]:
                if p.is_cuda and p.numel() > biggest.get(p.device, 0):
                    biggest[p.device] = p.numel()
        for dev, n in biggest.items():
            tmp = torch.empty(int(n * mult), device=dev, dtype=torch.float32)
            del tmp

    # ------------------------------------------------------------------ state init
    def _init_group(self, group, params_with_grad, grads, states):
        S.init_group(self, group, params_with_grad, grads, states)

    # ------------------------------------------------------------------ step
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        if not hasattr(self, "_allocator_warmed_up"):
            self._warmup_allocator()
            self._allocator_warmed_up = True
        # A step plans every parameter on the host and holds those temporaries until
        # its launches are queued.  A cyclic collection running meanwhile would move
        # them to the oldest generation, whose full pass (tens of ms with torch
        # loaded) then stalls the launch stream; with automatic collection held off
        # for the step they are freed by reference counting first.
        gc_on = gc.isenabled()
        if gc_on:
            gc.disable()
        try:
            with nat.range_marker(b"adafactor8bit.step"):
                self._step_groups()
        finally:
            if gc_on:
                gc.enable()
        return loss

    def _step_groups(self):
        for group in self.param_groups:
            params, grads, states = [], [], []
            self._init_group(group, params, grads, states)
            if not params:
                continue
            for p in params:
                if not p.is_cuda:
                    raise RuntimeError("adafactor8bit (MI355X build): parameters must be on a ROCm "
                                       "device; there is no CPU path")
            S.ensure_qmap(params[0].device)
            sr_on = group.get("stochastic_round_writeback", False)
            for p, st in zip(params, states):
                if sr_on and p.dtype in (torch.bfloat16, torch.float16) and "sr_seed" not in st:
                    st["sr_seed"] = self._sr_seed_counter
                    self._sr_seed_counter += 1
            dsc = _advance_device_step(self, group, params, states) if group.get("capturable") else None
            try:
                with nat.range_marker(b"adafactor8bit.group"):
                    self._step_group(group, params, grads, states, dsc)
            except Exception:
                if dsc is not None:   # the device count moved on; rebuild it from the restored host counts
                    self._ws.pop((params[0].device, "devstep", id(group)), None)
                raise

    # ------------------------------------------------------------------ dispatch
    def _step_group(self, group, params, grads, states, dsc=None):
        """Plan and launch one group.  The plans advance each parameter's step
        counter; if a launch raises, the counters go back, so a step that did not
        run is not counted.  ``dsc``: the device block of this step's scalars
        (capturable groups)."""
        before = [st.get("step", 0) for st in states]
        try:
            self._launch_group(group, params, grads, states, dsc)
        except Exception:
            for st, s0 in zip(states, before):
                st["step"] = s0
            raise

    def _launch_group(self, group, params, grads, states, dsc=None):
        apollo_rank = group.get("apollo_rank", 0)
        if dsc is not None and isinstance(group["lr"], Tensor):
            # the kernels read this step's lr from the device block: plan with a
            # placeholder so no host scalar is formed from the tensor
            group = dict(group, lr=1.0)
        batches: Dict[tuple, list] = {}
        ap_batches: Dict[tuple, list] = {}
        copy_back = []
        for p, g, st in zip(params, grads, states):
            if p.numel() == 0:
                # the reference's update of an empty tensor is a sequence of no-op tensor
                # ops: the step is counted, nothing is launched
                st["step"] = st.get("step", 0) + 1
                continue
            if g.data_ptr() % 16:
                # the kernels load 16 bytes at a time: a gradient that starts off a 16-byte
                # boundary (a slice of a flat buffer) is copied to one kept per parameter
                key = (g.device, "galign", id(p))
                gw = self._ws.get(key)
                if gw is None or gw.shape != g.shape or gw.dtype != g.dtype:
                    gw = torch.empty(g.shape, dtype=g.dtype, device=g.device)
                    self._ws[key] = gw
                gw.copy_(g)
                g = gw
            if not p.is_contiguous() or p.data_ptr() % 16:
                # the reference steps a contiguous copy and writes it back (optimizer.py:2002-2007,
                # 2608-2614); the copy is kept so workspaces keyed by the tensor stay valid.  A
                # parameter that starts off a 16-byte boundary steps an aligned copy the same way
                key = (p.device, "contig", id(p))
                work = self._ws.get(key)
                if work is None or work.shape != p.shape or work.dtype != p.dtype:
                    work = torch.empty(p.shape, dtype=p.dtype, device=p.device)
                    self._ws[key] = work
                work.copy_(p)
                copy_back.append((p, work))
                p = work
            if apollo_rank > 0 and "apollo_seed" in st:
                bkey, rec, fin = _apollo_prep(self, p, g, st, group, dsc)
                ap_batches.setdefault(bkey, []).append((rec, fin))
                continue
            plan = _plan_param(p, _grad_work(self, p, g, g.dtype, group["maximize"]), st, group)
            plan.dsc = dsc
            if plan.path == "q1d" and plan.alpha_t is not None and plan.mbuf is None:
                _persist_scale(self, plan, group, dsc)
            if plan.path == "q1d_fp32m":
                _prep_q1d_fp32m(self, plan)
            elif plan.path == "f1d_qm":
                _prep_f1d_qm(self, plan)
            key = plan.batch_key()
            if key is None:
                if dsc is not None:
                    raise NotImplementedError(
                        f"adafactor8bit: capturable=True covers the multi-tensor paths only; a '{plan.path}' "
                        f"parameter of shape {tuple(p.shape)} needs a per-tensor launch")
                _run_single(self, plan)
            else:
                batches.setdefault(key, []).append(plan)
        for key, plans in batches.items():
            _run_batch(self, key, plans)
        for bkey, items in ap_batches.items():
            _run_apollo_batch(self, group, bkey, items, dsc)
        for p, work in copy_back:
            p.copy_(work)


# ====================================================================== device step (capturable)
def _no_upload_in_capture(upload):
    """A tensor table is uploaded from host memory, which a captured graph would
    replay from whatever that memory holds later: tables must exist before capture."""
    if upload and torch.cuda.is_current_stream_capturing():
        raise RuntimeError("adafactor8bit: a step being captured would upload a tensor table; run one eager "
                           "step with the same parameters, gradients and state first")


def _step_spec(group):
    """The group's a8_step_spec: the host planner's scalar rules (_plan_param,
    _plan_factored; optimizer.py:2012-2039, 832-856) as data."""
    beta1, beta2, beta2_decay = group.get("beta1"), group["beta2"], group["beta2_decay"]
    lr, lr_dev = group["lr"], None
    if isinstance(lr, Tensor):
        lr_dev = _device_lr(lr, group)
        lr = 0.0
    sgd = beta2 is None and beta2_decay is None
    eps1 = group["eps"][0]
    eps1 = 1e-30 if eps1 is None else eps1
    adam_denom = (not group.get("factored", True)) and beta2 is not None and group.get("beta3") is None
    bias_mode = 0
    if beta1 is not None and not group["relative_step"] and not sgd:
        bc = group.get("bias_correction")
        if (adam_denom if bc is None else bool(bc)):
            bias_mode = 1 if beta2 is not None else 2
    wd = group["weight_decay"]
    wd_mode = 0 if wd == 0 else (1 if group.get("scale_weight_decay", True) else 2)
    # APOLLO's bias correction is on unless bias_correction=False (optimizer.py:3015-3023)
    ap_bias = 0
    if beta1 is not None and not group["relative_step"]:
        bc = group.get("bias_correction")
        if bc is None or bool(bc):
            ap_bias = 1 if beta2 is not None else 2
    return nat.StepSpec(beta1 if beta1 is not None else 0.0, beta2 if beta2 is not None else 0.0,
                        beta2_decay if beta2_decay is not None else 0.0, eps1, float(lr), _f32(wd),
                        0 if sgd else (1 if beta2 is not None else 2), int(bool(group["relative_step"])), bias_mode,
                        int(adam_denom), wd_mode, bias_mode, ap_bias, lr_dev)


def _device_lr(lr, group):
    """A tensor learning rate of a capturable group: read on the device at every step
    (a scheduler that fill_()s it changes the lr of graph replays too)."""
    p0 = group["params"][0]
    if not (lr.numel() == 1 and lr.dtype == torch.float32 and lr.device == p0.device):
        raise NotImplementedError("adafactor8bit: capturable=True takes a float learning rate or a one-element "
                                  "float32 tensor on the parameters' device")
    if group["relative_step"]:
        raise NotImplementedError("adafactor8bit: capturable=True with relative_step needs a float learning rate")
    return lr.data_ptr()


def _advance_device_step(opt, group, params, states):
    """Advance the group's device step count and write this step's scalars
    (a8_step_advance); returns the scalar block.  The count starts from the
    parameters' host count, which must be the same for the whole group."""
    dev = params[0].device
    key = (dev, "devstep", id(group))
    ent = opt._ws.get(key)
    if ent is None:
        steps = {int(st.get("step", 0)) for st in states}
        if len(steps) != 1:
            raise RuntimeError(f"adafactor8bit: capturable=True needs one step count per group, found {sorted(steps)}")
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("adafactor8bit: run one eager step before capturing a capturable optimizer's step")
        ent = {"ctr": torch.tensor([steps.pop()], dtype=torch.int64, device=dev),
               "scal": torch.zeros(nat.STEP_SCALARS_BYTES // 4, dtype=torch.float32, device=dev),
               "group": group}
        opt._ws[key] = ent
    ent["spec"] = _step_spec(group)
    nat.check(nat.lib().a8_step_advance(ctypes.byref(ent["spec"]), ent["ctr"].data_ptr(), ent["scal"].data_ptr(),
                                        nat.stream_of(dev)), "a8_step_advance")
    return ent["scal"]


# ====================================================================== block sizes
def _pow2_in(x, lo, hi):
    return isinstance(x, int) and lo <= x <= hi and (x & (x - 1)) == 0


def _check_block_sizes(group):
    """Raise ValueError if a parameter of ``group`` would reach a kernel that cannot
    run its block sizes.  The constructor already enforces the reference's own
    rules (optimizer.py:1395-1416: B_V a multiple of 128, B_M a multiple of 4 and
    at least 32, B_V % B_M == 0).  Every route takes every size those rules allow
    up to 2^30 (the kernels' block sizes are 32-bit ints):
      * quantised 1-D V (AL8/AL16) with coded momentum or none: powers of two in
        [128, 2048] take the unit layout, the others one workgroup per V block
        (a V block of more than 2048 M blocks in segments of 2048);
      * coded momentum on the SGD route and with fp32 V on the 1-D route, and on
        the factored route: powers of two up to 2048 take the unit / tiled
        layouts, the others whole M blocks per workgroup;
      * quantised 1-D V with fp32 momentum (the stand-alone AL EMA) and the
        APOLLO route's low-rank V: one workgroup per V block beyond the unit
        layout's sizes.
    The factored row / column statistics take any B_V."""
    if not group.get("quantize", True):
        return
    bs, mbs = group.get("block_size", 2048), group.get("m_block_size", 256)
    vqt, mqt = group.get("v_quant_type", "al8"), group.get("m_quant_type", "uf8")
    coded_m = group.get("beta1") is not None and mqt != "fp32"
    if not any(p.numel() >= group.get("min_8bit_size", 4096) for p in group["params"]):
        return
    if vqt != "fp32" and bs > _MAX_BLOCK:
        raise ValueError(f"block_size={bs}: the kernels of this build take at most {_MAX_BLOCK}.")
    if coded_m and mbs > _MAX_BLOCK:
        raise ValueError(f"m_block_size={mbs}: the kernels of this build take at most {_MAX_BLOCK}.")


_MAX_BLOCK = 1 << 30


# ====================================================================== planning
class _Plan:
    """Host-side scalar preparation of one parameter's step (optimizer.py:1944-2040)."""
    __slots__ = ("p", "g", "st", "group", "path", "step", "beta_val", "alpha_val", "alpha_t",
                 "rho_val", "rho_t", "eps1", "eps2", "eps_sq", "log_eps_sq", "adam_denom", "eps_d",
                 "eps_g", "mom_only", "beta1", "d", "fira", "margin", "decay_val", "decay_t",
                 "sr", "quant", "vqt", "mqt", "bs", "mbs", "has_m", "maximize", "beta3", "scale_param",
                 "bias_mode", "bias_fac", "wd", "wd_mode", "rms_kernel", "kwd", "vbuf", "mbuf", "_keep", "dsc",
                 "al_floor", "al_vbits", "pers")

    def batch_key(self):
        if self.path == "factored":
            return ("factored", self.p.device, self.p.dtype, self.g.dtype, self.step, self.quant,
                    self.vqt, self.bs, self.has_m, self.mqt, self.mbs, self.sr, self.beta3)
        if self.path not in ("q1d", "f1d", "sgd") or self.mbuf is not None:
            return None
        if (self.alpha_t is not None or self.decay_t is not None) and not self.pers:
            return None
        if self.p.data_ptr() % 16 or self.g.data_ptr() % 16:
            return None
        if self.path == "f1d" and (self.d > 0 or self.fira or self.rms_kernel):
            return ("f1dc", self.p.device, self.p.dtype, self.g.dtype, self.step, self.sr, self.has_m,
                    self.vbuf is not None,
                    self.beta1, self.beta_val, self.eps_d, self.eps_g, self.eps_sq, self.adam_denom, self.mom_only,
                    self.alpha_val, self.decay_val, self.kwd, self.group["weight_decay"], self.d, self.fira,
                    self.margin, self.rms_kernel, self.eps2)
        if self.path == "q1d" and (self.d > 0 or self.fira):
            return ("q1dc", self.p.device, self.p.dtype, self.g.dtype, self.step, self.sr, self.pers, self.vqt,
                    self.al_vbits,
                    self.mqt if self.has_m else None, self.bs, self.mbs, self.has_m, self.beta1,
                    self.beta_val, self.eps_d, self.eps_g, self.eps_sq, self.adam_denom, self.mom_only,
                    self.alpha_val, self.decay_val, self.d, self.fira, self.margin)
        if self.path == "sgd" and (self.d > 0 or self.fira):
            mq = self.has_m and self.quant and self.mqt != "fp32" and "m_q" in self.st
            return ("sgdc", self.p.device, self.p.dtype, self.g.dtype, self.step, self.sr, self.has_m, mq,
                    self.mqt if mq else None, self.mbs if mq else 0, self.beta1, self.alpha_val, self.decay_val,
                    self.d, self.fira, self.margin)
        if self.d > 0 or self.fira:
            return None
        if self.path == "sgd":
            mq = self.has_m and self.quant and self.mqt != "fp32" and "m_q" in self.st
            return ("sgd", self.p.device, self.p.dtype, self.g.dtype, self.step, self.sr, self.has_m, mq,
                    self.mqt if mq else None, self.mbs if mq else 0, self.beta1, self.alpha_val, self.decay_val)
        return (self.path, self.p.device, self.p.dtype, self.g.dtype, self.step, self.sr, self.vqt,
                self.vbuf is not None, self.al_vbits, self.pers,
                self.mqt if self.has_m else None, self.bs, self.mbs, self.has_m, self.beta1,
                self.beta_val, self.eps_d, self.eps_g, self.eps_sq, self.adam_denom, self.mom_only,
                self.alpha_val, self.decay_val)


def _grad_work(opt, p, grad, dtype, negate):
    """The gradient the kernels read.  p.grad itself when it is contiguous, of
    ``dtype`` and not negated; otherwise a copy -- contiguous, converted (fp32 for
    fp16 / fp64 APOLLO, as the reference's grad.float(), optimizer.py:2601) and/or
    negated (maximize, optimizer.py:1971-1973, 2604-2605) -- in a buffer kept per
    parameter, so that its address is the same every step: multi-tensor tables stay
    valid and a captured step reads the buffer its copy kernel refills."""
    if grad.is_contiguous() and grad.dtype == dtype and not negate:
        return grad
    key = (p.device, "gwork", id(p))
    buf = opt._ws.get(key)
    if buf is None or buf.shape != grad.shape or buf.dtype != dtype:
        buf = torch.empty(grad.shape, dtype=dtype, device=grad.device)
        opt._ws[key] = buf
    if negate and grad.dtype == dtype:
        torch.neg(grad, out=buf)
    else:
        buf.copy_(grad)
        if negate:
            buf.neg_()
    return buf


def _plan_param(p, grad, st, group) -> _Plan:
    P = _Plan()
    P.p, P.st, P.group = p, st, group
    P.pers = False
    P.vbuf = None
    P.mbuf = None
    beta1, beta2, beta2_decay, beta3 = group.get("beta1"), group["beta2"], group["beta2_decay"], group.get("beta3")
    eps1, eps2 = group["eps"]
    eps1 = 1e-30 if eps1 is None else eps1
    d = group["d"]
    factored = group.get("factored", True)
    sgd = beta2 is None and beta2_decay is None
    full_rank = grad.dim() < 2 or not factored or sgd
    P.eps1, P.eps2 = eps1, eps2
    P.eps_sq = max(eps1 * eps1, _LOG_QUANT_FLOOR)
    P.log_eps_sq = math.log2(P.eps_sq)
    # the V refit of the fused 1-D step: the CPU quantiser's rule (floor -126), or with
    # al_refit_rule="kernel" the reference's fused CUDA kernels' rule, whose floor is
    # log_eps_sq (optimizer.py:1961-1962 passes it to kernels.cu:772-774)
    krule = group.get("al_refit_rule", "fallback") == "kernel"
    P.al_floor = _f32(P.log_eps_sq) if krule else _AL_FLOOR
    P.al_vbits = (16 if st.get("v_quant_type", "al8") == "al16" else 8) | (nat.AL_KERNEL_RULE if krule else 0)
    P.adam_denom = (not factored) and (beta2 is not None) and (beta3 is None)
    P.eps_d = eps1 if P.adam_denom else 0.0
    P.eps_g = eps1 if not P.adam_denom else 0.0
    mo = group.get("momentum_only_1d")
    P.mom_only = (not P.adam_denom) if mo is None else bool(mo)
    P.maximize = group["maximize"]   # the caller hands the negated gradient (_grad_work)
    P.g = grad if grad.is_contiguous() else grad.contiguous()
    P.quant = st.get("is_quantized", False)
    P.vqt = st.get("v_quant_type", "al8")
    P.bs = st.get("block_size", group.get("block_size", 2048))
    P.has_m = beta1 is not None
    P.mbs = st.get("m_block_size", group.get("m_block_size", 256)) if P.has_m else 0
    P.mqt = st.get("m_quant_type", "uf8") if P.has_m else "uf8"
    P.beta1 = beta1
    P.d = d
    P.fira = group.get("enable_fira_for_adafactor", False)
    P.margin = group.get("fira_margin", 0.01)
    # lag_norm: the PyTorch branches clip by this step's norm whatever lag_norm says
    # (the one-pass lagged clip, _dispatch_cuda_clip optimizer.py:1048-1073, is a CUDA-
    # branch approximation); this build follows them, as for every other rule

    P.beta3 = beta3
    if sgd:
        P.path = "sgd"
    elif full_rank:
        if P.quant and P.vqt != "fp32":
            P.path = "q1d" if (not P.has_m or P.mqt != "fp32") else "q1d_fp32m"
        else:
            P.path = "f1d" if (not P.has_m or not P.quant or P.mqt == "fp32") else "f1d_qm"
    else:
        P.path = "factored"

    step = st["step"] + 1
    st["step"] = step
    P.step = step
    if sgd:
        P.beta_val = 0.0
    elif beta2 is not None:
        P.beta_val = 1.0 - beta2
    else:
        P.beta_val = math.pow(step, beta2_decay)

    P.sr = group.get("stochastic_round_writeback", False) and p.dtype in (torch.bfloat16, torch.float16)
    if P.path == "factored":
        _plan_factored(P, group, beta1, beta2, sgd)
        return P

    # alpha / rho: optimizer.py:832-856 (+ bias correction 2020-2030)
    lr = group["lr"]
    P.alpha_t = P.rho_t = None
    relative_step, scale_parameter = group["relative_step"], group["scale_parameter"]
    if scale_parameter and p.dtype == torch.float64:
        # the reference's _compute_alpha (optimizer.py:850-852) takes the norm with
        # dtype=float32, which torch refuses for a float64 tensor: the same error here
        torch.linalg.vector_norm(p, ord=2, dtype=torch.float32)
    if isinstance(lr, Tensor):
        rho_t = lr.to(device=p.device, dtype=torch.float32)
        if relative_step:
            rho_t = torch.minimum(torch.tensor(float(step), device=p.device).rsqrt(), rho_t)
        P.rho_t, P.rho_val = rho_t, None
    else:
        P.rho_val = _f32(min(lr, 1.0 / math.sqrt(step)) if relative_step else lr)
    bc_applies = beta1 is not None and not relative_step and not sgd and bool(
        P.adam_denom if group.get("bias_correction") is None else group.get("bias_correction"))
    # fp32-state vectors can take alpha = max(rms(p), eps2) * rho inside the batched
    # kernels (one pass computes sum(p^2)); _materialize_alpha computes it here when
    # the plan runs on its own.
    P.rms_kernel = bool(scale_parameter and P.path == "f1d" and P.rho_t is None and not bc_applies)
    P.kwd = 0
    if P.rms_kernel:
        P.alpha_t, P.alpha_val = None, P.rho_val
    elif scale_parameter:
        rms = torch.linalg.vector_norm(p, ord=2, dtype=torch.float32) / math.sqrt(p.numel())
        rho = P.rho_t if P.rho_t is not None else P.rho_val
        P.alpha_t = torch.clamp(rms, min=eps2) * rho
        P.alpha_val = None
    elif P.rho_t is not None:
        P.alpha_t, P.alpha_val = P.rho_t, None
    else:
        P.alpha_val = P.rho_val
    if beta1 is not None and not relative_step and not sgd:
        bc_on = P.adam_denom if group.get("bias_correction") is None else group.get("bias_correction")
        if bc_on:
            bc1 = 1.0 - beta1 ** step
            if beta2 is not None:
                bc2 = 1.0 - beta2 ** step
                fac = math.sqrt(bc2) / bc1
                if P.alpha_t is not None:
                    P.alpha_t = P.alpha_t * fac
                else:
                    P.alpha_val = _f32(_F32(P.alpha_val) * _F32(fac))
                if P.adam_denom:
                    P.eps_d = eps1 * math.sqrt(bc2)
            else:
                if P.alpha_t is not None:
                    P.alpha_t = P.alpha_t / bc1
                else:
                    P.alpha_val = _f32(_F32(P.alpha_val) / _F32(bc1))

    # weight decay: optimizer.py:2032-2039 (fused into the kernels as p*decay)
    wd = group["weight_decay"]
    P.decay_val, P.decay_t = None, None
    if wd != 0:
        use_alpha = group.get("scale_weight_decay", True)
        if use_alpha and P.rms_kernel:
            P.kwd = 1   # 1 - alpha*wd with the kernel's alpha
        elif use_alpha:
            if P.alpha_t is not None:
                P.decay_t = 1.0 - (P.alpha_t * wd)
            else:
                P.decay_val = _f32(_F32(1.0) - _F32(_F32(P.alpha_val) * _F32(wd)))
        else:
            if P.rho_t is not None:
                P.decay_t = 1.0 - (P.rho_t * wd)
            else:
                P.decay_val = _f32(_F32(1.0) - _F32(_F32(P.rho_val) * _F32(wd)))

    return P


def _plan_factored(P, group, beta1, beta2, sgd):
    """Scalar preparation of the factored path: the step size itself (relative
    step, RMS scaling, bias correction, optimizer.py:832-856, 2020-2030) and the
    weight-decay factor (2032-2039) are formed on the device from these inputs."""
    lr = group["lr"]
    relative_step = group["relative_step"]
    P.scale_param = bool(group["scale_parameter"])
    if isinstance(lr, Tensor):
        rho_t = lr.to(device=P.p.device, dtype=torch.float32).reshape(())
        if relative_step:
            rho_t = torch.minimum(torch.tensor(float(P.step), device=P.p.device).rsqrt(), rho_t)
        P.rho_t, P.rho_val = rho_t.contiguous(), 0.0
    else:
        P.rho_t = None
        P.rho_val = _f32(min(lr, 1.0 / math.sqrt(P.step)) if relative_step else lr)
    P.alpha_t, P.alpha_val = None, None
    P.bias_mode, P.bias_fac = 0, 1.0
    if beta1 is not None and not relative_step and not sgd:
        bc_on = P.adam_denom if group.get("bias_correction") is None else group.get("bias_correction")
        if bc_on:
            bc1 = 1.0 - beta1 ** P.step
            if beta2 is not None:
                P.bias_mode, P.bias_fac = 1, _f32(math.sqrt(1.0 - beta2 ** P.step) / bc1)
            else:
                P.bias_mode, P.bias_fac = 2, _f32(bc1)
    wd = group["weight_decay"]
    P.wd = _f32(wd)
    P.wd_mode = 0 if wd == 0 else (1 if group.get("scale_weight_decay", True) else 2)
    P.decay_val, P.decay_t = None, None


def _dev_scalar(opt, device, key, value):
    ws = opt._ws.setdefault((device, "scalars"), {})
    t = ws.get(key)
    if t is None:
        t = torch.empty((), dtype=torch.float32, device=device)
        ws[key] = t
    t.fill_(value)
    return t


def _v_buf(opt, device, numel):
    key = (device, "v_buf")
    b = opt._ws.get(key)
    if b is None or b.numel() < numel:
        b = torch.empty(numel, dtype=torch.float32, device=device)
        opt._ws[key] = b
    return b[:numel]


def _norm_buf(opt, device, which="norm_buf"):
    key = (device, which)
    b = opt._ws.get(key)
    if b is None:
        b = torch.zeros(1, dtype=torch.float32, device=device)
        opt._ws[key] = b
    else:
        b.zero_()
    return b


def _norm_parts(opt, device, n):
    """Workspace of a norm pass's per-workgroup partial sums (float64): the library
    adds a tensor's partials in index order, so the sum has the same bits run to
    run.  Shared by the passes of a step, which run one after another on the stream."""
    key = (device, "norm_parts")
    b = opt._ws.get(key)
    n = max(int(n), 1)
    if b is None or b.numel() < n:
        b = torch.empty(n, dtype=torch.float64, device=device)
        opt._ws[key] = b
    return b


def _parts_of(P):
    """Doubles of norm-pass workspace one tensor of plan P needs."""
    L = nat.lib()
    n = P.p.numel()
    if P.path == "q1d":
        return int(L.a8_norm_parts_1d(n, P.bs, P.mbs if P.has_m else P.bs))
    if P.path == "sgd":
        _, _, _, kind = _sgd_momentum(P)
        return int(L.a8_norm_parts_sgd(n, P.mbs if kind == 1 else 0))
    return int(L.a8_norm_parts_full(n))


def _alpha_args(P):
    if P.alpha_t is not None:
        a = P.alpha_t.reshape(()).to(torch.float32)
        return a, 0.0
    return None, P.alpha_val


def _decay_args(P):
    if P.decay_t is not None:
        return P.decay_t.reshape(()).to(torch.float32), 1.0, 1
    if P.decay_val is not None:
        return None, P.decay_val, 1
    return None, 1.0, 0


def _launch_1d(opt, P, mode, alpha_t, alpha_val, norm_buf=None, prev_norm=None, v_buf=None):
    L = nat.lib()
    st, p, g = P.st, P.p, P.g
    dec_t, dec_val, has_dec = _decay_args(P)
    parts = _norm_parts(opt, p.device, _parts_of(P)) if norm_buf is not None else None
    if P.path == "q1d":
        vq = st["variance_q"]
        m_q = st["m_q"] if P.has_m else None
        m_scale = st["m_scale"] if P.has_m else None
        m_bits = S.m_bits(P.mqt) if P.has_m else 0
        m_mode = S.m_mode(P.mqt) if P.has_m else 0
        rc = L.a8_fused_update_1d(
            mode, int(P.sr), nat.dtype_code(p.dtype), nat.ptr(p), nat.ptr(g), nat.ptr(m_q),
            nat.ptr(m_scale), nat.ptr(vq), nat.ptr(st["variance_scale"]), nat.ptr(st["variance_min_log"]),
            nat.ptr(v_buf), nat.ptr(norm_buf), nat.ptr(parts), nat.ptr(alpha_t), nat.ptr(prev_norm),
            nat.ptr(dec_t), int(st.get("sr_seed", 0)), int(P.step), P.beta1 if P.has_m else 0.0, P.beta_val, P.eps_d,
            int(P.adam_denom), P.al_floor, P.eps_g, P.eps_sq, p.numel(), P.bs,
            P.mbs if P.has_m else P.bs, m_bits, m_mode, P.d, P.al_vbits,
            int(P.mom_only), float(alpha_val), float(dec_val), int(has_dec),
            nat.stream_of(p.device))
        nat.check(rc, "a8_fused_update_1d")
        if mode != nat.MODE_APPLY:
            _block_view(st, "variance", P.bs)
    else:
        m = st.get("m") if P.has_m else None
        if m is not None and not m.is_contiguous():
            m = m.contiguous()
            st["m"] = m
        beta1 = P.beta1 if P.has_m else 0.0
        if P.mbuf is not None:   # this step's m' is ready: lerp weight 1 - beta1 = 0 keeps it
            m, beta1 = P.mbuf, 1.0
        var = _variance_of(P)
        rc = L.a8_fused_update_1d_full(
            mode, nat.dtype_code(p.dtype), nat.ptr(p), nat.ptr(g), nat.ptr(var), nat.ptr(m),
            nat.ptr(norm_buf), nat.ptr(parts), nat.ptr(alpha_t), nat.ptr(prev_norm), nat.ptr(dec_t),
            beta1, P.beta_val, P.eps_sq, P.eps_d, int(P.adam_denom), P.eps_g,
            p.numel(), P.d, int(P.mom_only), float(alpha_val), float(dec_val), int(has_dec),
            int(P.sr), int(st.get("sr_seed", 0)), int(P.step), int(P.vbuf is not None), nat.stream_of(p.device))
        nat.check(rc, "a8_fused_update_1d_full")


def _block_view(st, prefix, bs):
    """After a re-quantisation the reference stores V codes as [nblocks, block_size]
    (the block view returned by _log_quantize_nonneg, optimizer.py:302-324)."""
    q = st[f"{prefix}_q"]
    if q.dim() == 1:
        st[f"{prefix}_q"] = q.view(-1, bs)


def _fira_apply(opt, st, norm_buf, alpha_t, alpha_val, margin, device):
    """NORM -> Fira -> APPLY glue of _apply_fira_cuda (optimizer.py:785-793)."""
    if alpha_t is None:
        alpha_t = _dev_scalar(opt, device, "fira_alpha", alpha_val)
    prev = st.get("fira_prev_norm")
    out = torch.empty(3, dtype=torch.float32, device=device)
    if prev is not None and not torch.is_tensor(prev):
        prev = torch.tensor(prev, dtype=torch.float32, device=device)
    rc = nat.lib().a8_fira_scalar(nat.ptr(norm_buf), nat.ptr(prev), nat.ptr(alpha_t), nat.ptr(out), 1,
                                  int(prev is not None), 1, _f32(1.0 + margin), nat.stream_of(device))
    nat.check(rc, "a8_fira_scalar")
    st["fira_prev_norm"] = out[1].view(())
    return out[0].view(()), out[2].view(1)


def _sgd_momentum(P):
    """Momentum buffers of an SGD step: (m_q, m_scale, m_fp32, kind) with kind 0
    none, 1 quantised, 2 fp32 (optimizer.py:2046-2068)."""
    if not P.has_m:
        return None, None, None, 0
    st = P.st
    if P.quant and P.mqt != "fp32" and "m_q" in st:
        return st["m_q"], st["m_scale"], None, 1
    if "m" not in st:
        st["m"] = torch.zeros_like(P.g, dtype=torch.float32)
    if not st["m"].is_contiguous():
        st["m"] = st["m"].contiguous()
    return None, None, st["m"], 2


def _run_sgd(opt, P):
    """SGD branch of _update_param_8bit (optimizer.py:2045-2077): one pass, or
    NORM -> (Fira) -> APPLY when the update is clipped (d > 0) or Fira is on."""
    L = nat.lib()
    st, dev = P.st, P.p.device
    m_q, m_scale, m, kind = _sgd_momentum(P)
    m_bits = S.m_bits(P.mqt) if kind == 1 else 0
    m_mode = S.m_mode(P.mqt) if kind == 1 else 0
    alpha_t, alpha_val = _alpha_args(P)
    dec_t, dec_val, has_dec = _decay_args(P)
    strm = nat.stream_of(dev)

    def launch(mode, norm_buf=None, fira=None):
        parts = _norm_parts(opt, dev, _parts_of(P)) if mode == nat.MODE_NORM else None
        rc = L.a8_sgd_step(mode, nat.dtype_code(P.p.dtype), int(P.sr), nat.ptr(P.p), nat.ptr(P.g), nat.ptr(m_q),
                           nat.ptr(m_scale), nat.ptr(m), nat.ptr(norm_buf), nat.ptr(parts), nat.ptr(fira),
                           nat.ptr(alpha_t),
                           nat.ptr(dec_t), P.p.numel(), P.beta1 if P.has_m else 0.0, m_bits, m_mode,
                           P.mbs if kind == 1 else 32, P.d, float(alpha_val), float(dec_val), has_dec,
                           int(st.get("sr_seed", 0)), int(P.step), strm)
        nat.check(rc, "a8_sgd_step")

    if not (P.d > 0.0 or P.fira):
        launch(nat.MODE_NOCLIP)
        return
    nb = _norm_buf(opt, dev)
    launch(nat.MODE_NORM, norm_buf=nb)
    fira = None
    if P.fira:
        # _apply_fira_pytorch (optimizer.py:796-810): scale from ||u||, prev-norm state
        prev = st.get("fira_prev_norm")
        if prev is not None and not torch.is_tensor(prev):
            prev = torch.tensor(prev, dtype=torch.float32, device=dev)
        fira = torch.empty(3, dtype=torch.float32, device=dev)
        rc = L.a8_fira_scalar(nat.ptr(nb), nat.ptr(prev), nat.ptr(_dev_scalar(opt, dev, "one", 1.0)),
                              nat.ptr(fira), 1, int(prev is not None), 1, _f32(1.0 + P.margin), strm)
        nat.check(rc, "a8_fira_scalar")
        st["fira_prev_norm"] = fira[1].view(())
    launch(nat.MODE_APPLY, norm_buf=nb, fira=fira)


def _variance_of(P):
    """The fp32 second moment an fp32-state launch reads: this step's V' from the
    quantised-V pre-pass (v_ready), or the fp32 state itself."""
    if P.vbuf is not None:
        return P.vbuf
    var = P.st["variance"]
    if not var.is_contiguous():
        var = var.contiguous()
        P.st["variance"] = var
    return var


def _prep_q1d_fp32m(opt, P):
    """Quantised V with fp32 momentum (optimizer.py:2078-2087): the V EMA and its AL
    re-encode run first (a8_log_quantize_lerp, x = g^2 + eps_g), writing this step's
    fp32 V' to a per-parameter buffer; the update then takes the fp32-state route
    with that V' (v_ready), as the reference feeds _v_fp32 to _fallback_1d_update."""
    st, p, g = P.st, P.p, P.g
    dev = p.device
    if P.al_vbits & nat.AL_KERNEL_RULE:
        raise NotImplementedError(
            "adafactor8bit: al_refit_rule='kernel' covers the fused 1-D step (quantised or no momentum); "
            "quantised V with fp32 momentum is refitted by fused_log_quantize_lerp's own rule in the reference")
    if "m" not in st:
        st["m"] = torch.zeros_like(g, dtype=torch.float32)
    if not st["m"].is_contiguous():
        st["m"] = st["m"].contiguous()
    key = (dev, "vready", id(p))
    buf = opt._ws.get(key)
    if buf is None or buf.numel() != p.numel():
        buf = torch.empty(p.numel(), dtype=torch.float32, device=dev)
        opt._ws[key] = buf
    if g.dtype != p.dtype:
        raise NotImplementedError("adafactor8bit: gradient dtype must match the parameter dtype")
    gx = g.float() if g.dtype == torch.float64 else g   # fp64: the gradient is read as fp32
    rc = nat.lib().a8_log_quantize_lerp(
        st["variance_q"].data_ptr(), st["variance_scale"].data_ptr(), st["variance_min_log"].data_ptr(),
        gx.data_ptr(), nat.dtype_code(gx.dtype), buf.data_ptr(), float(P.beta_val), int(P.bs), 1, _f32(P.eps_g),
        p.numel(), _AL_FLOOR, 16 if P.vqt == "al16" else 8, nat.stream_of(dev))
    P._keep = gx
    nat.check(rc, "a8_log_quantize_lerp")
    _block_view(st, "variance", P.bs)
    P.vbuf = buf
    P.path = "f1d"


def _prep_f1d_qm(opt, P):
    """fp32 V with quantised momentum.  The reference runs its PyTorch branch here
    with or without its CUDA module (optimizer.py:2185-2191 into
    _fallback_1d_update 886-910).  V takes the branch's mul_ / addcmul_ EMA
    (a8_vema_fp32); the momentum EMA and its re-encode run in a8_m_quantize_lerp,
    whose fp32 output is this step's m'.  The update then takes the fp32-state
    route with V and m' as given.  Momentum-only (optimizer.py:894-901): U =
    g / sqrt(max(v, eps^2)) with the RMS clip, m' = lerp(m, U / clip, 1 - beta1)
    (a8_apollo_came_rms and a8_apollo_came_m_res compute exactly these), then the
    re-encode of m' and the update with m' as the step (no clip), as the
    fp32-momentum route runs it."""
    st, p, g = P.st, P.p, P.g
    if g.dtype != p.dtype:
        raise NotImplementedError("adafactor8bit: gradient dtype must match the parameter dtype")
    if g.dtype == torch.float64:   # the gradient is read as fp32 (the update kernel reads P.g itself)
        g = g.float()
    dev = p.device
    if not st["variance"].is_contiguous():
        st["variance"] = st["variance"].contiguous()
    var = st["variance"]
    L = nat.lib()
    strm = nat.stream_of(dev)
    nat.check(L.a8_vema_fp32(var.data_ptr(), g.data_ptr(), nat.dtype_code(g.dtype), float(P.beta_val),
                             _f32(P.eps_g), p.numel(), strm), "a8_vema_fp32")
    key = (dev, "mready", id(p))
    buf = opt._ws.get(key)
    if buf is None or buf.numel() != p.numel():
        buf = torch.empty(p.numel(), dtype=torch.float32, device=dev)
        opt._ws[key] = buf
    if P.mom_only:
        n = p.numel()
        g32 = g if g.dtype == torch.float32 else g.float()
        aux = opt._ws.get((dev, "mready_aux", id(p)))
        if aux is None or aux.numel() != 2 * n + 1:
            aux = torch.zeros(2 * n + 1, dtype=torch.float32, device=dev)
            opt._ws[(dev, "mready_aux", id(p))] = aux
        clip = aux[2 * n:]
        if P.d > 0.0:   # clamp((||U|| / sqrt(n)) / d, min=1) (optimizer.py:897-899)
            clip.zero_()
            nat.check(L.a8_apollo_came_rms(g32.data_ptr(), var.data_ptr(), clip.data_ptr(), _f32(P.eps_sq), n,
                                           strm), "a8_apollo_came_rms")
            clip.copy_(torch.clamp((torch.sqrt(clip) / math.sqrt(n)) / P.d, min=1.0))
        else:
            clip.fill_(1.0)
        # the residual outputs of the CAME form are not used here
        nat.check(L.a8_apollo_came_m_res(g32.data_ptr(), var.data_ptr(), st["m_q"].data_ptr(),
                                         st["m_scale"].data_ptr(), aux.data_ptr(), buf.data_ptr(),
                                         aux[n:].data_ptr(), clip.data_ptr(), float(P.beta1), 0.0, 0.0,
                                         _f32(P.eps_sq), int(P.mbs), n, S.m_bits(P.mqt), S.m_mode(P.mqt), strm),
                  "a8_apollo_came_m_res")
        # re-encode m' (lerp weight 1 keeps it exactly)
        nat.check(L.a8_m_quantize_lerp(st["m_q"].data_ptr(), st["m_scale"].data_ptr(), buf.data_ptr(), nat.F32,
                                       None, 0.0, int(P.mbs), n, S.m_bits(P.mqt), S.m_mode(P.mqt), strm),
                  "a8_m_quantize_lerp")
        P._keep = (g32, aux)
    else:
        nat.check(L.a8_m_quantize_lerp(st["m_q"].data_ptr(), st["m_scale"].data_ptr(), g.data_ptr(),
                                       nat.dtype_code(g.dtype), buf.data_ptr(), float(P.beta1), int(P.mbs),
                                       p.numel(), S.m_bits(P.mqt), S.m_mode(P.mqt), strm), "a8_m_quantize_lerp")
    P.vbuf = var
    P.mbuf = buf
    P.path = "f1d"


def _materialize_alpha(P):
    """alpha (and its weight decay) of a plan that deferred them to the batched
    kernels, computed as _compute_alpha does (optimizer.py:851-855, 2032-2039)."""
    if not P.rms_kernel:
        return
    rms = torch.linalg.vector_norm(P.p, ord=2, dtype=torch.float32) / math.sqrt(P.p.numel())
    P.alpha_t = torch.clamp(rms, min=P.eps2) * P.rho_val
    P.alpha_val = None
    if P.kwd:
        P.decay_t = 1.0 - (P.alpha_t * P.group["weight_decay"])
    P.rms_kernel, P.kwd = False, 0


def _persist_scale(opt, P, group, dsc):
    """A quantised 1-D plan whose step size is a tensor -- scale_parameter's
    max(rms(p), eps2) * rho, bias corrected (optimizer.py:851-855, 2020-2030), or a
    tensor learning rate -- keeps it, and its weight-decay factor 1 - alpha * wd
    (optimizer.py:2032-2039), in two floats kept per parameter: their addresses go
    into the multi-tensor table (per-tensor alpha and decay, read before the
    launch's scalars), so the plan joins the group's launch and a captured step
    refills them.  Under capturable=True rho and the bias factor are the device
    step block's (its rho and bias_factor: the same values, the same operation
    order as the host path)."""
    dev = P.p.device
    key = (dev, "alpha", id(P.p))
    buf = opt._ws.get(key)
    if buf is None:
        buf = torch.empty(2, dtype=torch.float32, device=dev)
        opt._ws[key] = buf
    a_buf, d_buf = buf[0:1], buf[1:2]
    if dsc is not None:
        # the plan's alpha used the placeholder lr: re-form it from the step block
        beta1, beta2 = group.get("beta1"), group["beta2"]
        sgd = beta2 is None and group["beta2_decay"] is None
        rms = torch.linalg.vector_norm(P.p, ord=2, dtype=torch.float32) / math.sqrt(P.p.numel())
        a = torch.clamp(rms, min=P.eps2) * dsc[6]   # rho
        bc = group.get("bias_correction")
        if beta1 is not None and not group["relative_step"] and not sgd and \
                bool(P.adam_denom if bc is None else bc):
            a = a * dsc[5] if beta2 is not None else a / dsc[5]   # sqrt(bc2) / bc1, or bc1
        a_buf.copy_(a.reshape(1))
        wd = group["weight_decay"]
        if wd != 0 and group.get("scale_weight_decay", True):
            d_buf.copy_((1.0 - (a * wd)).reshape(1))
            P.decay_t = d_buf
        else:
            P.decay_t = None   # the block's decay (1 - rho * wd, or none)
    else:
        a_buf.copy_(P.alpha_t.reshape(1).to(torch.float32))
        if P.decay_t is not None:
            d_buf.copy_(P.decay_t.reshape(1).to(torch.float32))
            P.decay_t = d_buf
    P.alpha_t, P.alpha_val, P.pers = a_buf, 0.0, True


def _run_single(opt, P):
    _materialize_alpha(P)
    if P.path == "factored":
        _run_factored(opt, [P])
        return
    if P.path == "sgd":
        _run_sgd(opt, P)
        return
    if P.path not in ("q1d", "f1d"):
        raise NotImplementedError(f"adafactor8bit: '{P.path}' update path is not available in this build yet")
    alpha_t, alpha_val = _alpha_args(P)
    dev = P.p.device
    need_norm = P.d > 0.0 or P.fira
    if not need_norm:
        _launch_1d(opt, P, nat.MODE_NOCLIP, alpha_t, alpha_val)
        return
    st = P.st
    nb = _norm_buf(opt, dev)
    vb = _v_buf(opt, dev, P.p.numel()) if P.path == "q1d" else None
    _launch_1d(opt, P, nat.MODE_NORM, None, 0.0, norm_buf=nb, v_buf=vb)
    if P.fira and P.has_m and P.mom_only:
        # momentum-only: the U-clip uses ||U|| (NORM), Fira the new momentum's
        # norm ||M'|| (optimizer.py:890-896, _apply_update_pytorch 866-875)
        nbm = _norm_buf(opt, dev, "norm_buf_m")
        _launch_1d(opt, P, nat.MODE_MNORM, None, 0.0, norm_buf=nbm, prev_norm=nb, v_buf=vb)
        alpha_t, _ = _fira_apply(opt, st, nbm, alpha_t, alpha_val, P.margin, dev)
    elif P.fira:
        alpha_t, nb = _fira_apply(opt, st, nb, alpha_t, alpha_val, P.margin, dev)
    _launch_1d(opt, P, nat.MODE_APPLY, alpha_t, alpha_val, norm_buf=nb, v_buf=vb)


def _run_batch_f1dc(opt, key, plans):
    """fp32-state vectors with an RMS clip, Fira or scale_parameter as one group:
    NORM (sum u^2, and sum p^2 for scale_parameter) -> MNORM (momentum-only Fira)
    -> Fira scalar over all tensors -> APPLY, each one launch (the per-tensor
    sequence of _run_single, optimizer.py:1048-1077, 785-793)."""
    P0 = plans[0]
    dev = P0.p.device
    L = nat.lib()
    n = len(plans)
    fira = bool(P0.fira)
    mnorm = fira and P0.has_m and P0.mom_only
    for pl in plans:
        if pl.has_m and not pl.st["m"].is_contiguous():
            pl.st["m"] = pl.st["m"].contiguous()
    ws = opt._ws.setdefault((dev, "f1dc"), {})
    ck = (tuple((pl.p.data_ptr(), pl.g.data_ptr(), _variance_of(pl).data_ptr()) for pl in plans), P0.sr,
          P0.has_m, fira, mnorm, P0.rms_kernel)
    refs = [tuple(v.data_ptr() for k, v in pl.st.items() if torch.is_tensor(v) and k != "fira_prev_norm")
            for pl in plans]
    ent = ws.get(ck)
    if ent is None or ent["refs"] != refs:
        acc = torch.zeros(3 * n, dtype=torch.float32, device=dev)    # sum u^2 | sum M'^2 | sum p^2
        fout = torch.zeros(3 * n, dtype=torch.float32, device=dev)   # Fira: scale | prev norm | clean sum
        a0, f0 = acc.data_ptr(), fout.data_ptr()
        poffs, ptot = [], 0
        for pl in plans:   # per-tensor slices of the passes' partial-sum workspace
            poffs.append(ptot)
            ptot += _parts_of(pl)
        parts = torch.empty(max(ptot, 1), dtype=torch.float64, device=dev)
        arrs = {}
        for mode in (nat.MODE_NORM, nat.MODE_MNORM, nat.MODE_APPLY):
            if mode == nat.MODE_MNORM and not mnorm:
                continue
            arr = (nat.TensorFull * n)()
            for i, pl in enumerate(plans):
                st = pl.st
                nb = a0 + 4 * i
                psq = a0 + 4 * (2 * n + i) if pl.rms_kernel else None
                prev = None
                if mode == nat.MODE_MNORM:
                    nb, prev = a0 + 4 * (n + i), a0 + 4 * i
                elif mode == nat.MODE_APPLY and fira and not mnorm:
                    nb = f0 + 4 * (2 * n + i)
                fs = f0 + 4 * i if (mode == nat.MODE_APPLY and fira) else None
                arr[i] = nat.TensorFull(pl.p.data_ptr(), pl.g.data_ptr(), _variance_of(pl).data_ptr(),
                                        nat.ptr(st.get("m") if pl.has_m else None), nb, None, prev, None,
                                        pl.p.numel(), int(st.get("sr_seed", 0)), psq, fs,
                                        parts.data_ptr() + 8 * poffs[i])
            arrs[mode] = [arr, torch.empty(int(L.a8_table_bytes_full(n)), dtype=torch.uint8, device=dev), 1]
        ent = {"refs": refs, "acc": acc, "fout": fout, "parts": parts, "arrs": arrs}
        if len(ws) > 16:
            ws.clear()
        ws[ck] = ent
    acc, fout = ent["acc"], ent["fout"]
    strm = nat.stream_of(dev)
    has_dec = int(P0.decay_val is not None)
    dec_val = P0.decay_val if has_dec else 1.0

    def launch(mode):
        arr, table, up = ent["arrs"][mode]
        _no_upload_in_capture(up)
        rc = L.a8_fused_update_1d_full_multi(
            mode, nat.dtype_code(P0.p.dtype), arr, n, table.data_ptr(), table.numel(),
            P0.beta1 if P0.has_m else 0.0, P0.beta_val, P0.eps_sq, P0.eps_d, int(P0.adam_denom), P0.eps_g, P0.d,
            int(P0.mom_only), float(P0.alpha_val), float(dec_val), has_dec, int(P0.sr), int(P0.step),
            int(P0.rms_kernel), _f32(P0.eps2), int(P0.kwd), _f32(P0.group["weight_decay"]),
            int(P0.vbuf is not None), up, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_fused_update_1d_full_multi")
        ent["arrs"][mode][2] = 0

    acc.zero_()
    launch(nat.MODE_NORM)
    if mnorm:
        launch(nat.MODE_MNORM)
    if fira:
        # A tensor without a previous norm behaves as one whose previous norm is
        # below 1e-6 (scale 1, next = current), so every slot takes has_prev = 1.
        prev_ok = True
        for i, pl in enumerate(plans):
            pv = pl.st.get("fira_prev_norm")
            if not (torch.is_tensor(pv) and pv.data_ptr() == fout.data_ptr() + 4 * (n + i)):
                prev_ok = False
        if not prev_ok:
            vals = []
            for pl in plans:
                pv = pl.st.get("fira_prev_norm")
                vals.append(torch.zeros((), dtype=torch.float32, device=dev) if pv is None else
                            torch.as_tensor(pv, dtype=torch.float32).to(dev).reshape(()))
            fout[n:2 * n].copy_(torch.stack(vals))
        x = acc[n:2 * n] if mnorm else acc[0:n]
        rc = L.a8_fira_scalar(x.data_ptr(), fout.data_ptr() + 4 * n, None, fout.data_ptr(), n, 1, 2,
                              _f32(1.0 + P0.margin), strm)
        nat.check(rc, "a8_fira_scalar")
        if not prev_ok:
            for i, pl in enumerate(plans):
                pl.st["fira_prev_norm"] = fout[n + i].view(())
    launch(nat.MODE_APPLY)


def _run_batch_q1dc(opt, key, plans):
    """Quantised 1-D tensors with an RMS clip or Fira as one group: NORM (V' to
    each tensor's slice of one v_buf, sum u^2) -> MNORM (momentum-only Fira) ->
    one Fira launch over all tensors -> APPLY, each one multi-tensor launch (the
    per-tensor sequence of _run_single / _dispatch_1d_cuda, optimizer.py:1080-1170,
    785-793).  Fira's scale reaches APPLY as each tensor's fira_scale."""
    P0 = plans[0]
    dev = P0.p.device
    L = nat.lib()
    n = len(plans)
    fira = bool(P0.fira)
    mnorm = fira and P0.has_m and P0.mom_only
    ws = opt._ws.setdefault((dev, "q1dc"), {})
    ck = (tuple((pl.p.data_ptr(), pl.g.data_ptr(), pl.st["variance_q"].data_ptr(),
                 nat.ptr(pl.alpha_t if pl.pers else None), nat.ptr(pl.decay_t if pl.pers else None))
                for pl in plans), P0.sr, P0.has_m, fira, mnorm)
    refs = [tuple(v.data_ptr() for k, v in pl.st.items() if torch.is_tensor(v) and k != "fira_prev_norm")
            for pl in plans]
    ent = ws.get(ck)
    if ent is None or ent["refs"] != refs:
        offs, tot = [], 0
        for pl in plans:   # v_buf slices start 16-byte aligned
            offs.append(tot)
            tot += (pl.p.numel() + 3) // 4 * 4
        vbuf = torch.empty(max(tot, 4), dtype=torch.float32, device=dev)
        poffs, ptot = [], 0
        for pl in plans:   # per-tensor slices of the passes' partial-sum workspace
            poffs.append(ptot)
            ptot += _parts_of(pl)
        parts = torch.empty(max(ptot, 1), dtype=torch.float64, device=dev)
        acc = torch.zeros(2 * n, dtype=torch.float32, device=dev)    # sum u^2 | sum M'^2
        fout = torch.zeros(3 * n, dtype=torch.float32, device=dev)   # Fira: scale | prev norm | clean sum
        a0, f0, v0 = acc.data_ptr(), fout.data_ptr(), vbuf.data_ptr()
        arrs = {}
        for mode in (nat.MODE_NORM, nat.MODE_MNORM, nat.MODE_APPLY):
            if mode == nat.MODE_MNORM and not mnorm:
                continue
            arr = (nat.Tensor1D * n)()
            for i, pl in enumerate(plans):
                st = pl.st
                nb, prev, fs = a0 + 4 * i, None, None
                if mode == nat.MODE_MNORM:
                    nb, prev = a0 + 4 * (n + i), a0 + 4 * i
                elif mode == nat.MODE_APPLY and fira:
                    fs = f0 + 4 * i
                    if not mnorm:   # the update clip reads the Fira launch's finite sum
                        nb = f0 + 4 * (2 * n + i)
                ap = mode == nat.MODE_APPLY and pl.pers
                arr[i] = nat.Tensor1D(
                    pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(st.get("m_q") if pl.has_m else None),
                    nat.ptr(st.get("m_scale") if pl.has_m else None), st["variance_q"].data_ptr(),
                    st["variance_scale"].data_ptr(), st["variance_min_log"].data_ptr(), v0 + 4 * offs[i], nb,
                    nat.ptr(pl.alpha_t if ap else None), prev, nat.ptr(pl.decay_t if ap else None),
                    pl.p.numel(), int(st.get("sr_seed", 0)), fs, parts.data_ptr() + 8 * poffs[i])
            arrs[mode] = [arr, torch.empty(int(L.a8_table_bytes_1d(n)), dtype=torch.uint8, device=dev), 1]
        ent = {"refs": refs, "acc": acc, "fout": fout, "vbuf": vbuf, "parts": parts, "arrs": arrs}
        if len(ws) > 16:
            ws.clear()
        ws[ck] = ent
    acc, fout = ent["acc"], ent["fout"]
    strm = nat.stream_of(dev)
    has_dec = int(P0.decay_val is not None)
    dec_val = P0.decay_val if has_dec else 1.0

    def launch(mode):
        arr, table, up = ent["arrs"][mode]
        _no_upload_in_capture(up)
        rc = L.a8_fused_update_1d_multi(
            mode, int(P0.sr), nat.dtype_code(P0.p.dtype), arr, n, table.data_ptr(), table.numel(),
            P0.beta1 if P0.has_m else 0.0, P0.beta_val, P0.eps_d, int(P0.adam_denom), P0.al_floor,
            P0.eps_g, P0.eps_sq, P0.bs, P0.mbs if P0.has_m else P0.bs,
            S.m_bits(P0.mqt) if P0.has_m else 0, S.m_mode(P0.mqt) if P0.has_m else 0, P0.d,
            P0.al_vbits, int(P0.mom_only), int(P0.step), float(P0.alpha_val),
            float(dec_val), has_dec, up, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_fused_update_1d_multi")
        ent["arrs"][mode][2] = 0

    acc.zero_()
    launch(nat.MODE_NORM)
    for pl in plans:
        _block_view(pl.st, "variance", pl.bs)
    if mnorm:
        launch(nat.MODE_MNORM)
    if fira:
        # A tensor without a previous norm behaves as one whose previous norm is
        # below 1e-6 (scale 1, next = current), so every slot takes has_prev = 1.
        prev_ok = True
        for i, pl in enumerate(plans):
            pv = pl.st.get("fira_prev_norm")
            if not (torch.is_tensor(pv) and pv.data_ptr() == fout.data_ptr() + 4 * (n + i)):
                prev_ok = False
        if not prev_ok:
            vals = []
            for pl in plans:
                pv = pl.st.get("fira_prev_norm")
                vals.append(torch.zeros((), dtype=torch.float32, device=dev) if pv is None else
                            torch.as_tensor(pv, dtype=torch.float32).to(dev).reshape(()))
            fout[n:2 * n].copy_(torch.stack(vals))
        x = acc[n:2 * n] if mnorm else acc[0:n]
        rc = L.a8_fira_scalar(x.data_ptr(), fout.data_ptr() + 4 * n, None, fout.data_ptr(), n, 1, 2,
                              _f32(1.0 + P0.margin), strm)
        nat.check(rc, "a8_fira_scalar")
        if not prev_ok:
            for i, pl in enumerate(plans):
                pl.st["fira_prev_norm"] = fout[n + i].view(())
    launch(nat.MODE_APPLY)


def _run_batch_sgdc(opt, key, plans):
    """SGD tensors with an RMS clip or Fira as one group: NORM (each tensor's sum of
    u^2 in its own slot, its partials added in index order) -> one Fira launch over
    all tensors -> APPLY, each one multi-tensor launch (the per-tensor sequence of
    _run_sgd, optimizer.py:2045-2077, 796-810).  APPLY reads each tensor's Fira
    scale and finite sum from that launch's output (a8_tensor_sgd.fira, fira_sum)."""
    P0 = plans[0]
    dev = P0.p.device
    L = nat.lib()
    n = len(plans)
    fira = bool(P0.fira)
    moms = [_sgd_momentum(pl) for pl in plans]
    kind = moms[0][3]
    ws = opt._ws.setdefault((dev, "sgdc"), {})
    ck = (tuple((pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(mo[0]), nat.ptr(mo[2])) for pl, mo in zip(plans, moms)),
          P0.sr, kind, fira)
    refs = [tuple(v.data_ptr() for k, v in pl.st.items() if torch.is_tensor(v) and k != "fira_prev_norm")
            for pl in plans]
    ent = ws.get(ck)
    if ent is None or ent["refs"] != refs:
        poffs, ptot = [], 0
        for pl in plans:   # per-tensor slices of the NORM pass's partial-sum workspace
            poffs.append(ptot)
            ptot += _parts_of(pl)
        parts = torch.empty(max(ptot, 1), dtype=torch.float64, device=dev)
        acc = torch.zeros(n, dtype=torch.float32, device=dev)        # sum u^2
        fout = torch.zeros(3 * n, dtype=torch.float32, device=dev)   # Fira: scale | prev norm | finite sum
        a0, f0 = acc.data_ptr(), fout.data_ptr()
        arrs = {}
        for mode in (nat.MODE_NORM, nat.MODE_APPLY):
            arr = (nat.TensorSgd * n)()
            for i, (pl, (m_q, m_scale, m, _)) in enumerate(zip(plans, moms)):
                fs = f0 + 4 * i if (mode == nat.MODE_APPLY and fira) else None
                arr[i] = nat.TensorSgd(pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(m_q), nat.ptr(m_scale), nat.ptr(m),
                                       a0 + 4 * i, fs, None, None, pl.p.numel(), int(pl.st.get("sr_seed", 0)),
                                       parts.data_ptr() + 8 * poffs[i], f0 + 4 * (2 * n + i) if fs else None)
            arrs[mode] = [arr, torch.empty(int(L.a8_table_bytes_sgd(n)), dtype=torch.uint8, device=dev), 1]
        ent = {"refs": refs, "acc": acc, "fout": fout, "parts": parts, "arrs": arrs}
        if len(ws) > 16:
            ws.clear()
        ws[ck] = ent
    acc, fout = ent["acc"], ent["fout"]
    strm = nat.stream_of(dev)
    has_dec = int(P0.decay_val is not None)
    dec_val = P0.decay_val if has_dec else 1.0
    mbs = P0.mbs if kind == 1 else 32

    def launch(mode):
        arr, table, up = ent["arrs"][mode]
        _no_upload_in_capture(up)
        rc = L.a8_sgd_step_multi(
            mode, nat.dtype_code(P0.p.dtype), int(P0.sr), arr, n, table.data_ptr(), table.numel(),
            P0.beta1 if P0.has_m else 0.0, kind, S.m_bits(P0.mqt) if kind == 1 else 0,
            S.m_mode(P0.mqt) if kind == 1 else 0, mbs, P0.d, float(P0.alpha_val), float(dec_val), has_dec,
            int(P0.step), up, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_sgd_step_multi")
        ent["arrs"][mode][2] = 0

    acc.zero_()
    launch(nat.MODE_NORM)
    if fira:
        # as in _run_batch_q1dc: a tensor without a previous norm takes 0 (scale 1,
        # next = current), so every slot has one
        prev_ok = all(torch.is_tensor(pl.st.get("fira_prev_norm")) and
                      pl.st["fira_prev_norm"].data_ptr() == fout.data_ptr() + 4 * (n + i)
                      for i, pl in enumerate(plans))
        if not prev_ok:
            vals = []
            for pl in plans:
                pv = pl.st.get("fira_prev_norm")
                vals.append(torch.zeros((), dtype=torch.float32, device=dev) if pv is None else
                            torch.as_tensor(pv, dtype=torch.float32).to(dev).reshape(()))
            fout[n:2 * n].copy_(torch.stack(vals))
        rc = L.a8_fira_scalar(acc.data_ptr(), fout.data_ptr() + 4 * n, None, fout.data_ptr(), n, 1, 2,
                              _f32(1.0 + P0.margin), strm)
        nat.check(rc, "a8_fira_scalar")
        if not prev_ok:
            for i, pl in enumerate(plans):
                pl.st["fira_prev_norm"] = fout[n + i].view(())
    launch(nat.MODE_APPLY)


def _run_batch(opt, key, plans):
    path = key[0]
    if path == "factored":
        _run_factored(opt, plans)
        return
    if path == "f1dc":   # also for one tensor: scale_parameter's sum of p^2 is the kernel's fixed-order sum
        _run_batch_f1dc(opt, key, plans)
        return
    if len(plans) == 1 and plans[0].dsc is None:
        _run_single(opt, plans[0])
        return
    if path == "q1dc":
        _run_batch_q1dc(opt, key, plans)
        return
    if path == "sgdc":
        _run_batch_sgdc(opt, key, plans)
        return
    P0 = plans[0]
    dev = P0.p.device
    L = nat.lib()
    n = len(plans)
    ptrs = tuple((pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(pl.vbuf), nat.ptr(pl.alpha_t if pl.pers else None),
                  nat.ptr(pl.decay_t if pl.pers else None)) for pl in plans)
    # The table holds only pointers, sizes and seeds; step-dependent scalars go
    # to the launch, so one upload serves every later step.
    cache_key = (path, dev, key[5], ptrs)   # key[5]: stochastic rounding (seeds in the table)
    ws = opt._ws.setdefault((dev, "tables"), {})
    ent = ws.get(cache_key)
    upload = 0
    if ent is None:
        if path == "sgd":
            arr = (nat.TensorSgd * n)()
            for i, pl in enumerate(plans):
                m_q, m_scale, m, _ = _sgd_momentum(pl)
                arr[i] = nat.TensorSgd(pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(m_q), nat.ptr(m_scale),
                                       nat.ptr(m), None, None, None, None, pl.p.numel(),
                                       int(pl.st.get("sr_seed", 0)))
            nbytes = L.a8_table_bytes_sgd(n)
        elif path == "q1d":
            arr = (nat.Tensor1D * n)()
            for i, pl in enumerate(plans):
                st = pl.st
                arr[i] = nat.Tensor1D(
                    pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(st.get("m_q") if pl.has_m else None),
                    nat.ptr(st.get("m_scale") if pl.has_m else None), st["variance_q"].data_ptr(),
                    st["variance_scale"].data_ptr(), st["variance_min_log"].data_ptr(), None, None,
                    nat.ptr(pl.alpha_t if pl.pers else None), None, nat.ptr(pl.decay_t if pl.pers else None),
                    pl.p.numel(), int(st.get("sr_seed", 0)))
            nbytes = L.a8_table_bytes_1d(n)
        else:
            arr = (nat.TensorFull * n)()
            for i, pl in enumerate(plans):
                st = pl.st
                arr[i] = nat.TensorFull(pl.p.data_ptr(), pl.g.data_ptr(), _variance_of(pl).data_ptr(),
                                        nat.ptr(st.get("m") if pl.has_m else None), None, None, None,
                                        None, pl.p.numel(), int(st.get("sr_seed", 0)))
            nbytes = L.a8_table_bytes_full(n)
        table = torch.empty(int(nbytes), dtype=torch.uint8, device=dev)
        # state tensors referenced by the table must stay the same objects
        refs = None
        ent = [arr, table, nbytes, refs]
        if len(ws) > 64:
            ws.clear()
        ws[cache_key] = ent
        upload = 1
    else:
        refs = [tuple(v.data_ptr() for v in pl.st.values() if torch.is_tensor(v)) for pl in plans]
        if refs != ent[3]:
            ws.pop(cache_key)
            return _run_batch(opt, key, plans)
    arr, table, nbytes, _ = ent
    has_dec = int(P0.decay_val is not None)
    dec_val = P0.decay_val if has_dec else 1.0
    strm = nat.stream_of(dev)
    _no_upload_in_capture(upload)
    if path == "sgd":
        kind = 0 if not P0.has_m else (1 if key[7] else 2)
        rc = L.a8_sgd_step_multi(
            nat.MODE_NOCLIP, nat.dtype_code(P0.p.dtype), int(P0.sr), arr, n, table.data_ptr(), nbytes,
            P0.beta1 if P0.has_m else 0.0, kind, S.m_bits(P0.mqt) if kind == 1 else 0,
            S.m_mode(P0.mqt) if kind == 1 else 0, P0.mbs if kind == 1 else 32, P0.d, float(P0.alpha_val),
            float(dec_val), has_dec, int(P0.step), upload, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_sgd_step_multi")
        if upload:
            ent[3] = [tuple(v.data_ptr() for v in pl.st.values() if torch.is_tensor(v)) for pl in plans]
    elif path == "q1d":
        rc = L.a8_fused_update_1d_multi(
            nat.MODE_NOCLIP, int(P0.sr), nat.dtype_code(P0.p.dtype), arr, n, table.data_ptr(), nbytes,
            P0.beta1 if P0.has_m else 0.0, P0.beta_val, P0.eps_d, int(P0.adam_denom), P0.al_floor,
            P0.eps_g, P0.eps_sq, P0.bs, P0.mbs if P0.has_m else P0.bs,
            S.m_bits(P0.mqt) if P0.has_m else 0, S.m_mode(P0.mqt) if P0.has_m else 0, P0.d,
            P0.al_vbits, int(P0.mom_only), int(P0.step), float(P0.alpha_val),
            float(dec_val), has_dec, upload, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_fused_update_1d_multi")
        for pl in plans:
            _block_view(pl.st, "variance", pl.bs)
        if upload:
            ent[3] = [tuple(v.data_ptr() for v in pl.st.values() if torch.is_tensor(v)) for pl in plans]
    else:
        rc = L.a8_fused_update_1d_full_multi(
            nat.MODE_NOCLIP, nat.dtype_code(P0.p.dtype), arr, n, table.data_ptr(), nbytes,
            P0.beta1 if P0.has_m else 0.0, P0.beta_val, P0.eps_sq, P0.eps_d, int(P0.adam_denom),
            P0.eps_g, P0.d, int(P0.mom_only), float(P0.alpha_val), float(dec_val), has_dec, int(P0.sr),
            int(P0.step), 0, 0.0, 0, 0.0, int(P0.vbuf is not None), upload, nat.ptr(P0.dsc), strm)
        nat.check(rc, "a8_fused_update_1d_full_multi")
        if upload:
            ent[3] = [tuple(v.data_ptr() for v in pl.st.values() if torch.is_tensor(v)) for pl in plans]


def _apollo_proj(st, shape, step, device, cache):
    """_get_apollo_proj_matrix (optimizer.py:2557-2584): the projection P^T of this
    step and whether it was (re)generated."""
    rank = int(st["apollo_rank"])
    gap = int(st["apollo_update_proj_gap"])
    last = int(st.get("last_proj_step", -gap))
    refresh = (step - last) >= gap
    if not refresh and cache and st.get("apollo_proj_matrix_T") is not None:
        return st["apollo_proj_matrix_T"], False
    if refresh:
        st["current_proj_seed"] = int(st["apollo_seed"])
        st["apollo_seed"] = next_seed(st["current_proj_seed"])
        st["last_proj_step"] = step
    R, C = shape[-2], shape[-1]
    m_shape = (rank, C) if R >= C else (R, rank)
    seed = st.get("current_proj_seed", st["apollo_seed"])
    proj = stable_randn(m_shape, seed=seed, device=device, dtype=torch.float32)
    # IEEE division by a device scalar (a Python scalar would become a reciprocal multiply)
    proj = proj / torch.tensor(math.sqrt(rank), dtype=torch.float32, device=device)
    proj_T = proj.T.to(torch.float32).contiguous()
    if cache:
        st["apollo_proj_matrix_T"] = proj_T
    return proj_T, True


def _apollo_proj_device(opt, st, shape, step, device, group):
    """P^T of a capturable step.  It lives in a persistent buffer, and the projection
    schedule -- the refresh decision, the reference's seed chain (next_seed) and the
    generation of a new P -- runs on the device (a8_apollo_step_multi with
    step_scalars), so replayed steps refresh the projection as eager ones do.  The
    first such step of a matrix (eager) takes P^T from the host schedule
    (_get_apollo_proj_matrix, optimizer.py:2557-2584) and hands the schedule over:
    refreshes after that draw P with the device generator (a8_apollo_proj_gen), in
    place of stable_randn's torch generator, which is seeded on the host."""
    key = (device, "apollo_pdev", id(st))
    ent = opt._ws.get(key)
    if ent is None:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("adafactor8bit: run one eager step of a capturable APOLLO group before capturing")
        cache = group.get("apollo_cache_proj", False)
        proj_T, _ = _apollo_proj(st, shape, step, device, cache)
        gap = int(st["apollo_update_proj_gap"])
        if gap <= 0:
            raise NotImplementedError("adafactor8bit: capturable APOLLO needs apollo_update_proj_gap > 0")
        pt = proj_T.detach().to(torch.float32).contiguous().clone()
        seed = int(st["apollo_seed"])
        # {last_proj_step, apollo_seed, current_proj_seed, fresh = 2: split P^T as given}
        ps = torch.tensor([int(st.get("last_proj_step", -gap)), seed, int(st.get("current_proj_seed", seed)), 2],
                          dtype=torch.int64, device=device)
        ent = {"pt": pt, "ps": ps, "st": st}
        opt._ws[key] = ent
        if cache:
            st["apollo_proj_matrix_T"] = pt
    return ent["pt"], ent["ps"]


def _sync_apollo_schedule(opt):
    """Copy the device projection schedules of capturable APOLLO matrices back to
    their state (last_proj_step, apollo_seed, current_proj_seed)."""
    for key, ent in list(opt._ws.items()):
        if isinstance(key, tuple) and len(key) == 3 and key[1] == "apollo_pdev":
            last, seed, cur, _ = (int(x) for x in ent["ps"].tolist())
            st = ent["st"]
            st["last_proj_step"], st["apollo_seed"], st["current_proj_seed"] = last, seed, cur


def _apollo_prep(opt, p, grad, st, group, dsc=None):
    """Host side of one APOLLO parameter's step (optimizer.py:2587-3084): step
    counter, projection refresh, lazy low-rank state, per-step scalars.  Returns
    (batch key, tensor record, finish) for the grouped launch.  The factorised
    and CAME variants carry an a8_apollo_x_args record for the low-rank stage
    between the projection and finish phases.  With ``dsc`` (capturable groups)
    the per-step scalars and the projection schedule come from the device."""
    beta1, beta2, beta2_decay = group.get("beta1"), group["beta2"], group["beta2_decay"]
    factorize = bool(group.get("apollo_factorize", False))
    came = group.get("beta3") is not None
    if came and beta1 is None:
        raise ValueError("CAME (beta3) strictly requires momentum (beta1) to compute update instability.")
    if dsc is not None and int(st["apollo_update_proj_gap"]) <= 0:
        raise NotImplementedError("adafactor8bit: capturable APOLLO needs apollo_update_proj_gap > 0")
    if p.dtype not in (torch.float32, torch.bfloat16, torch.float16, torch.float64):
        raise NotImplementedError("adafactor8bit: APOLLO needs fp32, bf16, fp16 or fp64 parameters")
    if p.dtype == torch.float64 and group["scale_parameter"]:
        # the reference's alpha (optimizer.py:850-852) takes the norm with dtype=float32,
        # which torch refuses for a float64 tensor: the same error here
        torch.linalg.vector_norm(p, ord=2, dtype=torch.float32)
    if not p.is_contiguous():
        raise NotImplementedError("adafactor8bit: non-contiguous parameters are not supported")
    if p.dtype in (torch.float16, torch.float64):
        # the projection runs on fp32 G, as the reference's grad.float() (optimizer.py:2601)
        gdt = torch.float32
    elif grad.dtype != p.dtype:
        if p.dtype != torch.float32:
            raise NotImplementedError("adafactor8bit: gradient dtype must match the parameter dtype")
        gdt = torch.float32
    else:
        gdt = grad.dtype
    g = _grad_work(opt, p, grad, gdt, group["maximize"])
    dev = p.device
    R = p.shape[0]
    C = p.numel() // R
    rank = int(st["apollo_rank"])
    step = st["step"] + 1
    st["step"] = step
    vqt = st.get("v_quant_type", "al8")
    mqt = st.get("m_quant_type", "uf8") if beta1 is not None else "uf8"
    beta_val = 1.0 - beta2 if beta2 is not None else math.pow(step, beta2_decay)
    lr = group["lr"]
    rho_t = None
    if isinstance(lr, Tensor):
        rho_t = lr.to(device=dev, dtype=torch.float32).reshape(())
        if group["relative_step"]:
            rho_t = torch.minimum(torch.tensor(float(step), device=dev).rsqrt(), rho_t)
        rho_t = rho_t.contiguous()
        rho_val = 0.0
    else:
        rho_val = _f32(min(lr, 1.0 / math.sqrt(step)) if group["relative_step"] else lr)
    right = R >= C
    pstate = None
    if dsc is not None:
        proj_T, pstate = _apollo_proj_device(opt, st, (R, C), step, dev, group)
        fresh = False
    else:
        proj_T, fresh = _apollo_proj(st, (R, C), step, dev, group.get("apollo_cache_proj", False))
    n_low = R * rank if right else rank * C
    quant = st.get("is_quantized", False)
    bs = st.get("block_size", group.get("block_size", 2048))
    if factorize:
        first = st.get("row_var_low") is None
    else:
        first = st.get("v_low_q") is None and st.get("v_low") is None
    vbits = 0 if (not quant or vqt == "fp32") else (16 if vqt == "al16" else 8)
    has_m = beta1 is not None
    m_fp32 = has_m and (not quant or mqt == "fp32")
    mbs = st.get("m_block_size", group.get("m_block_size", 256))
    # the fused low-rank stage (k_ap_low) takes power-of-two blocks; other sizes
    # run the plain stage of a8_apollo_lowrank_x
    xmode = bool(factorize or came or (vbits and not _pow2_in(bs, 128, 2048))) or \
        (has_m and not m_fp32 and not _pow2_in(mbs, 32, 2048))
    low_shape = (R, rank) if right else (rank, C)
    if factorize:   # optimizer.py:2693-2699 creates the row / column EMAs on the first step
        if first:
            st["row_var_low"] = torch.zeros((low_shape[0], 1), dtype=torch.float32, device=dev)
            st["col_var_low"] = torch.zeros((1, low_shape[1]), dtype=torch.float32, device=dev)
    elif first:   # optimizer.py:2770-2779 creates the low-rank V state on the first step
        if vbits:
            S.new_al_slot(st, "v_low", (n_low,), bs, vqt, dev)
        else:
            st["v_low"] = torch.zeros(n_low, dtype=torch.float32, device=dev)
    if has_m:
        if m_fp32:
            if st.get("m_low") is None:
                st["m_low"] = torch.zeros((R, rank) if right else (rank, C), dtype=torch.float32, device=dev)
        elif st.get("m_low_q") is None:
            S.new_momentum_codes(st, "m_low", n_low, mbs, mqt, dev)
    fira = bool(group.get("enable_fira_for_apollo", True))
    has_prev = 0
    if fira:
        prev = st.get("scaled_grad_norm_prev")
        if prev is None:
            st["scaled_grad_norm_prev"] = torch.zeros((), dtype=torch.float32, device=dev)
        else:
            if not torch.is_tensor(prev) or prev.device != dev or prev.dtype != torch.float32:
                st["scaled_grad_norm_prev"] = torch.as_tensor(prev, dtype=torch.float32).to(dev).reshape(())
            has_prev = 1
    bias_mode, bias_fac = 0, 1.0
    if has_m and not group["relative_step"]:
        bc_on = True if group.get("bias_correction") is None else group.get("bias_correction")
        if bc_on:
            bc1 = 1.0 - beta1 ** step
            if beta2 is not None:
                bias_mode, bias_fac = 1, _f32(math.sqrt(1.0 - beta2 ** step) / bc1)
            else:
                bias_mode, bias_fac = 2, _f32(bc1)
    key = (dev, "apollo", id(p))
    ent = opt._ws.get(key)
    nws = int(nat.lib().a8_apollo_workspace_floats(R, C, rank, 1))
    if ent is None or ent["ws"].numel() < nws:
        ent = {"ws": torch.empty(nws, dtype=torch.float32, device=dev), "proj": None}
        opt._ws[key] = ent
    if dsc is None and (ent["proj"] is None or ent["proj"] != (proj_T.data_ptr(), proj_T._version)):
        fresh = True
    ent["proj"] = (proj_T.data_ptr(), proj_T._version)
    sr = bool(group.get("stochastic_round_writeback", False)) and p.dtype in (torch.bfloat16, torch.float16)
    if dsc is not None:
        # the device block supplies step, bias factor, V weight and lr: the records
        # (and so the uploaded tables) stay the same from step to step
        step_rec, bias_rec, beta_key, rho_key = 0, 0.0, 0.0, 0.0
    else:
        step_rec, bias_rec, beta_key, rho_key = int(step), float(bias_fac), float(beta_val), float(rho_val)
    if xmode:
        xargs, xkeep = _apollo_x_args(opt, st, group, dev, ent["ws"], low_shape, n_low, factorize, came, first,
                                      vbits, vqt, bs, has_m, m_fp32, mqt, mbs, quant, beta_key, beta1)
        # the stage leaves the per-row sums of u^2 and g_low^2 where the finish phase
        # reads them (right side, rank a power of two in [8, 512]: phase 3)
        xargs.u_rowsums = int(right and _pow2_in(rank, 8, 512))
        t = nat.ApolloTensor(
            p.data_ptr(), g.data_ptr(), R, C, proj_T.data_ptr(), rank, None, None, None, None, None, None, None,
            nat.ptr(st.get("scaled_grad_norm_prev")) if fira else None, has_prev,
            nat.ptr(rho_t), ent["ws"].data_ptr(), int(st.get("sr_seed", 0)),
            int(first), int(fresh), step_rec, bias_rec, nat.ptr(pstate),
            int(st["apollo_update_proj_gap"]) if pstate is not None else 0)
        bkey = (p.dtype, sr, "x", has_m, True, mqt, 0, 0, beta_key, rho_key, bias_mode)
        keep = (g, proj_T, rho_t, xkeep, pstate)
        return bkey, t, (st, "x", bs, keep, xargs)
    t = nat.ApolloTensor(
        p.data_ptr(), g.data_ptr(), R, C, proj_T.data_ptr(), rank,
        nat.ptr(st.get("v_low_q")) if vbits else None, nat.ptr(st.get("v_low_scale")) if vbits else None,
        nat.ptr(st.get("v_low_min_log")) if vbits else None, None if vbits else st["v_low"].data_ptr(),
        nat.ptr(st.get("m_low_q")) if (has_m and not m_fp32) else None,
        nat.ptr(st.get("m_low_scale")) if (has_m and not m_fp32) else None,
        st["m_low"].data_ptr() if m_fp32 else None,
        nat.ptr(st.get("scaled_grad_norm_prev")) if fira else None, has_prev,
        nat.ptr(rho_t), ent["ws"].data_ptr(), int(st.get("sr_seed", 0)),
        int(first), int(fresh), step_rec, bias_rec, nat.ptr(pstate),
        int(st["apollo_update_proj_gap"]) if pstate is not None else 0)
    bkey = (p.dtype, sr, vbits, has_m, m_fp32, mqt, int(mbs), int(bs), beta_key, rho_key, bias_mode)
    keep = (g, proj_T, rho_t, pstate)   # alive until the launch is queued
    return bkey, t, (st, vbits, bs, keep, None)


def _apollo_x_args(opt, st, group, dev, ws, low_shape, n_low, factorize, came, first, vbits, vqt, bs, has_m,
                   m_fp32, mqt, mbs, quant, beta_val, beta1):
    """Lazy factorised / CAME low-rank state (optimizer.py:2689-2758, 2800-2815)
    and the a8_apollo_x_args record of one matrix."""
    cqt = st.get("c_quant_type") or vqt
    cbits = 0 if (not quant or cqt == "fp32") else (16 if cqt == "al16" else 8)
    if came and not factorize and st.get("res_low_q") is None and st.get("res_low") is None:
        if cbits:
            S.new_al_slot(st, "res_low", low_shape, bs, cqt, dev)
        else:
            st["res_low"] = torch.zeros(low_shape, dtype=torch.float32, device=dev)
    if came and factorize:
        rs, cs = (low_shape[0], 1), (1, low_shape[1])
        if cbits:
            if st.get("conf_row_low_q") is None:
                S.new_al_slot(st, "conf_row_low", rs, bs, cqt, dev)
                S.new_al_slot(st, "conf_col_low", cs, bs, cqt, dev)
        elif st.get("conf_row_low") is None:
            st["conf_row_low"] = torch.zeros(rs, dtype=torch.float32, device=dev)
            st["conf_col_low"] = torch.zeros(cs, dtype=torch.float32, device=dev)
    for k in ("row_var_low", "col_var_low", "m_low", "res_low", "conf_row_low", "conf_col_low", "v_low"):
        if torch.is_tensor(st.get(k)) and not st[k].is_contiguous():
            st[k] = st[k].contiguous()
    key = (dev, "apollo_x", id(st))   # one per matrix: the batched stage runs them together
    xws = opt._ws.get(key)
    nx = int(nat.lib().a8_apollo_x_workspace_floats(low_shape[0], low_shape[1]))
    if xws is None or xws.numel() < nx:
        xws = torch.empty(nx, dtype=torch.float32, device=dev)
        opt._ws[key] = xws
    aeps = group.get("apollo_eps", 1e-6)
    eps_sq = max(aeps * aeps, _LOG_QUANT_FLOOR)
    # the record is rebuilt only when a state tensor, a workspace or a hyper-parameter changed
    sig = (ws.data_ptr(), xws.data_ptr(), low_shape, factorize, came, has_m, m_fp32, vbits, cbits, mqt, int(bs),
           int(mbs), beta1, group.get("beta3"), aeps, group.get("eps_came", 1e-16), group["d"],
           tuple(v.data_ptr() for v in st.values() if torch.is_tensor(v)))
    cached = opt._ws.get((dev, "apollo_xargs", id(st)))
    if cached is not None and cached[0] == sig:
        a = cached[1]
        a.first_step = int(first)
        a.beta_v = float(beta_val)
        return a, (xws, cbits)
    P = nat.ptr
    a = nat.ApolloXArgs(
        ws.data_ptr(), ws.data_ptr() + 4 * n_low, xws.data_ptr(), low_shape[0], low_shape[1],
        int(factorize), int(came), int(has_m), int(first),
        P(st.get("v_low_q")) if (vbits and not factorize) else None,
        P(st.get("v_low_scale")) if (vbits and not factorize) else None,
        P(st.get("v_low_min_log")) if (vbits and not factorize) else None,
        P(st.get("v_low")) if (not vbits and not factorize) else None, 0 if factorize else vbits, int(bs),
        P(st.get("row_var_low")) if factorize else None, P(st.get("col_var_low")) if factorize else None,
        P(st.get("m_low_q")) if (has_m and not m_fp32) else None,
        P(st.get("m_low_scale")) if (has_m and not m_fp32) else None,
        P(st.get("m_low")) if (has_m and m_fp32) else None,
        S.m_bits(mqt) if has_m else 8, S.m_mode(mqt) if has_m else 0, int(mbs),
        P(st.get("res_low_q")) if (came and not factorize and cbits) else None,
        P(st.get("res_low_scale")) if (came and not factorize and cbits) else None,
        P(st.get("res_low_min_log")) if (came and not factorize and cbits) else None,
        P(st.get("res_low")) if (came and not factorize and not cbits) else None,
        P(st.get("conf_row_low_q")) if (came and factorize and cbits) else None,
        P(st.get("conf_row_low_scale")) if (came and factorize and cbits) else None,
        P(st.get("conf_row_low_min_log")) if (came and factorize and cbits) else None,
        P(st.get("conf_row_low")) if (came and factorize and not cbits) else None,
        P(st.get("conf_col_low_q")) if (came and factorize and cbits) else None,
        P(st.get("conf_col_low_scale")) if (came and factorize and cbits) else None,
        P(st.get("conf_col_low_min_log")) if (came and factorize and cbits) else None,
        P(st.get("conf_col_low")) if (came and factorize and not cbits) else None,
        cbits if came else 0, float(beta_val), float(beta1) if has_m else 0.0,
        float(group["beta3"]) if came else 0.0, _f32(aeps), _f32(eps_sq), _f32(math.log2(eps_sq)),
        _f32(group.get("eps_came", 1e-16)), float(group["d"]))
    opt._ws[(dev, "apollo_xargs", id(st))] = (sig, a)
    return a, (xws, cbits)


def _run_apollo_batch(opt, group, bkey, items, dsc=None):
    """One a8_apollo_step_multi launch sequence for the APOLLO matrices of a group
    that share dtype, state formats and step scalars.  With ``dsc`` (capturable)
    the table is uploaded only when its records change, and never under capture."""
    pdt, sr, vbits, has_m, m_fp32, mqt, mbs, bs, beta_val, rho_val, bias_mode = bkey
    n = len(items)
    arr = (nat.ApolloTensor * n)(*[t for t, _ in items])
    L = nat.lib()
    pdev = items[0][1][3][0].device   # the first record's gradient
    tkey = (pdev, "ap_table", id(group), bkey) if dsc is not None else (pdev, "ap_table")
    need = int(L.a8_apollo_table_bytes(n))
    tab = opt._ws.get(tkey)
    if tab is None or tab.numel() < need:
        tab = torch.empty(max(need, 4096), dtype=torch.uint8, device=pdev)
        opt._ws[tkey] = tab
    upload = 1
    if dsc is not None:
        blob = bytes(arr)
        bk = (pdev, "ap_table_blob", id(group), bkey)
        if n > 1 and opt._ws.get(bk) == blob:
            upload = 0
        _no_upload_in_capture(upload if n > 1 else 0)
        opt._ws[bk] = blob
    beta1 = group.get("beta1")
    aeps = group.get("apollo_eps", 1e-6)
    eps_sq = max(aeps * aeps, _LOG_QUANT_FLOOR)
    wd = group["weight_decay"]
    wd_mode = 0 if wd == 0 else (1 if group.get("scale_weight_decay", True) else 2)
    fira = bool(group.get("enable_fira_for_apollo", True))
    stream = nat.stream_of(pdev)
    tail = (int(group.get("apollo_scale_type", "channel") == "channel"), float(group.get("apollo_scale", 1.0)),
            int(bool(group.get("apollo_scale_front", False))), int(fira), float(group.get("fira_margin", 0.01)),
            float(group["d"]), float(rho_val), _f32(group["eps"][1]), int(bool(group["scale_parameter"])),
            bias_mode, _f32(wd), wd_mode, stream)
    if dsc is not None:
        beta_val, tail = 0.0, tail[:6] + (0.0,) + tail[7:]   # from the device block
    if vbits == "x":
        # projection, the factorised / CAME low-rank stage per matrix, then scale and
        # writeback; phase 3 reads the table phase 1 left.  Capturable groups keep the
        # stage's tables per group and upload them only when a record changes.
        head = (nat.dtype_code(pdt), int(sr), arr, n, tab.data_ptr(), tab.numel(), float(beta_val),
                float(beta1) if has_m else 0.0, int(has_m), _f32(aeps), _f32(math.log2(eps_sq)), 0, 2048, 8, 0, 1,
                256)
        dptr = nat.ptr(dsc)
        nat.check(L.a8_apollo_step_multi_phase(1, *head, *tail[:-1], upload, dptr, tail[-1]),
                  "a8_apollo_step_multi_phase(1)")
        xarr = (nat.ApolloXArgs * n)(*[it[1][4] for it in items])
        xneed = int(L.a8_apollo_x_table_bytes(n))
        xkey = (pdev, "apx_table", id(group), bkey) if dsc is not None else (pdev, "apx_table")
        xtab = opt._ws.get(xkey)
        if xtab is None or xtab.numel() < xneed:
            xtab = torch.empty(max(xneed, 4096), dtype=torch.uint8, device=pdev)
            opt._ws[xkey] = xtab
        xupload = 1
        if dsc is not None:
            xblob = bytes(xarr)
            xbk = (pdev, "apx_table_blob", id(group), bkey)
            if opt._ws.get(xbk) == (xtab.data_ptr(), xblob):
                xupload = 0
            _no_upload_in_capture(xupload)
            opt._ws[xbk] = (xtab.data_ptr(), xblob)
        nat.check(L.a8_apollo_lowrank_x_multi(xarr, n, xtab.data_ptr(), xtab.numel(), xupload, dptr, stream),
                  "a8_apollo_lowrank_x_multi")
        nat.check(L.a8_apollo_step_multi_phase(3, *head, *tail[:-1], 0, dptr, tail[-1]),
                  "a8_apollo_step_multi_phase(3)")
        for _, (st, _vb, bsz, keep, xargs) in items:
            if xargs.v_bits:
                _block_view(st, "v_low", bsz)
            if xargs.c_bits and not xargs.factorize:
                _block_view(st, "res_low", bsz)
            if xargs.c_bits and xargs.factorize:
                _block_view(st, "conf_row_low", bsz)
                _block_view(st, "conf_col_low", bsz)
        return
    rc = L.a8_apollo_step_multi(
        nat.dtype_code(pdt), int(sr), arr, n, tab.data_ptr(), tab.numel(), float(beta_val),
        float(beta1) if has_m else 0.0, int(has_m), _f32(aeps), _f32(math.log2(eps_sq)), vbits, int(bs),
        S.m_bits(mqt) if has_m else 8, S.m_mode(mqt) if has_m else 0, int(m_fp32), int(mbs), *tail[:-1], upload,
        nat.ptr(dsc), tail[-1])
    nat.check(rc, "a8_apollo_step_multi")
    if vbits:
        for _, (st, vb, bsz, _keep, _x) in items:
            _block_view(st, "v_low", bsz)


def _run_factored(opt, plans):
    """One factored step for a group of matrices (optimizer.py:2198-2252, 920-970):
    statistics, row/column V EMA, update (and the norm pass for RMS clipping or
    Fira) in a8_factored_step's few launches."""
    P0 = plans[0]
    came = P0.beta3 is not None and P0.has_m
    vbits = 0 if (not P0.quant or P0.vqt == "fp32") else (16 if P0.vqt == "al16" else 8)
    cbits = 0
    if came:
        cqt = P0.st.get("c_quant_type") or P0.vqt
        cbits = 0 if (not P0.quant or cqt == "fp32") else (16 if cqt == "al16" else 8)
    m32 = P0.has_m and (not P0.quant or P0.mqt == "fp32" or "m_q" not in P0.st)
    for pl in plans:
        if pl.has_m and m32:
            st = pl.st
            if "m" not in st:
                st["m"] = torch.zeros_like(pl.g, dtype=torch.float32)
            if not st["m"].is_contiguous():
                st["m"] = st["m"].contiguous()
        if not pl.p.is_contiguous():
            raise NotImplementedError("adafactor8bit: non-contiguous parameters are not supported")
        if pl.g.dtype != pl.p.dtype:
            if pl.p.dtype == torch.float32:
                pl.g = pl.g.float()
            else:
                raise NotImplementedError("adafactor8bit: gradient dtype must match the parameter dtype")
    dev = P0.p.device
    L = nat.lib()
    n = len(plans)
    fira = bool(P0.fira)
    has_prev = []
    for pl in plans:
        st = pl.st
        if fira:
            prev = st.get("fira_prev_norm")
            if prev is None:
                # a zero previous norm takes the limiter's reset branch (scale 1, next =
                # this norm), which is what the first step does without one; one table
                # then serves every step
                st["fira_prev_norm"] = torch.zeros((), dtype=torch.float32, device=dev)
                has_prev.append(1)
            else:
                if not torch.is_tensor(prev) or prev.device != dev or prev.dtype != torch.float32:
                    prev = torch.as_tensor(prev, dtype=torch.float32).to(dev).reshape(())
                    st["fira_prev_norm"] = prev
                has_prev.append(1)
        else:
            has_prev.append(0)
        if vbits == 0:
            for k in ("row_var", "col_var"):
                if not st[k].is_contiguous():
                    st[k] = st[k].contiguous()
        if came and cbits == 0:
            for k in ("conf_row", "conf_col"):
                if not st[k].is_contiguous():
                    st[k] = st[k].contiguous()

    sig = tuple((pl.p.data_ptr(), pl.g.data_ptr(), nat.ptr(pl.rho_t), hp,
                 tuple(v.data_ptr() for v in pl.st.values() if torch.is_tensor(v)))
                for pl, hp in zip(plans, has_prev))
    wsd = opt._ws.setdefault((dev, "tables2d"), {})
    # one table per batch of parameters (two groups whose batches have the same
    # shapes, an embedding and a head say, must not take turns re-uploading one)
    tkey = tuple((pl.p.data_ptr(), tuple(pl.g.shape)) for pl in plans)
    ent = wsd.get(tkey)
    upload = 0
    if ent is None or ent["sig"] != sig:
        sizes = []
        for pl in plans:
            sh = pl.g.shape
            R, C = int(sh[-2]), int(sh[-1])
            B = pl.g.numel() // (R * C)
            sizes.append((B, R, C, int(L.a8_factored_workspace_floats(B, R, C))))
        offs, tot = [], 0
        for (_, _, _, w) in sizes:
            offs.append(tot)
            tot += (w + 63) // 64 * 64
        if ent is not None and ent["ws"].numel() >= tot and ent["n"] == n:
            wbuf, table = ent["ws"], ent["table"]
        else:
            wbuf = torch.empty(max(tot, 1), dtype=torch.float32, device=dev)
            table = torch.empty(int(L.a8_table_bytes_2d(n)), dtype=torch.uint8, device=dev)
        arr = (nat.Tensor2D * n)()
        base = wbuf.data_ptr()
        for i, (pl, (B, R, C, _)) in enumerate(zip(plans, sizes)):
            st = pl.st
            q = vbits != 0
            cq = cbits != 0
            conf = [None] * 8
            if came:
                conf = [nat.ptr(st["conf_row_q"]) if cq else None,
                        nat.ptr(st["conf_row_scale"]) if cq else None,
                        nat.ptr(st["conf_row_min_log"]) if cq else None,
                        None if cq else st["conf_row"].data_ptr(),
                        nat.ptr(st["conf_col_q"]) if cq else None,
                        nat.ptr(st["conf_col_scale"]) if cq else None,
                        nat.ptr(st["conf_col_min_log"]) if cq else None,
                        None if cq else st["conf_col"].data_ptr()]
            arr[i] = nat.Tensor2D(
                pl.p.data_ptr(), pl.g.data_ptr(),
                nat.ptr(st.get("m_q") if pl.has_m and not m32 else None),
                nat.ptr(st.get("m_scale") if pl.has_m and not m32 else None),
                nat.ptr(st["row_var_q"]) if q else None, nat.ptr(st["row_var_scale"]) if q else None,
                nat.ptr(st["row_var_min_log"]) if q else None, None if q else st["row_var"].data_ptr(),
                nat.ptr(st["col_var_q"]) if q else None, nat.ptr(st["col_var_scale"]) if q else None,
                nat.ptr(st["col_var_min_log"]) if q else None, None if q else st["col_var"].data_ptr(),
                *conf, base + 4 * offs[i], nat.ptr(pl.rho_t),
                nat.ptr(st.get("fira_prev_norm")) if fira else None, has_prev[i],
                B, R, C, int(st.get("sr_seed", 0)), nat.ptr(st["m"]) if pl.has_m and m32 else None)
        ent = {"sig": sig, "arr": arr, "ws": wbuf, "table": table, "n": n}
        if len(wsd) > 64:
            wsd.clear()
        wsd[tkey] = ent
        upload = 1
    arr, table = ent["arr"], ent["table"]
    _no_upload_in_capture(upload)
    rc = L.a8_factored_step(
        nat.dtype_code(P0.p.dtype), int(P0.sr), arr, n, table.data_ptr(), table.numel(), upload,
        P0.beta_val, _f32(P0.eps1), _f32(P0.eps2), float(P0.rho_val), int(P0.scale_param),
        int(P0.bias_mode), float(P0.bias_fac), float(P0.wd), int(P0.wd_mode), float(P0.d), int(fira),
        float(P0.margin), _AL_FLOOR, vbits, int(P0.bs), P0.beta1 if P0.has_m else 0.0,
        int(P0.mbs) if P0.has_m else 32, S.m_bits(P0.mqt) if P0.has_m else 8,
        S.m_mode(P0.mqt) if P0.has_m else 0, int(P0.step), int(came),
        float(P0.beta3) if came else 0.0, _f32(P0.group.get("eps_came", 1e-16)), cbits, nat.ptr(P0.dsc),
        nat.stream_of(dev))
    nat.check(rc, "a8_factored_step")
    if vbits:
        for pl in plans:
            _block_view(pl.st, "row_var", pl.bs)
            _block_view(pl.st, "col_var", pl.bs)
    if cbits:
        for pl in plans:
            _block_view(pl.st, "conf_row", pl.bs)
            _block_view(pl.st, "conf_col", pl.bs)
