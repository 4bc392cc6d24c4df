"""Optimizer-state layout: creation, type tags and the dynamic codebook.

The keys, dtypes, shapes and padding are the reference's checkpoint format
(adafactor8bit/optimizer.py:389-401 ``_init_v_state``, 574-590 ``_m_init_state``,
1618-1864 ``_init_group``):

  V (AL8/AL16): ``<p>_q`` uint8/int16 [numel padded to block_size],
                ``<p>_scale`` fp32 ones, ``<p>_min_log`` fp32 zeros [nblocks],
                ``<p>_shape``, ``<p>_pad``; fp32 state is ``<p>`` with the tensor shape.
  M (UF8/D8):   ``m_q`` uint8 [numel padded to m_block_size] filled 128 / 127,
  M (UF4/D4):   ``m_q`` uint8 [padded/2] filled 0x88 / 0x77 (even element in
                the high nibble), ``m_scale`` fp32 ones, ``m_block_size``.
Tensors with fewer than ``min_8bit_size`` elements keep fp32 state.
"""
import logging
import math

import torch

from . import _native as nat

logger = logging.getLogger("adafactor8bit.optimizer")

_VALID_M = ("uf4", "uf8", "d4", "d8", "fp32")


def m_bits(mqt: str) -> int:
    return 4 if mqt in ("uf4", "d4") else 8


def m_mode(mqt: str) -> int:
    return 0 if mqt in ("uf4", "uf8") else 1


# ---------------------------------------------------------------- codebook
def dynamic_map(total_bits: int) -> torch.Tensor:
    """Signed dynamic codebook (Dettmers et al. 2022) as the reference builds it
    (optimizer.py:416-441): per exponent level i < E the midpoints of
    linspace(0.1, 1, 2^(i+N-E)+1) scaled by +/-10^(i-E+1), the extra +/-midpoints
    when N > E, then 0 and 1; sorted.  E = 7 (8-bit) or 3 (4-bit), N = bits-1."""
    e = 7 if total_bits == 8 else 3
    nb = total_bits - 1
    out = []
    for i in range(e):
        k = int(2 ** (i + nb - e) + 1)
        edges = torch.linspace(0.1, 1, k, dtype=torch.float32)
        mids = (edges[:-1] + edges[1:]) / 2.0
        s = 10 ** (-(e - 1) + i)
        out.extend((s * mids).tolist())
        out.extend((-s * mids).tolist())
    extra = 2 ** (nb - e) - 1
    if extra > 0:
        edges = torch.linspace(0.1, 1, extra + 1, dtype=torch.float32)
        mids = (edges[:-1] + edges[1:]) / 2.0
        out.extend(mids.tolist())
        out.extend((-mids).tolist())
    out.extend([0.0, 1.0])
    if len(out) != 2 ** total_bits:
        raise AssertionError(f"Expected {2 ** total_bits} items, got {len(out)}")
    out.sort()
    return torch.tensor(out, dtype=torch.float32)


_QMAP_DONE = set()


def ensure_qmap(device):
    """Upload the codebooks to the device once (optimizer.py:109-133)."""
    key = str(device)
    if key in _QMAP_DONE:
        return
    q8 = dynamic_map(8).contiguous()
    q4 = dynamic_map(4).contiguous()
    with torch.cuda.device(device):
        rc = nat.lib().a8_set_qmap(q8.data_ptr(), q4.data_ptr())
    nat.check(rc, "a8_set_qmap")
    _QMAP_DONE.add(key)


# ---------------------------------------------------------------- init helpers
def init_v_state(state, prefix, shape, block_size, device, vqt="al8"):
    numel = math.prod(shape) if not isinstance(shape, int) else shape
    if vqt == "fp32":
        state[prefix] = torch.zeros(shape, dtype=torch.float32, device=device)
        return
    pad = (block_size - numel % block_size) % block_size
    nb = (numel + pad) // block_size
    dt = torch.uint8 if vqt == "al8" else torch.int16
    state[f"{prefix}_q"] = torch.zeros(numel + pad, dtype=dt, device=device)
    state[f"{prefix}_scale"] = torch.ones(nb, dtype=torch.float32, device=device)
    state[f"{prefix}_min_log"] = torch.zeros(nb, dtype=torch.float32, device=device)
    state[f"{prefix}_shape"] = shape
    state[f"{prefix}_pad"] = pad


def init_v_or_fp32(state, prefix, shape, block_size, device, vqt, use_quant):
    if use_quant and vqt != "fp32":
        init_v_state(state, prefix, shape, block_size, device, vqt)
    else:
        state[prefix] = torch.zeros(shape, dtype=torch.float32, device=device)


def m_init_state(state, numel, m_block_size, mqt, device, shape=None, prefix="m"):
    if mqt == "fp32":
        if shape is None:
            raise AssertionError("_m_init_state: shape is required for fp32 momentum")
        state[prefix] = torch.zeros(shape, dtype=torch.float32, device=device)
    else:
        padded = ((numel + m_block_size - 1) // m_block_size) * m_block_size
        if m_bits(mqt) == 4:
            fill = 0x88 if mqt == "uf4" else 0x77
            state[f"{prefix}_q"] = torch.full((padded // 2,), fill, dtype=torch.uint8, device=device)
        else:
            fill = 128 if mqt == "uf8" else 127
            state[f"{prefix}_q"] = torch.full((padded,), fill, dtype=torch.uint8, device=device)
        state[f"{prefix}_scale"] = torch.ones(padded // m_block_size, dtype=torch.float32, device=device)
        state["m_block_size"] = m_block_size
    state["m_quant_type"] = mqt


def init_m_or_fp32(state, numel, m_block_size, mqt, device, shape, use_quant):
    if use_quant and mqt != "fp32":
        m_init_state(state, numel, m_block_size, mqt, device, shape=shape)
    else:
        state["m"] = torch.zeros(shape, dtype=torch.float32, device=device)
        state["m_quant_type"] = "fp32"


def reset_keep_step(state):
    step = state.get("step", 0)
    seed = state.get("sr_seed")
    state.clear()
    state["step"] = step
    if seed is not None:
        state["sr_seed"] = seed


# ---------------------------------------------------------------- _init_group
def init_group(opt, group, params_with_grad, grads, states):
    """Create fresh state and keep existing state consistent with the group's
    configuration (optimizer.py:1618-1864).  Configuration changes that need a
    re-encoding of existing state (quantize on/off, codec change of live state)
    reset that state with a warning, like the reference's block/type changes."""
    quantize = group.get("quantize", True)
    bs = group.get("block_size", 2048)
    mbs = group.get("m_block_size", 256)
    mqt = group.get("m_quant_type", "uf8")
    vqt = group.get("v_quant_type", "al8")
    cqt = group.get("c_quant_type") or vqt
    min8 = group.get("min_8bit_size", 4096)
    apollo_rank = group.get("apollo_rank", 0)
    apollo_factorize = group.get("apollo_factorize", False)
    factored = group.get("factored", True)
    beta1, beta2, beta2_decay, beta3 = (group.get("beta1"), group.get("beta2"),
                                        group.get("beta2_decay"), group.get("beta3"))
    sgd = beta2 is None and beta2_decay is None
    for p in group["params"]:
        if p.grad is None:
            continue
        use_quant = quantize and not (p.numel() < min8)
        params_with_grad.append(p)
        grads.append(p.grad)
        st = opt.state[p]
        use_apollo = apollo_rank > 0 and p.grad.dim() >= 2
        want_factored = p.grad.dim() >= 2 and factored
        needs_init = len(st) == 0
        if not needs_init:
            old_mqt = st.get("m_quant_type", "uf8")
            if old_mqt not in _VALID_M:
                st["m_quant_type"] = old_mqt = "uf8"
            old_mbs = st.get("m_block_size", mbs)
            if not isinstance(old_mbs, int):
                st["m_block_size"] = old_mbs = mbs
            if (old_mqt != mqt or old_mbs != mbs) and use_quant:
                logger.warning(f"Adafactor8Bit: M config changed (type: '{old_mqt}'->'{mqt}', block: "
                               f"{old_mbs}->{mbs}) for param shape {p.shape}. Momentum history will be "
                               f"reset to zero.")
                for k in ("m_q", "m_scale", "m_block_size", "m", "m_low_q", "m_low_scale", "m_low"):
                    st.pop(k, None)
                st["m_quant_type"] = mqt
            for k in ("m_q", "m_low_q"):
                if k in st and st[k].dtype != torch.uint8:
                    logger.warning(f"Adafactor8Bit: Momentum dtype mismatch (Current: {st[k].dtype}, "
                                   f"Target: torch.uint8) for {k}. Re-initializing.")
                    st.pop(k, None)
                    st.pop(k.replace("_q", "_scale"), None)
                    st.pop("m_block_size", None)
                    st.pop("m_quant_type", None)
            old_vqt = st.get("v_quant_type", "al8")
            old_cqt = st.get("c_quant_type", old_vqt)
            old_bs = st.get("block_size", bs)
            if (old_vqt != vqt or old_cqt != cqt or old_bs != bs) and use_quant:
                logger.warning(f"Adafactor8Bit: V/C/Block config changed (V: '{old_vqt}'->'{vqt}', C: "
                               f"'{old_cqt}'->'{cqt}', BS: {old_bs}->{bs}) for param shape {p.shape}. "
                               f"Re-initializing state.")
                reset_keep_step(st)
                needs_init = True
            is_apollo_state = "apollo_seed" in st
            if use_apollo != is_apollo_state and not needs_init:
                logger.warning(f"Adafactor8Bit: Apollo/Adafactor mode changed for param shape {p.shape}. "
                               f"Re-initializing state.")
                reset_keep_step(st)
                needs_init = True
            elif use_apollo and is_apollo_state and not needs_init:
                toggled = (st.get("beta3") is None) != (beta3 is None)
                if (st.get("apollo_rank") != apollo_rank
                        or st.get("apollo_factorize", False) != apollo_factorize or toggled):
                    logger.warning(f"Adafactor8Bit: Apollo/CAME config changed for param shape {p.shape}. "
                                   f"Re-initializing state.")
                    reset_keep_step(st)
                    needs_init = True
                else:
                    st["beta3"] = beta3
            elif not sgd and not needs_init:
                is_fact = "row_var" in st or "row_var_q" in st
                if is_fact != want_factored:
                    logger.warning(f"Adafactor8Bit: factored mode mismatch for param shape {p.shape}. "
                                   f"Re-initializing state.")
                    reset_keep_step(st)
                    needs_init = True
            if not needs_init and bool(st.get("is_quantized", False)) != bool(use_quant):
                logger.warning(f"Adafactor8Bit: quantize flag changed for param shape {p.shape}. "
                               f"Re-initializing state.")
                reset_keep_step(st)
                needs_init = True
        if needs_init:
            _fresh_state(opt, st, p, group, use_quant, use_apollo, want_factored, sgd, bs, mbs, mqt,
                         vqt, cqt, beta1, beta3, apollo_rank, apollo_factorize)
        else:
            _keep_state(st, p, use_quant, use_apollo, want_factored, bs, mbs, mqt, cqt, beta1, beta3)
        states.append(st)


def _fresh_state(opt, st, p, group, use_quant, use_apollo, want_factored, sgd, bs, mbs, mqt, vqt, cqt,
                 beta1, beta3, apollo_rank, apollo_factorize):
    if "step" not in st:
        st["step"] = 0
    st["is_quantized"] = use_quant
    st["block_size"] = bs
    st["v_quant_type"] = vqt
    st["c_quant_type"] = cqt
    dev = p.device
    if sgd:
        if beta1 is not None:
            if use_quant and mqt != "fp32":
                m_init_state(st, p.numel(), mbs, mqt, dev)
            else:
                st["m"] = torch.zeros_like(p.grad, dtype=torch.float32, device=dev,
                                           memory_format=torch.preserve_format)
                st["m_quant_type"] = "fp32"
    elif use_apollo:
        seed = opt._apollo_seed_counter
        opt._apollo_seed_counter += 1
        gap = group.get("apollo_update_proj_gap", 200)
        st["apollo_seed"] = seed
        st["apollo_rank"] = apollo_rank
        st["apollo_factorize"] = apollo_factorize
        st["beta3"] = beta3
        st["apollo_update_proj_gap"] = gap
        st["last_proj_step"] = -gap
        st["apollo_proj_matrix_T"] = None
        st["m_quant_type"] = mqt
        for k in ("v_low_q", "v_low_scale", "v_low_min_log", "v_low_shape", "v_low_pad", "v_low"):
            st[k] = None
        if beta3 is not None:
            names = (("conf_row_low", "conf_col_low") if apollo_factorize else ("res_low",))
            for nm in names:
                for suf in ("_q", "_scale", "_min_log", "_shape", "_pad", ""):
                    st[nm + suf] = None
    elif want_factored:
        shape = p.grad.shape
        R, C = shape[-2], shape[-1]
        rs = list(shape[:-2]) + [R, 1]
        cs = list(shape[:-2]) + [1, C]
        init_v_or_fp32(st, "row_var", rs, bs, dev, vqt, use_quant)
        init_v_or_fp32(st, "col_var", cs, bs, dev, vqt, use_quant)
        if beta1 is not None:
            init_m_or_fp32(st, p.numel(), mbs, mqt, dev, p.shape, use_quant)
        if beta3 is not None:
            init_v_or_fp32(st, "conf_row", rs, bs, dev, cqt, use_quant)
            init_v_or_fp32(st, "conf_col", cs, bs, dev, cqt, use_quant)
    else:
        init_v_or_fp32(st, "variance", p.grad.shape, bs, dev, vqt, use_quant)
        if beta1 is not None:
            init_m_or_fp32(st, p.numel(), mbs, mqt, dev, p.shape, use_quant)


def _keep_state(st, p, use_quant, use_apollo, want_factored, bs, mbs, mqt, cqt, beta1, beta3):
    """optimizer.py:1744-1862: device/dtype fix-ups and CAME/momentum (re)creation."""
    for k in list(st.keys()):
        v = st[k]
        if isinstance(v, torch.Tensor):
            if v.device != p.device:
                st[k] = v = v.to(p.device)
            if k.endswith("_q"):
                if "m_q" in k or "m_low_q" in k:
                    if v.dtype != torch.uint8:
                        st[k] = v.to(torch.uint8)
                else:
                    conf = k.startswith("conf") or k.startswith("res_low")
                    qt = st.get("c_quant_type" if conf else "v_quant_type", "al8")
                    want = torch.int16 if qt == "al16" else torch.uint8
                    if v.dtype != want:
                        st[k] = v.to(want)
            if (k.endswith("_scale") or k.endswith("_min_log")) and st[k].dtype != torch.float32:
                st[k] = st[k].to(torch.float32)
    cbs = st.get("block_size", bs)
    if not use_apollo:
        if beta3 is None:
            for pre in ("conf_row", "conf_col"):
                st.pop(pre, None)
                for suf in ("q", "scale", "min_log", "shape", "pad"):
                    st.pop(f"{pre}_{suf}", None)
        elif want_factored:
            shape = p.grad.shape
            R, C = shape[-2], shape[-1]
            rs = list(shape[:-2]) + [R, 1]
            cs = list(shape[:-2]) + [1, C]
            if "conf_row" not in st and "conf_row_q" not in st:
                init_v_or_fp32(st, "conf_row", rs, cbs, p.device, cqt, use_quant)
            if "conf_col" not in st and "conf_col_q" not in st:
                init_v_or_fp32(st, "conf_col", cs, cbs, p.device, cqt, use_quant)
    if beta1 is not None and "m_q" not in st and not use_apollo:
        mb = st.get("m_block_size", mbs)
        if use_quant and mqt != "fp32":
            if "m" in st:
                raise NotImplementedError("re-encoding fp32 momentum into 8-bit codes is not available "
                                          "in this build yet")
            m_init_state(st, p.numel(), mb, mqt, p.device, shape=p.shape)
            st["m_block_size"] = mb
        elif "m" not in st and mqt == "fp32":
            st["m"] = torch.zeros(p.shape, dtype=torch.float32, device=p.device)
            st["m_quant_type"] = "fp32"
    if "is_quantized" not in st:
        st["is_quantized"] = use_quant if use_apollo else ("variance_q" in st or "row_var_q" in st
                                                           or "m_q" in st)
    if "block_size" not in st:
        st["block_size"] = bs
    if beta1 is None:
        for k in ("m_q", "m_scale", "m_block_size", "m_quant_type", "m"):
            st.pop(k, None)


def state_bytes(state) -> int:
    """Bytes held by tensor entries of one parameter's state."""
    return sum(v.numel() * v.element_size() for v in state.values() if torch.is_tensor(v))
