"""Optimizer state: layout, creation, and reconciliation with a group's configuration.

Stored format.  The keys, dtypes, shapes and padding are the reference's
checkpoint format (adafactor8bit/optimizer.py:389-401 ``_init_v_state``,
574-590 ``_m_init_state``, 1618-1864 ``_init_group``), so ``state_dict()`` files
move between the two implementations:

  second-moment-like slot ``<s>`` as AL codes: ``<s>_q`` uint8 (AL8) or int16
      (AL16) [numel padded to block_size], ``<s>_scale`` fp32 ones and
      ``<s>_min_log`` fp32 zeros [nblocks], ``<s>_shape``, ``<s>_pad``;
      as fp32 state: ``<s>`` with the tensor's shape;
  momentum slot ``m`` / ``m_low`` as codes: ``<m>_q`` uint8 [numel padded to
      m_block_size] filled 128 (UF8) / 127 (D8), or [padded / 2] filled 0x88
      (UF4) / 0x77 (D4) with the even element in the high nibble, ``<m>_scale``
      fp32 ones, plus the ``m_block_size`` and ``m_quant_type`` tags;
      as fp32 state: ``<m>``.
Tensors with fewer than ``min_8bit_size`` elements keep fp32 state.

Design.  A parameter's state is a set of slots (``SLOTS``), each either coded or
fp32.  ``Config`` is what a parameter's group asks for: the route the parameter
takes (SGD, APOLLO, factored, full-rank) and the codec of each slot family.
``init_group`` brings stored state in line with its ``Config`` in one pass of
small rules (``_tidy_momentum``, ``_reset_reason``, ``_place``, ``_to_codes`` /
``_to_fp32``, ``_sync_confidence``, ``_sync_momentum``, ``_backfill``).  The
outcome of each rule is the reference's: the same configuration changes reset
the state (keeping ``step`` and ``sr_seed``), reset only the momentum, or
re-encode existing state between codes and fp32 (``_migrate_quantize_flag``,
optimizer.py:976-1045, and fp32 momentum meeting a codec, 1838-1846).
Re-encoding runs on the GPU through the library's codec entry points.
"""
import dataclasses
import logging
import math
from typing import Any, Dict, Optional

import torch

from . import _native as nat

logger = logging.getLogger("adafactor8bit.optimizer")

_VALID_M = ("uf4", "uf8", "d4", "d8", "fp32")
_AL_FLOOR = -126.0          # default min_log floor of the reference's _quant_v (optimizer.py:299)
_AL_SUFFIXES = ("_q", "_scale", "_min_log", "_shape", "_pad")


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


# ---------------------------------------------------------------- slots
@dataclasses.dataclass(frozen=True)
class Slot:
    name: str
    family: str      # "v" (v_quant_type), "c" (c_quant_type) or "m" (m_quant_type, momentum)
    lowrank: bool    # an APOLLO low-rank slot, created by the step itself


SLOTS: Dict[str, Slot] = {s.name: s for s in (
    Slot("variance", "v", False), Slot("row_var", "v", False), Slot("col_var", "v", False),
    Slot("v_low", "v", True),
    Slot("conf_row", "c", False), Slot("conf_col", "c", False),
    Slot("res_low", "c", True), Slot("conf_row_low", "c", True), Slot("conf_col_low", "c", True),
    Slot("m", "m", False), Slot("m_low", "m", True),
)}
_AL_SLOTS = tuple(n for n, s in SLOTS.items() if s.family != "m")


def _code_dtype(st, key):
    """dtype a stored tensor must have: momentum codes uint8, AL codes uint8 / int16
    by their family's tag, block metadata fp32; anything else keeps its own."""
    if key.endswith("_q"):
        if "m_q" in key or "m_low_q" in key:
            return torch.uint8
        conf = key.startswith("conf") or key.startswith("res_low")
        qt = st.get("c_quant_type" if conf else "v_quant_type", "al8")
        return torch.int16 if qt == "al16" else torch.uint8
    if key.endswith("_scale") or key.endswith("_min_log"):
        return torch.float32
    return None


@dataclasses.dataclass(frozen=True)
class Config:
    """What a parameter's group asks of its state (optimizer.py:1620-1650)."""
    route: str          # "sgd", "apollo", "factored" or "full"
    quant: bool         # coded state (quantize and numel >= min_8bit_size)
    bs: int
    mbs: int
    vqt: str
    cqt: str
    mqt: str
    beta1: Optional[float]
    beta3: Optional[float]
    rank: int
    factorize: bool
    gap: int

    @classmethod
    def of(cls, group, p) -> "Config":
        sgd = group.get("beta2") is None and group.get("beta2_decay") is None
        rank = group.get("apollo_rank", 0)
        dim = p.grad.dim() if p.grad is not None else p.dim()
        if sgd:
            route = "sgd"
        elif rank > 0 and dim >= 2:
            route = "apollo"
        elif dim >= 2 and group.get("factored", True):
            route = "factored"
        else:
            route = "full"
        vqt = group.get("v_quant_type", "al8")
        return cls(route=route,
                   quant=bool(group.get("quantize", True)) and p.numel() >= group.get("min_8bit_size", 4096),
                   bs=group.get("block_size", 2048), mbs=group.get("m_block_size", 256), vqt=vqt,
                   cqt=group.get("c_quant_type") or vqt, mqt=group.get("m_quant_type", "uf8"),
                   beta1=group.get("beta1"), beta3=group.get("beta3"), rank=rank,
                   factorize=bool(group.get("apollo_factorize", False)),
                   gap=group.get("apollo_update_proj_gap", 200))

    def codec(self, family: str) -> str:
        qt = {"v": self.vqt, "c": self.cqt, "m": self.mqt}[family]
        return qt if self.quant else "fp32"


def _rowcol_shapes(shape):
    lead = list(shape[:-2])
    return lead + [shape[-2], 1], lead + [1, shape[-1]]


# ---------------------------------------------------------------- slot storage
def new_al_slot(st, name, shape, block_size, codec, device):
    """A fresh second-moment-like slot: fp32 zeros, or zero codes with unit scales."""
    if codec == "fp32":
        st[name] = torch.zeros(shape, dtype=torch.float32, device=device)
        return
    numel = math.prod(shape) if not isinstance(shape, int) else shape
    pad = (block_size - numel % block_size) % block_size
    nb = (numel + pad) // block_size
    st[name + "_q"] = torch.zeros(numel + pad, dtype=torch.int16 if codec == "al16" else torch.uint8, device=device)
    st[name + "_scale"] = torch.ones(nb, dtype=torch.float32, device=device)
    st[name + "_min_log"] = torch.zeros(nb, dtype=torch.float32, device=device)
    st[name + "_shape"] = shape
    st[name + "_pad"] = pad


def new_momentum_codes(st, prefix, numel, block_size, mqt, device):
    """Fresh momentum codes: every code decodes to 0, scales are 1."""
    padded = -(-numel // block_size) * block_size
    if m_bits(mqt) == 4:
        q = torch.full((padded // 2,), 0x88 if mqt == "uf4" else 0x77, dtype=torch.uint8, device=device)
    else:
        q = torch.full((padded,), 128 if mqt == "uf8" else 127, dtype=torch.uint8, device=device)
    st[prefix + "_q"] = q
    st[prefix + "_scale"] = torch.ones(padded // block_size, dtype=torch.float32, device=device)
    st["m_block_size"] = block_size
    st["m_quant_type"] = mqt


def _drop(st, *keys):
    for k in keys:
        st.pop(k, None)


def _drop_al_slot(st, name):
    _drop(st, name, *(name + s for s in _AL_SUFFIXES))


def _stream(t):
    return nat.stream_of(t.device)


def encode_al(st, name, x, block_size, codec):
    """fp32 values -> AL codes of slot ``name`` (the reference's _quant_v,
    optimizer.py:379-383): codes in the block view [nblocks, block_size], the
    value's shape and the padding."""
    x = x.detach().to(torch.float32).contiguous()
    n = x.numel()
    pad = (block_size - n % block_size) % block_size
    nb = (n + pad) // block_size
    q = torch.empty((nb, block_size), dtype=torch.int16 if codec == "al16" else torch.uint8, device=x.device)
    scale = torch.empty(nb, dtype=torch.float32, device=x.device)
    min_log = torch.empty(nb, dtype=torch.float32, device=x.device)
    nat.check(nat.lib().a8_al_encode(q.data_ptr(), scale.data_ptr(), min_log.data_ptr(), x.data_ptr(), n,
                                     int(block_size), 16 if codec == "al16" else 8, _AL_FLOOR, _stream(x)),
              "a8_al_encode")
    st[name + "_q"], st[name + "_scale"], st[name + "_min_log"] = q, scale, min_log
    st[name + "_shape"], st[name + "_pad"] = x.shape, pad


def decode_al(st, name):
    """Slot ``name``'s codes -> fp32 in its stored shape, removing the coded keys
    (the reference's _deq_v(pop=True), optimizer.py:358-371)."""
    q = st.pop(name + "_q")
    scale, min_log = st.pop(name + "_scale"), st.pop(name + "_min_log")
    shape, pad = st.pop(name + "_shape"), st.pop(name + "_pad")
    q = q.contiguous()
    n = q.numel() - int(pad)
    out = torch.empty(q.numel(), dtype=torch.float32, device=q.device)
    nat.check(nat.lib().a8_dequantize_log_nonneg(out.data_ptr(), q.data_ptr(), scale.contiguous().data_ptr(),
                                                 min_log.contiguous().data_ptr(), n,
                                                 q.numel() // scale.numel(), 16 if q.dtype == torch.int16 else 8,
                                                 _stream(q)), "a8_dequantize_log_nonneg")
    return out[:n].view(tuple(shape))


def encode_momentum(x, mqt, block_size):
    """fp32 momentum -> (codes, scales) (the reference's _m_quantize,
    optimizer.py:525-531): a lerp of weight 1 from fresh codes re-encodes x itself."""
    x = x.detach().to(torch.float32).contiguous()
    tmp: Dict[str, Any] = {}
    new_momentum_codes(tmp, "m", x.numel(), block_size, mqt, x.device)
    nat.check(nat.lib().a8_m_quantize_lerp(tmp["m_q"].data_ptr(), tmp["m_scale"].data_ptr(), x.data_ptr(), nat.F32,
                                           None, 0.0, int(block_size), x.numel(), m_bits(mqt), m_mode(mqt),
                                           _stream(x)), "a8_m_quantize_lerp")
    return tmp["m_q"], tmp["m_scale"]


def decode_momentum(q, scale, shape, block_size, mqt):
    """Momentum codes -> fp32 of ``shape`` (the reference's _m_dequantize,
    optimizer.py:535-541)."""
    n = math.prod(shape)
    out = torch.empty(max(n, 1), dtype=torch.float32, device=q.device)
    nat.check(nat.lib().a8_dequantize_momentum(out.data_ptr(), q.contiguous().data_ptr(),
                                               scale.contiguous().data_ptr(), n, int(block_size), m_bits(mqt),
                                               m_mode(mqt), _stream(q)), "a8_dequantize_momentum")
    return out[:n].view(tuple(shape))


# ---------------------------------------------------------------- fresh state
def _fresh(opt, st, p, cfg: Config):
    """optimizer.py:1712-1788: the state a parameter starts with on its route."""
    st.setdefault("step", 0)
    st["is_quantized"] = cfg.quant
    st["block_size"] = cfg.bs
    st["v_quant_type"] = cfg.vqt
    st["c_quant_type"] = cfg.cqt
    dev = p.device
    if cfg.route == "apollo":
        st["apollo_seed"] = opt._apollo_seed_counter
        opt._apollo_seed_counter += 1
        st["apollo_rank"] = cfg.rank
        st["apollo_factorize"] = cfg.factorize
        st["beta3"] = cfg.beta3
        st["apollo_update_proj_gap"] = cfg.gap
        st["last_proj_step"] = -cfg.gap
        st["apollo_proj_matrix_T"] = None
        st["m_quant_type"] = cfg.mqt
        # low-rank slots are created by the first step (their shape depends on the side)
        lazy = ["v_low"]
        if cfg.beta3 is not None:
            lazy += ["conf_row_low", "conf_col_low"] if cfg.factorize else ["res_low"]
        for name in lazy:
            for key in (name + s for s in _AL_SUFFIXES):
                st[key] = None
        for name in lazy[1:]:
            st[name] = None
        st["v_low"] = None
        return
    if cfg.route == "factored":
        rs, cs = _rowcol_shapes(p.grad.shape)
        new_al_slot(st, "row_var", rs, cfg.bs, cfg.codec("v"), dev)
        new_al_slot(st, "col_var", cs, cfg.bs, cfg.codec("v"), dev)
        if cfg.beta3 is not None:
            new_al_slot(st, "conf_row", rs, cfg.bs, cfg.codec("c"), dev)
            new_al_slot(st, "conf_col", cs, cfg.bs, cfg.codec("c"), dev)
    elif cfg.route == "full":
        new_al_slot(st, "variance", p.grad.shape, cfg.bs, cfg.codec("v"), dev)
    if cfg.beta1 is None:
        return
    if cfg.codec("m") != "fp32":
        new_momentum_codes(st, "m", p.numel(), cfg.mbs, cfg.mqt, dev)
    else:
        st["m"] = torch.zeros(p.shape, dtype=torch.float32, device=dev)
        st["m_quant_type"] = "fp32"


def _clear_keep_step(st):
    """optimizer.py:385-391: start over, keeping the step counter and SR seed."""
    keep = {k: st[k] for k in ("step", "sr_seed") if st.get(k) is not None}
    keep.setdefault("step", 0)
    st.clear()
    st.update(keep)


# ---------------------------------------------------------------- reconcile rules
def _tidy_momentum(st, p, cfg: Config):
    """Momentum tags and codes (optimizer.py:1667-1686): an unknown codec tag reads
    as UF8 and a non-integer block tag as the group's; a codec or block change of
    coded state resets the momentum; codes of any dtype other than uint8 are dropped."""
    if st.get("m_quant_type", "uf8") not in _VALID_M:
        st["m_quant_type"] = "uf8"
    if not isinstance(st.get("m_block_size", cfg.mbs), int):
        st["m_block_size"] = cfg.mbs
    old = (st.get("m_quant_type", "uf8"), st.get("m_block_size", cfg.mbs))
    if cfg.quant and old != (cfg.mqt, cfg.mbs):
        logger.warning(f"Adafactor8Bit: M config changed (type: '{old[0]}'->'{cfg.mqt}', block: {old[1]}->"
                       f"{cfg.mbs}) for param shape {p.shape}. Momentum history will be reset to zero.")
        _drop(st, "m_q", "m_scale", "m_block_size", "m", "m_low_q", "m_low_scale", "m_low")
        st["m_quant_type"] = cfg.mqt
    for key in ("m_q", "m_low_q"):
        v = st.get(key)
        if torch.is_tensor(v) and v.dtype != torch.uint8:
            logger.warning(f"Adafactor8Bit: Momentum dtype mismatch (Current: {v.dtype}, Target: torch.uint8) "
                           f"for {key}. Re-initializing.")
            _drop(st, key, key[:-2] + "_scale", "m_block_size", "m_quant_type")


def _reset_reason(st, p, cfg: Config) -> Optional[str]:
    """Configuration changes that restart the whole state (optimizer.py:1687-1710)."""
    old_v = st.get("v_quant_type", "al8")
    old = (old_v, st.get("c_quant_type", old_v), st.get("block_size", cfg.bs))
    if cfg.quant and old != (cfg.vqt, cfg.cqt, cfg.bs):
        return (f"V/C/Block config changed (V: '{old[0]}'->'{cfg.vqt}', C: '{old[1]}'->'{cfg.cqt}', BS: "
                f"{old[2]}->{cfg.bs}) for param shape {p.shape}. Re-initializing state.")
    was_apollo = "apollo_seed" in st
    if was_apollo != (cfg.route == "apollo"):
        return f"Apollo/Adafactor mode changed for param shape {p.shape}. Re-initializing state."
    if was_apollo:
        same = (st.get("apollo_rank") == cfg.rank and st.get("apollo_factorize", False) == cfg.factorize
                and (st.get("beta3") is None) == (cfg.beta3 is None))
        return None if same else f"Apollo/CAME config changed for param shape {p.shape}. Re-initializing state."
    if cfg.route != "sgd" and ("row_var" in st or "row_var_q" in st) != (cfg.route == "factored"):
        return f"factored mode mismatch for param shape {p.shape}. Re-initializing state."
    return None


def _place(st, device):
    """Every stored tensor on the parameter's device, codes and metadata in their
    format's dtype (optimizer.py:1791-1806)."""
    for k, v in list(st.items()):
        if not torch.is_tensor(v):
            continue
        want = _code_dtype(st, k) or v.dtype
        if v.device != device or v.dtype != want:
            st[k] = v.to(device=device, dtype=want)


def _is_plain(st, name):
    """The slot holds fp32 state that has no codes yet.  The low-rank V and residual
    slots exist with None codes until encoded; the other slots count their codes
    present when the key is (optimizer.py:979-1006)."""
    if not torch.is_tensor(st.get(name)):
        return False
    if name in ("v_low", "res_low"):
        return st.get(name + "_q") is None
    return name + "_q" not in st


def _to_codes(st, p, cfg: Config, bs, mbs):
    """quantize switched on for existing fp32 state (optimizer.py:978-1020)."""
    for name in _AL_SLOTS:
        fam = SLOTS[name].family
        qt = cfg.vqt if fam == "v" else cfg.cqt
        if qt == "fp32" or (fam == "c" and cfg.beta3 is None) or not _is_plain(st, name):
            continue
        encode_al(st, name, st[name], bs, qt)
        if name == "v_low":
            st[name] = None
        else:
            del st[name]
    if torch.is_tensor(st.get("m_low")) and st.get("m_low_q") is None and cfg.mqt != "fp32":
        b = st.get("m_block_size", mbs)
        st["m_low_q"], st["m_low_scale"] = encode_momentum(st.pop("m_low"), cfg.mqt, b)
        st["m_block_size"], st["m_quant_type"] = b, cfg.mqt
    if cfg.beta1 is not None and cfg.mqt != "fp32" and "m_q" not in st and "apollo_seed" not in st:
        _momentum_to_codes(st, p, cfg, st.get("m_block_size", mbs))
    st["is_quantized"] = True


def _to_fp32(st, p, cfg: Config, bs, mbs):
    """quantize switched off for existing coded state (optimizer.py:1022-1045)."""
    for name in _AL_SLOTS:
        if torch.is_tensor(st.get(name + "_q")):
            st[name] = decode_al(st, name)
    if "m_low_q" in st:
        logger.warning("Adafactor8Bit: Apollo m_low_q discarded due to quantize flag change. Momentum state will "
                       "be reset.")
        _drop(st, "m_low_q", "m_low_scale", "m_block_size")
    if torch.is_tensor(st.get("m_q")):
        st["m"] = decode_momentum(st.pop("m_q"), st.pop("m_scale"), p.shape, st.get("m_block_size", mbs),
                                  st.get("m_quant_type", "uf8"))
        _drop(st, "m_block_size", "m_quant_type")
    st["is_quantized"] = False


def _momentum_to_codes(st, p, cfg: Config, block):
    """Coded momentum for a parameter that has none: fp32 momentum is re-encoded
    (optimizer.py:1840-1844), otherwise fresh codes."""
    if torch.is_tensor(st.get("m")):
        st["m_q"], st["m_scale"] = encode_momentum(st.pop("m"), cfg.mqt, block)
        st["m_quant_type"] = cfg.mqt
    else:
        new_momentum_codes(st, "m", p.numel(), block, cfg.mqt, p.device)
    st["m_block_size"] = block


def _sync_confidence(st, p, cfg: Config):
    """CAME confidence of a full-rank route (optimizer.py:1814-1832): dropped when
    beta3 is off, created when a factored parameter lacks it."""
    if cfg.route == "apollo":
        return
    if cfg.beta3 is None:
        _drop_al_slot(st, "conf_row")
        _drop_al_slot(st, "conf_col")
    elif cfg.route == "factored":
        rs, cs = _rowcol_shapes(p.grad.shape)
        for name, shape in (("conf_row", rs), ("conf_col", cs)):
            if name not in st and name + "_q" not in st:
                new_al_slot(st, name, shape, st.get("block_size", cfg.bs), cfg.codec("c"), p.device)


def _sync_momentum(st, p, cfg: Config):
    """Momentum of a non-APOLLO parameter that has no codes (optimizer.py:1834-1849)."""
    if cfg.beta1 is None or cfg.route == "apollo" or "m_q" in st:
        return
    block = st.get("m_block_size", cfg.mbs)
    if cfg.quant and cfg.mqt != "fp32":
        _momentum_to_codes(st, p, cfg, block)
    elif "m" not in st and cfg.mqt == "fp32":
        st["m"] = torch.zeros(p.shape, dtype=torch.float32, device=p.device)
        st["m_quant_type"] = "fp32"


def _backfill(st, cfg: Config):
    """Tags an older state may lack, and no momentum keys without beta1
    (optimizer.py:1851-1862)."""
    if "is_quantized" not in st:
        st["is_quantized"] = cfg.quant if cfg.route == "apollo" else \
            any(k in st for k in ("variance_q", "row_var_q", "m_q"))
    st.setdefault("block_size", cfg.bs)
    if cfg.beta1 is None:
        _drop(st, "m_q", "m_scale", "m_block_size", "m_quant_type", "m")


def reconcile(opt, st, p, cfg: Config):
    """Bring one parameter's state in line with ``cfg``."""
    if not st:
        _fresh(opt, st, p, cfg)
        return
    _tidy_momentum(st, p, cfg)
    why = _reset_reason(st, p, cfg)
    if why is not None:
        logger.warning("Adafactor8Bit: " + why)
        _clear_keep_step(st)
        _fresh(opt, st, p, cfg)
        return
    if cfg.route == "apollo":
        st["beta3"] = cfg.beta3
    _place(st, p.device)
    bs = st.get("block_size", cfg.bs)
    mbs = st.get("m_block_size", cfg.mbs)
    if cfg.quant and not st.get("is_quantized", False):
        _to_codes(st, p, cfg, bs, mbs)
    elif not cfg.quant and st.get("is_quantized", False):
        _to_fp32(st, p, cfg, bs, mbs)
    _sync_confidence(st, p, cfg)
    _sync_momentum(st, p, cfg)
    _backfill(st, cfg)


def init_group(opt, group, params_with_grad, grads, states):
    """Collect the group's parameters with gradients and reconcile their state
    (optimizer.py:1618-1864)."""
    for p in group["params"]:
        if p.grad is None:
            continue
        params_with_grad.append(p)
        grads.append(p.grad)
        st = opt.state[p]
        reconcile(opt, st, p, Config.of(group, p))
        states.append(st)


# ---------------------------------------------------------------- checkpoints
_FULL_RANK_MOMENTUM = ("m", "m_q", "m_scale")


class Checkpoint:
    """A ``state_dict`` prepared for ``Optimizer.load_state_dict`` (the reference's
    load path, optimizer.py:1467-1553).

    The base loader casts every floating-point state tensor to its parameter's
    dtype; this state is stored in fp32 or integer codes whatever the parameter's
    dtype.  So the tensors are held back from the base loader (``skeleton`` keeps
    everything else) and attached afterwards in their stored dtype on the
    parameter's device.  APOLLO states drop the obsolete full-rank momentum; the
    codec tags and the seed counters come from the checkpoint (tags default to
    AL8 / UF8, counters to 0); a group saved without ``stochastic_round_writeback``
    keeps the current group's setting."""

    def __init__(self, state_dict, current_groups):
        self.tensors: Dict[Any, Dict[str, torch.Tensor]] = {}
        self.tags: Dict[Any, Dict[str, str]] = {}
        kept_state = {}
        for idx, st in state_dict.get("state", {}).items():
            if not isinstance(st, dict):
                kept_state[idx] = st
                continue
            apollo = "apollo_seed" in st
            entries = {k: v for k, v in st.items() if not (apollo and k in _FULL_RANK_MOMENTUM)}
            self.tensors[idx] = {k: v for k, v in entries.items() if torch.is_tensor(v) and k != "step"}
            kept_state[idx] = {k: v for k, v in entries.items() if k not in self.tensors[idx]}
            v_tag = st.get("v_quant_type", "al8")
            self.tags[idx] = {"v_quant_type": v_tag, "m_quant_type": st.get("m_quant_type", "uf8"),
                              "c_quant_type": st.get("c_quant_type", v_tag)}
        self.skeleton = dict(state_dict)
        self.skeleton["state"] = kept_state
        saved_groups = state_dict.get("param_groups", [])
        self.saved_ids = [i for g in saved_groups for i in g.get("params", [])]
        self.sr_backfill = None
        if len(saved_groups) == len(current_groups):
            self.sr_backfill = [None if (isinstance(sg, dict) and "stochastic_round_writeback" in sg)
                                else g.get("stochastic_round_writeback", False)
                                for sg, g in zip(saved_groups, current_groups)]
        self.counters = (state_dict.get("_apollo_seed_counter", 0), state_dict.get("_sr_seed_counter", 0))

    def restore(self, opt):
        """After the base loader ran: counters, SR policy, tensors, tags."""
        opt._apollo_seed_counter, opt._sr_seed_counter = self.counters
        if self.sr_backfill is not None:
            for g, policy in zip(opt.param_groups, self.sr_backfill):
                if policy is not None:
                    g["stochastic_round_writeback"] = policy
        params = [p for g in opt.param_groups for p in g["params"]]
        if len(params) == len(self.saved_ids):
            for sid, p in zip(self.saved_ids, params):
                if p in opt.state:
                    for k, v in self.tensors.get(sid, {}).items():
                        opt.state[p][k] = v.detach().to(device=p.device, dtype=v.dtype, copy=True).contiguous()
        for pos, p in enumerate(params):
            if p not in opt.state:
                continue
            st = opt.state[p]
            st.update(self.tags.get(pos, {"v_quant_type": "al8", "m_quant_type": "uf8", "c_quant_type": "al8"}))
            if torch.is_tensor(st.get("step")):
                st["step"] = int(st["step"])


def compact(opt):
    """optimizer.py:1555-1590: after a checkpoint load, move every GPU state tensor
    through host memory and back in one contiguous allocation per tensor, releasing
    the cached blocks in between, so the loaded state does not inherit the
    fragmentation of the load; codes and metadata come back in their format's dtype."""
    moved = []
    for p, st in opt.state.items():
        for k, v in list(st.items()):
            if torch.is_tensor(v) and v.is_cuda:
                moved.append((p, st, k, v.cpu()))
                st[k] = None
    if not moved:
        return
    torch.cuda.empty_cache()
    for p, st, k, host in moved:
        st[k] = host.to(device=p.device, dtype=_code_dtype(st, k) or host.dtype).contiguous()


def state_bytes(state) -> int:
    """Bytes held by tensor entries of one parameter's state."""
    return sum(v.numel() * v.element_size() for v in state.values() if torch.is_tensor(v))
