"""CPU restatement of the reference's stochastic-rounding stream (TEST
INFRASTRUCTURE ONLY: imported by tests/ as the checker, never by the product).

The reference's CUDA kernels round a bf16 / fp16 parameter write stochastically
with a counter-based generator (kernels.cu:48-87):

  counter = seed * 0x9E3779B97F4A7C15 + step * 0xD1B54A32D192ED03 + idx   (mod 2^64)
  bits    = top 32 bits of SplitMix64(counter)      (one increment by the golden gamma)
  u       = (bits >> 8) * 2^-24                     (uniform in [0, 1), 24 bits)
  bf16    = truncate(x) + 1 ulp  if u < (low 16 bits of x) / 65536
            (no round-up from or to infinity; NaN becomes the canonical quiet NaN)
  fp16    = the fp16 neighbours lo < x < hi around round-to-nearest(x); hi if
            u < (x - lo) / (hi - lo) in fp32 (kernels.cu:100-131; |x| > 65504
            saturates to +-65504, Inf / NaN keep their class, exact values stay)

``seed`` is the parameter's ``sr_seed`` (a per-parameter counter from 1,
optimizer.py:1886-1892), ``step`` the optimizer step and ``idx`` the element's
index in the flattened parameter.  Pinned by the SplitMix64 published first
output (state 0 -> 0xE220A8397B1DCDAF) and by each rounding's defining
properties in tests/test_oracle_sr.py.
"""
import numpy as np

_GOLD = np.uint64(0x9E3779B97F4A7C15)
_STEPK = np.uint64(0xD1B54A32D192ED03)


def splitmix64(state):
    """SplitMix64 output for a state (array of uint64): z = state + gamma, then
    the two xor-shift-multiply rounds and the final xor-shift (kernels.cu:48-54)."""
    with np.errstate(over="ignore"):
        z = np.asarray(state, dtype=np.uint64) + _GOLD
        z = (z ^ (z >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
        z = (z ^ (z >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
        return z ^ (z >> np.uint64(31))


def sr_bits(seed: int, step: int, idx) -> np.ndarray:
    """kernels.cu:56-61: the 32 random bits of element ``idx``."""
    with np.errstate(over="ignore"):
        c = (np.uint64(seed) * _GOLD + np.uint64(step) * _STEPK) + np.asarray(idx, dtype=np.uint64)
    return (splitmix64(c) >> np.uint64(32)).astype(np.uint32)


def sr_uniform(seed: int, step: int, idx) -> np.ndarray:
    """kernels.cu:63-65: u = (bits >> 8) / 2^24 in float32."""
    return (sr_bits(seed, step, idx) >> np.uint32(8)).astype(np.float32) * np.float32(1.0 / 16777216.0)


def sr_fp32_to_bf16_bits(x: np.ndarray, u: np.ndarray) -> np.ndarray:
    """kernels.cu:67-87: the bf16 bit pattern of x rounded stochastically with u."""
    b = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    is_nan = ((b & 0x7F800000) == 0x7F800000) & ((b & 0x007FFFFF) != 0)
    lo = b & np.uint32(0xFFFF0000)
    rem = b & np.uint32(0x0000FFFF)
    hi = lo + np.uint32(0x00010000)
    lo_inf = (lo & 0x7F800000) == 0x7F800000
    hi_inf = ((hi & 0x7F800000) == 0x7F800000) & ((hi & 0x007FFFFF) == 0)
    can_up = (rem != 0) & ~is_nan & ~lo_inf & ~hi_inf
    prob = np.where(can_up, rem.astype(np.float32) * np.float32(1.0 / 65536.0), np.float32(0.0))
    out = np.where(can_up & (np.asarray(u, dtype=np.float32) < prob), hi, lo)
    out = np.where(is_nan, (b & np.uint32(0x80000000)) | np.uint32(0x7FC00000), out)
    return (out >> np.uint32(16)).astype(np.uint16)


def sr_round_bf16(x: np.ndarray, seed: int, step: int, idx=None) -> np.ndarray:
    """bf16 bits of x (flat, float32) rounded with the stream of (seed, step)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if idx is None:
        idx = np.arange(x.size, dtype=np.uint64)
    return sr_fp32_to_bf16_bits(x, sr_uniform(seed, step, idx))


def _fp16_next_up(h):
    """kernels.cu:88-92 on fp16 bit patterns (uint16 arrays)."""
    h = np.asarray(h, dtype=np.uint16)
    up = np.where(h & np.uint16(0x8000), h - np.uint16(1), h + np.uint16(1)).astype(np.uint16)
    up = np.where(h == 0x8000, np.uint16(0x0001), up)
    return np.where(h == 0x7C00, h, up).astype(np.uint16)


def _fp16_next_down(h):
    """kernels.cu:94-98 on fp16 bit patterns."""
    h = np.asarray(h, dtype=np.uint16)
    dn = np.where(h & np.uint16(0x8000), h + np.uint16(1), h - np.uint16(1)).astype(np.uint16)
    dn = np.where(h == 0x0000, np.uint16(0x8001), dn)
    return np.where(h == 0xFC00, h, dn).astype(np.uint16)


def sr_fp32_to_fp16_bits(x: np.ndarray, u: np.ndarray) -> np.ndarray:
    """kernels.cu:100-131: the fp16 bit pattern of x rounded stochastically with u.
    Inf / NaN keep their class (quiet NaN 0x7E00 with x's sign); |x| > 65504
    saturates to the largest finite fp16; a value fp16 holds exactly is kept;
    otherwise the round-to-nearest result q and its neighbour on x's other side
    bracket x as lo < x < hi and x goes up with probability (x - lo) / (hi - lo),
    computed in fp32."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    u = np.asarray(u, dtype=np.float32).reshape(-1)
    b = x.view(np.uint32)
    sign = np.where(b & np.uint32(0x80000000), np.uint16(0x8000), np.uint16(0)).astype(np.uint16)
    special = (b & np.uint32(0x7F800000)) == 0x7F800000
    is_nan = special & ((b & np.uint32(0x007FFFFF)) != 0)
    with np.errstate(over="ignore", invalid="ignore"):
        q = x.astype(np.float16)                    # round to nearest, ties to even
        qb = q.view(np.uint16)
        qf = q.astype(np.float32)
        below = qf < x
        lo_b = np.where(below, qb, _fp16_next_down(qb)).astype(np.uint16)
        hi_b = np.where(below, _fp16_next_up(qb), qb).astype(np.uint16)
        lo = lo_b.view(np.float16).astype(np.float32)
        hi = hi_b.view(np.float16).astype(np.float32)
        prob = (x - lo) / (hi - lo)
        out = np.where(u < prob, hi_b, lo_b).astype(np.uint16)
    out = np.where(qf == x, qb, out)
    out = np.where(np.abs(x) > np.float32(65504.0), sign | np.uint16(0x7BFF), out)
    out = np.where(special, np.where(is_nan, sign | np.uint16(0x7E00), sign | np.uint16(0x7C00)), out)
    return out.astype(np.uint16)


def sr_round_fp16(x: np.ndarray, seed: int, step: int, idx=None) -> np.ndarray:
    """fp16 bits of x (flat, float32) rounded with the stream of (seed, step)."""
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    if idx is None:
        idx = np.arange(x.size, dtype=np.uint64)
    return sr_fp32_to_fp16_bits(x, sr_uniform(seed, step, idx))
