"""CPU restatement of the projection schedule of capturable APOLLO steps (TEST
INFRASTRUCTURE ONLY: imported by tests/ as the checker, never by the product).

The reference refreshes an APOLLO matrix's projection on the host
(_get_apollo_proj_matrix, optimizer.py:2557-2584): when step - last_proj_step >=
apollo_update_proj_gap, current_proj_seed = apollo_seed, apollo_seed =
next_seed(current_proj_seed) (optimizer.py:152-155) and P = stable_randn(shape,
current_proj_seed) / sqrt(rank) (optimizer.py:139-149).  A capturable step runs
that schedule on the device, which needs:

* ``next_seed``: the last of 15 ``torch.randint(0, 2**63 - 1)`` draws from a CPU
  generator seeded with the seed.  torch's CPU generator is MT19937 (Matsumoto and
  Nishimura, 1998) initialised from the seed's low 32 bits; a 64-bit draw joins
  two 32-bit outputs, the first as the high word, reduced modulo 2^63 - 1.
  Restated here from the published MT19937 and pinned against torch itself
  (tests/test_oracle_apollo_proj.py).
* a generator for P that the device can run: P's row-major element k is
  z / sqrt(r), z the Box-Muller transform (Box and Muller, 1958) of
  u1 = ((a >> 11) + 1) 2^-53 and u2 = (b >> 11) 2^-53, with a, b outputs 2k + 1
  and 2k + 2 of SplitMix64 (Steele, Lea and Flood, 2014) seeded with the seed,
  in double precision, rounded to fp32, then divided in fp32 by fp32(sqrt(r)).
  This is the build's own generator (stable_randn's torch generator is seeded on
  the host and cannot be replayed); it is pinned by SplitMix64's published
  outputs (oracle/sr.py) and by the distribution it must produce.
"""
import numpy as np

from oracle.sr import splitmix64

_M32 = 0xFFFFFFFF
_GOLD = np.uint64(0x9E3779B97F4A7C15)


def mt19937_outputs(seed: int, n: int):
    """The first n tempered outputs of MT19937 initialised with seed & 0xFFFFFFFF
    (init_genrand of the published algorithm; n <= 624)."""
    mt = [0] * 624
    mt[0] = seed & _M32
    for j in range(1, 624):
        mt[j] = (1812433253 * (mt[j - 1] ^ (mt[j - 1] >> 30)) + j) & _M32
    for i in range(624):
        y = (mt[i] & 0x80000000) | (mt[(i + 1) % 624] & 0x7FFFFFFF)
        mt[i] = mt[(i + 397) % 624] ^ (y >> 1) ^ (0x9908B0DF if y & 1 else 0)
    out = []
    for y in mt[:n]:
        y ^= y >> 11
        y ^= (y << 7) & 0x9D2C5680
        y ^= (y << 15) & 0xEFC60000
        y ^= y >> 18
        out.append(y & _M32)
    return out


def next_seed(seed: int, adv: int = 15) -> int:
    """optimizer.py:152-155 restated: the adv-th 64-bit draw modulo 2^63 - 1."""
    o = mt19937_outputs(seed, 2 * adv)
    return ((o[2 * adv - 2] << 32) | o[2 * adv - 1]) % (2 ** 63 - 1)


def normals(seed: int, k) -> np.ndarray:
    """z of P's row-major elements k (array), float32, before the 1/sqrt(r) scaling."""
    k = np.asarray(k, dtype=np.uint64)
    with np.errstate(over="ignore"):
        a = splitmix64(np.uint64(seed) + (np.uint64(2) * k) * _GOLD)                 # output 2k + 1
        b = splitmix64(np.uint64(seed) + (np.uint64(2) * k + np.uint64(1)) * _GOLD)  # output 2k + 2
    u1 = ((a >> np.uint64(11)) + np.uint64(1)).astype(np.float64) * 2.0 ** -53
    u2 = (b >> np.uint64(11)).astype(np.float64) * 2.0 ** -53
    z = np.sqrt(-2.0 * np.log(u1)) * np.cos(6.283185307179586 * u2)
    return z.astype(np.float32)


def proj_t(rows: int, cols: int, rank: int, seed: int) -> np.ndarray:
    """P^T of a rows x cols matrix at rank r: right side (rows >= cols) P is r x cols
    and P^T [cols x r]; left side P is rows x r and P^T [r x rows]."""
    right = rows >= cols
    pshape = (rank, cols) if right else (rows, rank)
    z = normals(seed, np.arange(pshape[0] * pshape[1], dtype=np.uint64)).reshape(pshape)
    p = z / np.float32(np.sqrt(float(rank)))
    return np.ascontiguousarray(p.T)
