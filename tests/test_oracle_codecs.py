"""Closed-form, brute-force and known-answer checks that pin the oracle's codecs
independently of the golden trajectories (CPU only)."""
import collections
import math

import pytest
import torch

from oracle import fallback as F


# ---------------------------------------------------------------- AL8 / AL16
def _decode_codes(codes, lmin, s, levels):
    """Block of values whose exact log2 sits on the code grid: v_k = 2^(lmin + (k-1)*s/(L-2))."""
    return torch.tensor([2.0 ** (lmin + (k - 1) * s / (levels - 2)) for k in codes], dtype=torch.float32)


@pytest.mark.parametrize("levels", [256, 65536])
def test_al_grid_values_encode_to_their_code(levels):
    # l_min = -20 and l_max = 4 are exact in float; every grid value must land on its own code.
    lmin, lmax = -20.0, 4.0
    top = levels - 1
    codes = list(range(1, top + 1)) if levels == 256 else list(range(1, top + 1, 97)) + [top]
    bs = 1 << (len(codes) - 1).bit_length()
    v = _decode_codes(codes, lmin, lmax - lmin, levels)
    v = torch.nn.functional.pad(v, (0, bs - v.numel()))
    q, scale, ml, pad = F.al_quantize(v, bs, levels=levels)
    assert pad == 0 and ml.item() == lmin and scale.item() == lmax - lmin
    got = q.reshape(-1)[:len(codes)].to(torch.int64)
    if levels == 65536:
        got = torch.where(got < 0, got + 65536, got)
    assert got.tolist() == codes
    assert (q.reshape(-1)[len(codes):] == 0).all()  # padding and zeros keep code 0


def test_al8_every_code_round_trips():
    lmin, lmax = -20.0, 4.0
    codes = list(range(0, 256))
    v = torch.cat([torch.zeros(1), _decode_codes(codes[1:], lmin, lmax - lmin, 256)])
    q, scale, ml, _ = F.al_quantize(v, 256)
    dec = F.al_dequantize(q, scale, ml, 256)
    q2, _, _, _ = F.al_quantize(dec, 256)
    assert q.reshape(-1).tolist() == codes
    assert torch.equal(q2.reshape(-1), q.reshape(-1))
    assert dec[0] == 0 and dec[1] == 2.0 ** lmin and dec[255] == 2.0 ** lmax


def test_al16_int16_storage_wraps():
    v = torch.tensor([2.0 ** -10, 1.0, 2.0 ** 10, 0.0])
    q, scale, ml, _ = F.al_quantize(v, 4, levels=65536)
    assert q.dtype == torch.int16
    assert q.reshape(-1).tolist() == [1, 32768 - 65536, -1, 0]  # 32768 and 65535 stored wrapped
    dec = F.al_dequantize(q, scale, ml, 4)
    assert dec.tolist() == [2.0 ** -10, 1.0, 2.0 ** 10, 0.0]


def test_al_zero_code_iff_zero_and_all_zero_block():
    g = torch.Generator().manual_seed(1)
    v = torch.rand(4096, generator=g) ** 8
    v[::7] = 0
    v[2048:] = 0  # second block all zero
    q, scale, ml, _ = F.al_quantize(v, 2048)
    q = q.reshape(-1)
    assert torch.equal(q == 0, v == 0)
    dec = F.al_dequantize(q, scale, ml, v.numel())
    assert torch.equal(dec == 0, v == 0)


def test_al_half_step_error_bound_and_monotone():
    g = torch.Generator().manual_seed(2)
    v = torch.exp(torch.randn(8192, generator=g) * 6)
    q, scale, ml, _ = F.al_quantize(v, 2048)
    dec = F.al_dequantize(q, scale, ml, v.numel())
    s = scale.repeat_interleave(2048)
    bound = torch.pow(2.0, s / 508.0) - 1.0  # half a log-space step
    rel = (dec / v - 1.0).abs()
    assert (rel <= bound * (1 + 1e-4) + 1e-6).all()
    for b in range(4):
        blk = slice(b * 2048, (b + 1) * 2048)
        order = torch.argsort(v[blk])
        assert (q.reshape(-1)[blk][order].diff().to(torch.int32) >= 0).all()


def test_al_floor_and_degenerate_block():
    tiny = torch.full((128,), 1e-44)  # log2 below the floor
    tiny[0] = 1.0
    _, _, ml, _ = F.al_quantize(tiny, 128)
    assert ml.item() == -126.0
    const = torch.full((128,), 3.0)
    q, scale, ml, _ = F.al_quantize(const, 128)
    assert ml.item() == math.log2(3.0) - 1.0 or abs(ml.item() - (math.log2(3.0) - 1.0)) < 1e-6
    assert scale.item() == pytest.approx(1.0, abs=1e-6)
    assert (q == 255).all()


# ---------------------------------------------------------------- UF8 / UF4
def test_uf8_all_codes_and_asymmetry():
    m = torch.arange(-128, 128, dtype=torch.float32) / 128.0  # absmax 1 (from -1)
    q, amax = F.uf_quantize(m, 256, 8)
    assert amax.item() == 1.0
    assert q.tolist() == list(range(256))
    assert torch.equal(F.uf_dequantize(q, amax, 256, 256, 8), m)
    # +absmax rounds to 128 and clamps to 127: the codec is asymmetric at the top
    q2, _ = F.uf_quantize(torch.tensor([1.0, -0.5] + [0.0] * 30), 32, 8)
    assert q2[0].item() == 255 and q2[1].item() == 64


def test_uf4_nibble_order_and_codes():
    m = torch.arange(-8, 8, dtype=torch.float32) / 8.0
    q, amax = F.uf_quantize(m, 16, 4)
    assert q.numel() == 8
    assert [(int(b) >> 4, int(b) & 15) for b in q] == [(2 * i, 2 * i + 1) for i in range(8)]
    assert torch.equal(F.uf_dequantize(q, amax, 16, 16, 4), m)


# ---------------------------------------------------------------- dynamic codebook
@pytest.mark.parametrize("bits,zero_at", [(8, 127), (4, 7)])
def test_dynamic_map_structure(bits, zero_at):
    qm = F.dynamic_map(bits)
    assert qm.numel() == 2 ** bits
    assert (qm.diff() > 0).all()
    assert qm[zero_at] == 0 and qm[-1] == 1.0
    assert qm[0] > -1.0  # the negative side stops short of -1
    # the host's own codebook (uploaded to the device) is the same table
    from adafactor8bit._state import dynamic_map as host_map
    assert torch.equal(host_map(bits), qm)


@pytest.mark.parametrize("bits", [8, 4])
def test_dynamic_codec_identity_on_codebook(bits):
    qm = F.dynamic_map(bits)
    n = qm.numel()
    q, amax = F.d_quantize(qm.clone(), n, bits)
    assert amax.item() == 1.0
    ids = q.long() if bits == 8 else F._unpack_nibbles(q).long()
    assert ids.tolist() == list(range(n))
    assert torch.equal(F.d_dequantize(q, amax, n, n, bits), qm)


def test_dynamic_codec_sign_is_kept():
    x = torch.tensor([1e-9, -1e-9, 1.0] + [0.0] * 29)
    q, _ = F.d_quantize(x, 32, 8)
    qm = F.dynamic_map(8)
    assert qm[q[0].long()] > 0 and qm[q[1].long()] < 0


# ---------------------------------------------------------------- Fira
def test_fira_truth_table():
    mu = 0.01
    st = {}
    assert F.fira_scale(st, torch.tensor(2.0), mu).item() == 1.0  # first step: no limit
    assert st["fira_prev_norm"].item() == 2.0
    st = {"fira_prev_norm": torch.tensor(1.0)}
    assert F.fira_scale(st, torch.tensor(1.005), mu).item() == 1.0  # growth below 1+mu passes
    assert st["fira_prev_norm"].item() == pytest.approx(1.005)
    st = {"fira_prev_norm": torch.tensor(1.0)}
    s = F.fira_scale(st, torch.tensor(4.0), mu).item()
    assert 4.0 * s == pytest.approx(1.0 + mu, rel=1e-6)  # limited to (1+mu) x previous
    assert st["fira_prev_norm"].item() == pytest.approx(1.0 + mu, rel=1e-6)
    st = {"fira_prev_norm": torch.tensor(1e-7)}
    assert F.fira_scale(st, torch.tensor(5.0), mu).item() == 1.0  # reset below 1e-6
    assert st["fira_prev_norm"].item() == 5.0
    st = {"fira_prev_norm": torch.tensor(1.0)}
    assert F.fira_scale(st, torch.tensor(float("nan")), mu).item() == 1.0  # non-finite -> 0
    assert st["fira_prev_norm"].item() == 0.0


# ---------------------------------------------------------------- State MiB known answers
def _tinyllama_shapes():
    H, Fd, KV, V, L = 2048, 5632, 256, 32000, 22
    shapes = [(V, H)]
    for _ in range(L):
        shapes += [(H, H), (KV, H), (KV, H), (H, H), (Fd, H), (Fd, H), (H, Fd), (H,), (H,)]
    return shapes + [(H,), (V, H)]


def _state_mib(**group):
    from adafactor8bit import _state as S

    class _Opt:
        state = collections.defaultdict(dict)
        _apollo_seed_counter = 0

    params = []
    for s in _tinyllama_shapes():
        p = torch.nn.Parameter(torch.empty(s, device="meta"))
        p.grad = torch.empty(s, device="meta")
        params.append(p)
    out = []
    S.init_group(_Opt(), dict(group, params=params), [], [], out)
    return sum(S.state_bytes(st) for st in out) / 2 ** 20


@pytest.mark.parametrize("group,mib", [
    (dict(beta1=0.9, beta2=0.999, factored=False, block_size=2048, m_quant_type="uf8",
          v_quant_type="al8"), 2119.2),
    (dict(beta1=0.9, beta2=0.999, beta3=0.9999, factored=True, block_size=2048, m_quant_type="uf8",
          v_quant_type="al8", c_quant_type="al8"), 1068.0),
    (dict(beta1=0.9, beta2=0.999, beta3=0.9999, factored=True, block_size=2048, m_quant_type="uf8",
          v_quant_type="al8", c_quant_type="fp32"), 1070.3),
    (dict(beta1=0.9, beta2=0.999, beta3=0.9999, factored=True, block_size=2048, m_quant_type="uf8",
          v_quant_type="al16", c_quant_type="al16"), 1069.8),
    (dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=True, block_size=256,
          v_quant_type="al8"), 1.2),
    (dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=True, block_size=2048,
          v_quant_type="al8"), 1.3),
])
def test_state_mib_matches_readme(group, mib):
    """README.md:63-77 'State' column for TinyLlama-1.1B (MiB of optimizer-owned tensors)."""
    assert round(_state_mib(**group), 1) == mib
