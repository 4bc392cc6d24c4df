"""Standalone state decoders (kernels.cu:2571-2632) against a numpy restatement.

dequantize_log_nonneg follows the fallback's arithmetic (optimizer.py:340-353):
x = ((q - 1) * s) / (L - 2) + l_min in fp32, then a correctly rounded exp2.  The
expectation is the same fp32 operations in numpy followed by a float64 exp2
rounded to fp32 (correctly rounded except when the float64 result lies within an
ulp of an fp32 rounding boundary, which these inputs do not hit): bit-exact.
dequantize_dynamic is a codebook lookup times the block scale, one fp32 product:
bit-exact.  Block sizes cover the LDS-table path (>= 512) and the direct path,
including sizes that are not powers of two, and ragged tails.
"""
import numpy as np
import pytest
import torch


def _al_expect(q, scale, min_log, bs, levels):
    c = q.astype(np.int64) & (levels - 1)
    b = np.arange(q.size) // bs
    x = (np.float32(1.0) * (c - 1).astype(np.float32) * scale[b]) / np.float32(levels - 2) + min_log[b]
    v = np.exp2(x.astype(np.float64)).astype(np.float32)
    return np.where(c == 0, np.float32(0.0), v)


@pytest.mark.gpu
@pytest.mark.parametrize("v_bits", [8, 16])
@pytest.mark.parametrize("numel,bs", [(8192, 2048), (5000, 2048), (6007, 512), (4099, 300), (1000, 128), (3, 2048)])
def test_dequantize_log_nonneg(v_bits, numel, bs):
    from adafactor8bit import adafactor8bit_cuda as K
    print(f"[decode log] v_bits={v_bits} numel={numel} bs={bs}", flush=True)
    rng = np.random.default_rng(numel * 31 + bs + v_bits)
    nb = -(-numel // bs)
    levels = 256 if v_bits == 8 else 65536
    c = rng.integers(0, levels, size=numel)
    c[:: 97] = 0
    c[1:: 89] = levels - 1
    scale = rng.uniform(0.0, 40.0, size=nb).astype(np.float32)
    scale[0] = 0.0   # a block whose values are all equal
    min_log = rng.uniform(-126.0, 0.0, size=nb).astype(np.float32)
    if v_bits == 8:
        q = torch.from_numpy(c.astype(np.uint8))
    else:
        q = torch.from_numpy(c.astype(np.uint16).view(np.int16))   # codes >= 32768 read negative
    out = torch.empty(numel, dtype=torch.float32, device="cuda")
    K.dequantize_log_nonneg(out, q.cuda(), torch.from_numpy(scale).cuda(), torch.from_numpy(min_log).cuda(),
                            numel, bs, v_bits)
    want = _al_expect(c, scale, min_log, bs, levels)
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


@pytest.mark.gpu
@pytest.mark.parametrize("m_bits", [8, 4])
@pytest.mark.parametrize("numel,bs", [(4096, 256), (5000, 256), (3000, 100), (2048, 2048)])
def test_dequantize_dynamic(m_bits, numel, bs):
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit._state import dynamic_map, ensure_qmap
    print(f"[decode dyn] m_bits={m_bits} numel={numel} bs={bs}", flush=True)
    ensure_qmap(torch.device("cuda", 0))
    rng = np.random.default_rng(numel + bs + m_bits)
    nb = -(-numel // bs)
    scale = rng.uniform(1e-6, 1.0, size=nb).astype(np.float32)
    qmap = dynamic_map(m_bits).numpy().astype(np.float32)
    if m_bits == 8:
        codes = rng.integers(0, 256, size=numel)
        q = codes.astype(np.uint8)
    else:
        codes = rng.integers(0, 16, size=numel + (numel & 1))
        q = ((codes[0::2] << 4) | codes[1::2]).astype(np.uint8)
        codes = codes[:numel]
    out = torch.empty(numel, dtype=torch.float32, device="cuda")
    K.dequantize_dynamic(out, torch.from_numpy(q).cuda(), torch.from_numpy(scale).cuda(), numel, bs, m_bits)
    want = qmap[codes] * scale[np.arange(numel) // bs]
    got = out.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), int((got != want).sum())


@pytest.mark.gpu
def test_decode_matches_optimizer_state():
    """Decode the V and M state of a real step and compare with the oracle's
    restatement of the reference decoders (metadata exact, values to the 1-ulp
    difference of the reference's CPU pow)."""
    from adafactor8bit import Adafactor8Bit
    from adafactor8bit import adafactor8bit_cuda as K
    from oracle.fallback import al_dequantize
    import inputs
    print("[decode state]", flush=True)
    p = torch.nn.Parameter(inputs.make_param((300, 70), 0, 4).cuda())
    opt = Adafactor8Bit([p], lr=1e-3, beta1=0.9, beta2=0.999, factored=False, relative_step=False,
                        scale_parameter=False, block_size=512, m_block_size=128, m_quant_type="d8")
    for t in range(1, 4):
        p.grad = inputs.make_grad((300, 70), 0, t, 4).cuda()
        opt.step()
    st = opt.state[p]
    q = st["variance_q"].reshape(-1)
    out = torch.empty(q.numel(), dtype=torch.float32, device="cuda")
    K.dequantize_log_nonneg(out, q, st["variance_scale"], st["variance_min_log"], q.numel(), 512, 8)
    ref = al_dequantize(q.cpu(), st["variance_scale"].cpu(), st["variance_min_log"].cpu(), q.numel())
    np.testing.assert_allclose(out.cpu().numpy(), ref.numpy(), rtol=2.5e-7, atol=0)
