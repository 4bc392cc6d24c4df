"""SGD path (optimizer.py:2045-2077) and the standalone momentum EMA
(fused_m_quantize_lerp, kernels.cu:523-588) on the GPU against the CPU oracle.

SGD involves no log-space codec: the momentum decode (UF: (q - c) * (s / c); D:
qmap[q] * s), the EMA (torch.lerp), the division by 1 - beta1, the absmax
requantisation and the parameter fma are the same fp32 operations on both
sides, so codes, scales, fp32 momentum and parameters are compared bit-exact
when nothing is clipped.  With d > 0 or Fira the step size depends on ||u||, a
reduction the oracle runs in torch's CPU order and the kernel in its own, so
the parameters are held to rtol 1e-6 (a few ulps of the step) while the
momentum state stays bit-exact (it does not depend on the step).  Fira's
prev-norm state is a norm: rtol 3e-5 as for the other paths.

The stochastic-rounding writeback is checked against the kernels.cu:48-87
stream restated in oracle/sr.py: a float32 twin of each bf16 parameter, stepped
from the same values, gives the exact fp32 value the bf16 write rounds.
"""
import numpy as np
import pytest
import torch

from inputs import make_grad, make_param

SGD = dict(beta1=None, beta2=None, beta2_decay=None, beta3=None, factored=False, relative_step=False,
           scale_parameter=False, scale_weight_decay=False, d=0.0, lr=1e-2)
SHAPES = [(33, 517), (300,), (5000,), (2048,), (7,), (64, 130)]


def _run_pair(kw, shapes=SHAPES, steps=4, multi=True, seed=0):
    from adafactor8bit import Adafactor8Bit
    from oracle.fallback import OracleOptimizer
    pc = [torch.nn.Parameter(make_param(s, i, seed)) for i, s in enumerate(shapes)]
    pg = [torch.nn.Parameter(p.detach().clone().cuda()) for p in pc]
    oc = OracleOptimizer(pc, **kw)
    og = Adafactor8Bit(pg if multi else [{"params": [p]} for p in pg], **kw)
    for t in range(1, steps + 1):
        for i, (a, b) in enumerate(zip(pc, pg)):
            g = make_grad(tuple(a.shape), i, t, seed)
            a.grad, b.grad = g, g.cuda()
        oc.step()
        og.step()
    torch.cuda.synchronize()
    return pc, pg, oc, og


CASES = [
    ("plain", {}),
    ("mom_uf8", dict(beta1=0.9)),
    ("mom_uf4", dict(beta1=0.9, m_quant_type="uf4")),
    ("mom_d8", dict(beta1=0.8, m_quant_type="d8")),
    ("mom_d4", dict(beta1=0.9, m_quant_type="d4", m_block_size=64)),
    ("mom_uf8_b2048", dict(beta1=0.95, m_block_size=2048)),
    ("mom_uf8_b32", dict(beta1=0.9, m_block_size=32)),
    ("mom_fp32", dict(beta1=0.9, m_quant_type="fp32")),
    ("mom_unquantized", dict(beta1=0.9, quantize=False)),
    ("wd", dict(beta1=0.9, weight_decay=0.1)),
    ("wd_scaled_maximize", dict(beta1=0.9, weight_decay=0.05, scale_weight_decay=True, maximize=True)),
    ("clip", dict(beta1=0.9, d=1.0, lr=1.0)),
    ("clip_nomom", dict(d=0.5, lr=1.0)),
    ("fira", dict(beta1=0.9, enable_fira_for_adafactor=True, fira_margin=0.01)),
    ("fira_clip_fp32m", dict(beta1=0.9, m_quant_type="fp32", enable_fira_for_adafactor=True, d=1.0)),
    ("scale_param", dict(beta1=0.9, scale_parameter=True)),
]


def _compare(name, pc, pg, oc, og, exact_params):
    for i, (a, b) in enumerate(zip(pc, pg)):
        ra, rb = a.detach().numpy(), b.detach().cpu().numpy()
        if exact_params:
            assert np.array_equal(ra.view(np.uint32), rb.view(np.uint32)), \
                f"{name} p{i}: {int((ra != rb).sum())} params differ"
        else:
            np.testing.assert_allclose(rb, ra, rtol=1e-6, atol=1e-9, err_msg=f"{name} p{i}")
        sc, sg = oc.state[id(a)], og.state[b]
        for k, v in sc.items():
            if not torch.is_tensor(v):
                continue
            assert k in sg, f"{name} p{i}: missing state {k}"
            mine = sg[k].detach().cpu()
            assert mine.dtype == v.dtype and tuple(mine.shape) == tuple(v.shape), (name, i, k)
            if k == "fira_prev_norm":
                np.testing.assert_allclose(mine.numpy(), v.numpy(), rtol=3e-5, err_msg=f"{name} p{i} {k}")
            else:
                assert torch.equal(mine, v), f"{name} p{i} {k}: {int((mine != v).sum())} differ"


@pytest.mark.gpu
@pytest.mark.parametrize("name,extra", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("multi", [True, False])
def test_sgd_matches_oracle(name, extra, multi):
    print(f"[sgd] {name} multi={multi}", flush=True)
    kw = dict(SGD, **extra)
    pc, pg, oc, og = _run_pair(kw, multi=multi)
    clipped = kw.get("d", 0.0) > 0 or kw.get("enable_fira_for_adafactor", False) or kw.get("scale_parameter")
    _compare(name, pc, pg, oc, og, exact_params=not clipped)


@pytest.mark.gpu
@pytest.mark.parametrize("mqt", ["uf8", "fp32", None])
def test_sgd_bf16_sr_writeback_stream(mqt):
    """bf16 params with stochastic rounding: every written bit pattern is the
    kernels.cu:48-87 rounding of the fp32 value a float32 twin computes."""
    from adafactor8bit import Adafactor8Bit
    from oracle.sr import sr_round_bf16
    print(f"[sgd sr] mqt={mqt}", flush=True)
    kw = dict(SGD, lr=0.05, weight_decay=0.1, stochastic_round_writeback=True)
    if mqt is not None:
        kw.update(beta1=0.9, m_quant_type=mqt)
    shapes = [(33, 517), (300,), (4096,)]
    pb = [torch.nn.Parameter(make_param(s, i, 3).to(torch.bfloat16).cuda()) for i, s in enumerate(shapes)]
    pf = [torch.nn.Parameter(p.detach().float()) for p in pb]
    ob, of = Adafactor8Bit(pb, **kw), Adafactor8Bit(pf, **dict(kw, stochastic_round_writeback=False))
    for t in range(1, 4):
        with torch.no_grad():
            for a, b in zip(pf, pb):
                a.copy_(b.float())
        for i, (a, b) in enumerate(zip(pf, pb)):
            g = make_grad(tuple(a.shape), i, t, 3).to(torch.bfloat16)
            b.grad, a.grad = g.cuda(), g.float().cuda()
        ob.step()
        of.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pf, pb)):
            seed = int(ob.state[b]["sr_seed"])
            want = sr_round_bf16(a.detach().cpu().numpy(), seed, t).astype(np.uint16)
            got = b.detach().cpu().reshape(-1).view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(got, want), f"step {t} p{i}: {int((got != want).sum())} differ"


@pytest.mark.gpu
@pytest.mark.parametrize("mqt", ["uf8", "uf4", "d8", "d4"])
@pytest.mark.parametrize("numel,bs", [(5000, 256), (4096, 2048), (3001, 32), (7, 64)])
@pytest.mark.parametrize("xdt", [torch.float32, torch.bfloat16])
def test_fused_m_quantize_lerp_matches_oracle(mqt, numel, bs, xdt):
    """The module's fused_m_quantize_lerp against _m_ema_pytorch's restatement,
    three EMA steps from the zero state: codes, scales and m' bit-exact."""
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit._state import ensure_qmap
    from oracle.fallback import m_ema, init_m, m_bits_of
    print(f"[m_ema] {mqt} numel={numel} bs={bs} x={xdt}", flush=True)
    ensure_qmap(torch.device("cuda", 0))
    st = {}
    init_m(st, numel, (numel,), bs, mqt, True)
    q, s = st["m_q"].clone().cuda(), st["m_scale"].clone().cuda()
    out = torch.empty(numel, dtype=torch.float32, device="cuda")
    bits = m_bits_of(mqt)
    mode = 1 if mqt.startswith("d") else 0
    for t in range(1, 4):
        x = make_grad((numel,), 0, t, 5).to(xdt)
        want = m_ema(st, x.float(), 0.9, mqt, bs, True)
        K.fused_m_quantize_lerp(q, s, x.cuda(), out, 0.9, bs, numel, bits, mode)
        torch.cuda.synchronize()
        assert torch.equal(q.cpu(), st["m_q"]), f"step {t}: {int((q.cpu() != st['m_q']).sum())} codes differ"
        assert torch.equal(s.cpu(), st["m_scale"]), f"step {t}: scales"
        assert torch.equal(out.cpu(), want.reshape(-1)), f"step {t}: m'"
