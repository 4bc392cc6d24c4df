"""The reference-named module (``adafactor8bit_cuda``) on the GPU, against the CPU oracle."""
import math

import numpy as np
import pytest
import torch

from inputs import make_grad, make_param

ADAMW = dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
             scale_parameter=False, scale_weight_decay=False, d=0.0, eps=(1e-8, 1e-3), lr=1e-4)


@pytest.mark.gpu
def test_fira_scalar_truth_table():
    """fira_scalar (kernels.cu:3030-3084) against the oracle's limiter (optimizer.py:760-782)."""
    from adafactor8bit import adafactor8bit_cuda as K
    from oracle.fallback import fira_scale
    print("[module] fira_scalar", flush=True)
    mu = 0.01
    cases = [  # (squared norm, previous norm or None)
        (4.0, None), (1.005 ** 2, 1.0), (16.0, 1.0), (25.0, 1e-7), (float("nan"), 1.0),
        (float("inf"), 2.0), (0.0, 3.0), (9.0, 0.5),
    ]
    for x, prev in cases:
        xt = torch.tensor([x], dtype=torch.float32, device="cuda")
        alpha = torch.tensor([0.125], dtype=torch.float32, device="cuda")
        pt = torch.tensor([prev if prev is not None else 0.0], dtype=torch.float32, device="cuda")
        out = K.fira_scalar(xt, pt, alpha, prev is not None, True, 1.0 + mu, 1.0 / (1.0 + mu)).cpu()
        st = {} if prev is None else {"fira_prev_norm": torch.tensor(prev, dtype=torch.float32)}
        curr = torch.tensor(x, dtype=torch.float32).sqrt()
        fs = fira_scale(st, curr, mu)
        assert out[0].item() == pytest.approx(0.125 * fs.item(), rel=2e-7), (x, prev)
        assert out[1].item() == pytest.approx(st["fira_prev_norm"].item(), rel=2e-7), (x, prev)
        assert out[2].item() == (float(np.float32(x)) if math.isfinite(x) else 0.0), (x, prev)


@pytest.mark.gpu
@pytest.mark.parametrize("mqt,vbits", [("uf8", 8), ("uf4", 8), ("d8", 8), ("uf8", 16)])
def test_module_noclip_step_matches_oracle(mqt, vbits):
    """fused_update_1d_noclip through the reference's positional signature: one AdamW step on a
    (61, 1003) fp32 param; codes bit-exact, metadata within rtol 3e-7, params within rtol 1e-5."""
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit import _state as S
    from oracle.fallback import OracleOptimizer
    print(f"[module] noclip {mqt} al{vbits}", flush=True)
    shape, bs, mbs = (61, 1003), 2048, 256
    vqt = "al8" if vbits == 8 else "al16"
    kw = dict(ADAMW, m_quant_type=mqt, v_quant_type=vqt, block_size=bs, m_block_size=mbs)
    pc = torch.nn.Parameter(make_param(shape, 0, 3))
    oc = OracleOptimizer([pc], **kw)
    g = make_grad(shape, 0, 1, 3)
    pc.grad = g
    pg = pc.detach().clone().cuda()
    oc.step()

    K.set_qmap(*[q.cuda() for q in K.qmaps()])
    st = {}
    S.new_al_slot(st, "variance", shape, bs, vqt, "cuda")
    S.new_momentum_codes(st, "m", pg.numel(), mbs, mqt, "cuda")
    bc1, bc2 = 1.0 - 0.9, 1.0 - 0.999
    alpha = (torch.tensor(1e-4, dtype=torch.float32) * (math.sqrt(bc2) / bc1)).reshape(1).cuda()
    eps1 = 1e-8
    K.fused_update_1d_noclip(
        pg, g.cuda(), st["m_q"], st["m_scale"], st["variance_q"], st["variance_scale"],
        st["variance_min_log"], alpha, 0.9, 1.0 - 0.999, eps1 * math.sqrt(bc2), True,
        math.log2(max(eps1 * eps1, 1.17549435e-38)), 0.0, pg.numel(), bs, mbs, S.m_bits(mqt),
        S.m_mode(mqt), vbits, False)
    torch.cuda.synchronize()
    so = oc.state[id(pc)]
    for k in ("variance_q", "m_q"):
        a = so[k].reshape(-1).numpy()
        b = st[k].reshape(-1).cpu().numpy()
        assert np.array_equal(a, b), f"{k}: {(a != b).sum()} codes differ"
    for k in ("variance_scale", "variance_min_log", "m_scale"):
        np.testing.assert_allclose(st[k].cpu().numpy(), so[k].reshape(-1).numpy(), rtol=3e-7, atol=0)
    # the update direction uses the hardware sqrt/reciprocal (<= 2 ulp): params to rtol 1e-5
    np.testing.assert_allclose(pg.cpu().numpy(), pc.detach().numpy(), rtol=1e-5, atol=0)


@pytest.mark.gpu
def test_module_rejects_wrong_code_dtype():
    from adafactor8bit import adafactor8bit_cuda as K
    print("[module] dtype check", flush=True)
    z = torch.zeros(4096, device="cuda")
    vq = torch.zeros(4096, dtype=torch.uint8, device="cuda")
    one = torch.ones(2, device="cuda")
    with pytest.raises(RuntimeError, match="v_bits=16"):
        K.fused_update_1d_vonly_noclip(z, z, vq, one, one, one, 0.001, 1e-8, True, -53.0, 0.0,
                                       4096, 2048, 16)


@pytest.mark.gpu
@pytest.mark.parametrize("full", [False, True])
def test_module_lag_is_noclip_at_the_lagged_scale(full):
    """fused_update_1d_lag / fused_update_1d_full_lag (kernels.cu:651-655, 1305-1309): the
    step is alpha / max(1, prev_norm / (sqrtf(numel) * d)) in fp32 and the pass sums this
    step's u^2.  The reference has no CPU branch for the lagged clip, so it is pinned by
    equivalences: parameters, codes and block metadata equal a NOCLIP step whose alpha is
    that fp32 quotient, and the sum equals the NORM pass's; momentum-only with a zero
    previous norm (a clip factor of 1) equals momentum-only NOCLIP."""
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit import _state as S
    print(f"[module] lag full={full}", flush=True)
    shape, bs, mbs, d = (61, 1003), 2048, 256, 1.0
    n = shape[0] * shape[1]
    K.set_qmap(*[q.cuda() for q in K.qmaps()])
    g = make_grad(shape, 0, 1, 5).cuda()
    p0 = make_param(shape, 0, 5).cuda()
    bc1, bc2 = 1.0 - 0.9, 1.0 - 0.999
    eps1 = 1e-8
    alpha = (torch.tensor(1e-3, dtype=torch.float32) * (math.sqrt(bc2) / bc1)).reshape(1).cuda()
    lfl = math.log2(max(eps1 * eps1, 1.17549435e-38))

    def fresh():
        st = {"p": p0.clone()}
        if full:
            st["v"] = torch.full(shape, 1e-6, dtype=torch.float32, device="cuda")
            st["m"] = torch.full(shape, 1e-4, dtype=torch.float32, device="cuda")
        else:
            S.new_al_slot(st, "variance", shape, bs, "al8", "cuda")
            S.new_momentum_codes(st, "m", n, mbs, "uf8", "cuda")
        return st

    def run(mode, st, a=None, prev=None, nb=None, mom_only=False):
        adam = not mom_only
        eps_d = eps1 * math.sqrt(bc2) if adam else 0.0
        eps_g = 0.0 if adam else eps1
        if full:
            common = (0.9, 1.0 - 0.999, max(eps1 * eps1, 1.17549435e-38), eps_d, adam, eps_g, n)
            if mode == "lag":
                K.fused_update_1d_full_lag(st["p"], g, st["v"], st["m"], nb, a, prev, *common, d, mom_only)
            elif mode == "noclip":
                K.fused_update_1d_full_noclip(st["p"], g, st["v"], st["m"], a, *common, mom_only)
            else:
                K.fused_update_1d_full_norm(g, st["v"], st["m"], nb, *common, mom_only)
            return
        q = (st["m_q"], st["m_scale"], st["variance_q"], st["variance_scale"], st["variance_min_log"])
        tail = (0.9, 1.0 - 0.999, eps_d, adam, lfl, eps_g, n, bs, mbs, 8, 0)
        if mode == "lag":
            K.fused_update_1d_lag(st["p"], g, *q, nb, a, prev, *tail, d, 8, mom_only)
        elif mode == "noclip":
            K.fused_update_1d_noclip(st["p"], g, *q, a, *tail, 8, mom_only)
        else:
            vb = torch.empty(n, dtype=torch.float32, device="cuda")
            K.fused_update_1d_norm(g, *q, vb, nb, *tail, 8, mom_only)

    keys = ("p", "v", "m") if full else ("p", "m_q", "m_scale", "variance_q", "variance_scale",
                                         "variance_min_log")
    prev = torch.tensor([7.5 * math.sqrt(n)], dtype=torch.float32, device="cuda")
    denom = max(np.float32(1.0), np.float32(prev.item()) / (np.sqrt(np.float32(n)) * np.float32(d)))
    assert denom > 7.0
    a2 = torch.tensor([np.float32(alpha.item()) / np.float32(denom)], dtype=torch.float32, device="cuda")
    sl, sn, sm = fresh(), fresh(), fresh()
    nbl = torch.zeros(1, dtype=torch.float32, device="cuda")
    nbn = torch.zeros(1, dtype=torch.float32, device="cuda")
    run("lag", sl, alpha, prev, nbl)
    run("noclip", sn, a2)
    run("norm", sm, nb=nbn)
    torch.cuda.synchronize()
    for k in keys:
        assert torch.equal(sl[k], sn[k]), k
    assert not torch.equal(sl["p"], p0)
    assert torch.equal(nbl, nbn) and nbl.item() > 0.0
    # momentum-only, zero previous norm: U is not clipped, the step is alpha
    sl, sn = fresh(), fresh()
    zero = torch.zeros(1, dtype=torch.float32, device="cuda")
    run("lag", sl, alpha, zero, torch.zeros(1, dtype=torch.float32, device="cuda"), mom_only=True)
    run("noclip", sn, alpha, mom_only=True)
    torch.cuda.synchronize()
    for k in keys:
        assert torch.equal(sl[k], sn[k]), ("momentum-only", k)


@pytest.mark.gpu
@pytest.mark.parametrize("full", [False, True], ids=["quantised", "fp32_state"])
def test_module_momentum_only_lag_divides_u(full):
    """Momentum-only LAG (kernels.cu:651-655, 1305-1309): the lagged factor divides U
    before the momentum EMA, and the step stays alpha.  With numel 4096 (sqrtf(numel)
    = 64 exactly), d = 1 and a previous norm of 512 the factor is 8 exactly, which is
    APPLY's factor for norm_buf = 512^2: the two passes give the same bits."""
    from adafactor8bit import adafactor8bit_cuda as K
    from adafactor8bit import _state as S
    print(f"[module] momentum-only lag full={full}", flush=True)
    shape, bs, mbs = (64, 64), 2048, 256
    n = 4096
    K.set_qmap(*[q.cuda() for q in K.qmaps()])
    g = make_grad(shape, 0, 1, 6).cuda()
    p0 = make_param(shape, 0, 6).cuda()
    alpha = torch.tensor([1e-3], dtype=torch.float32, device="cuda")
    eps1 = 1e-8
    eps_sq = max(eps1 * eps1, 1.17549435e-38)
    lfl = math.log2(eps_sq)

    def fresh():
        st = {"p": p0.clone()}
        if full:
            st["v"] = torch.full(shape, 1e-6, dtype=torch.float32, device="cuda")
            st["m"] = torch.full(shape, 1e-4, dtype=torch.float32, device="cuda")
        else:
            S.new_al_slot(st, "variance", shape, bs, "al8", "cuda")
            S.new_momentum_codes(st, "m", n, mbs, "uf8", "cuda")
        return st

    prev = torch.tensor([512.0], dtype=torch.float32, device="cuda")
    nb_apply = torch.tensor([512.0 * 512.0], dtype=torch.float32, device="cuda")
    sl, sa = fresh(), fresh()
    nbl = torch.zeros(1, dtype=torch.float32, device="cuda")
    if full:
        common = (0.9, 1.0 - 0.999, eps_sq, 0.0, False, eps1, n)
        K.fused_update_1d_full_lag(sl["p"], g, sl["v"], sl["m"], nbl, alpha, prev, *common, 1.0, True)
        # the three-pass flow: NORM writes V (and, momentum-only, leaves M), APPLY reads it
        K.fused_update_1d_full_norm(g, sa["v"], sa["m"], torch.zeros(1, dtype=torch.float32, device="cuda"),
                                    *common, True)
        K.fused_update_1d_full_apply(sa["p"], g, sa["v"], sa["m"], nb_apply, alpha, *common, 1.0, True)
        keys = ("p", "v", "m")
    else:
        tail = (0.9, 1.0 - 0.999, 0.0, False, lfl, eps1, n, bs, mbs, 8, 0)
        ql = (sl["m_q"], sl["m_scale"], sl["variance_q"], sl["variance_scale"], sl["variance_min_log"])
        qa = (sa["m_q"], sa["m_scale"], sa["variance_q"], sa["variance_scale"], sa["variance_min_log"])
        K.fused_update_1d_lag(sl["p"], g, *ql, nbl, alpha, prev, *tail, 1.0, 8, True)
        vb = torch.empty(n, dtype=torch.float32, device="cuda")
        K.fused_update_1d_norm(g, *qa, vb, torch.zeros(1, dtype=torch.float32, device="cuda"), *tail, 8, True)
        K.fused_update_1d_apply(sa["p"], g, *qa, vb, nb_apply, alpha, *tail, 1.0, 8, True)
        keys = ("p", "m_q", "m_scale", "variance_q", "variance_scale", "variance_min_log")
    torch.cuda.synchronize()
    for k in keys:
        assert torch.equal(sl[k], sa[k]), k
    assert not torch.equal(sl["p"], p0)
