"""a8_fused_update_1d_multi_noalloc (the multi-tensor AdamW step with its tensor table
in the library's own device array, no allocation) against a8_fused_update_1d_multi,
through the C ABI: bit-identical parameters and states over calls in a row, the
second one on a smaller set of tensors, then a call that reuses the table."""
import ctypes

import pytest
import torch

from inputs import make_grad, make_param

BV, BM = 2048, 256


def _state(numel, dev):
    nv = -(-numel // BV)
    nm = -(-numel // BM)
    return {"m_q": torch.full((nm * BM,), 128, dtype=torch.uint8, device=dev),
            "m_scale": torch.ones(nm, dtype=torch.float32, device=dev),
            "v_q": torch.zeros(nv * BV, dtype=torch.uint8, device=dev),
            "v_scale": torch.ones(nv, dtype=torch.float32, device=dev),
            "v_min_log": torch.zeros(nv, dtype=torch.float32, device=dev)}


def _records(nat, params, grads, states):
    arr = (nat.Tensor1D * len(params))()
    for i, (p, g, st) in enumerate(zip(params, grads, states)):
        arr[i] = nat.Tensor1D(p.data_ptr(), g.data_ptr(), st["m_q"].data_ptr(), st["m_scale"].data_ptr(),
                              st["v_q"].data_ptr(), st["v_scale"].data_ptr(), st["v_min_log"].data_ptr(), None,
                              None, None, None, None, p.numel(), 0)
    return arr


# AdamW UF8/AL8 (the adamw preset at step t): beta1, 1 - beta2, eps_d (bias-corrected),
# Adam denominator, AL floor, eps_g, eps_sq, B_V, B_M, m_bits 8, UF mode, d 0, AL8,
# momentum_only 0, step, alpha, no decay
def _hyper(t):
    return (0.9, 1.0 - 0.999, 1e-8 * (1.0 - 0.999 ** t) ** 0.5, 1, -126.0, 0.0, 1e-16, BV, BM, 8, 0, 0.0, 8, 0, t,
            1e-4 * (1.0 - 0.999 ** t) ** 0.5 / (1.0 - 0.9 ** t), 1.0, 0)


@pytest.mark.gpu
def test_noalloc_matches_multi_over_calls():
    from adafactor8bit import _native as nat
    L = nat.lib()
    dev = torch.device("cuda", 0)
    strm = torch.cuda.current_stream(dev).cuda_stream
    shapes = [(512, 300), (2048,), (77, 1000), (5000,), (4096,), (3, 700)]
    # the second call steps a smaller set: three of the tensors
    calls = [list(range(len(shapes))), [1, 3, 5], [1, 3, 5]]
    base = [make_param(s, i, 13).reshape(-1) for i, s in enumerate(shapes)]
    pa = [b.clone().to(dev) for b in base]
    pb = [b.clone().to(dev) for b in base]
    sa = [_state(b.numel(), dev) for b in base]
    sb = [_state(b.numel(), dev) for b in base]
    table = torch.empty(int(L.a8_table_bytes_1d(len(shapes))), dtype=torch.uint8, device=dev)
    # gradient buffers stay put: a table reused with upload == 0 holds their addresses
    gbuf = [torch.empty_like(p) for p in pa]
    for t, idx in enumerate(calls, start=1):
        print(f"[noalloc] call {t}: tensors {idx}", flush=True)
        for i in idx:
            gbuf[i].copy_(make_grad((base[i].numel(),), i, t, 13))
        grads = [gbuf[i] for i in idx]
        ra = _records(nat, [pa[i] for i in idx], grads, [sa[i] for i in idx])
        rb = _records(nat, [pb[i] for i in idx], grads, [sb[i] for i in idx])
        upload = 0 if t == 3 else 1   # the third call reuses the second call's table
        rc = L.a8_fused_update_1d_multi(0, 0, nat.F32, ra, len(idx), table.data_ptr(), table.numel(), *_hyper(t),
                                        1, None, strm)
        nat.check(rc, "a8_fused_update_1d_multi")
        rc = L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, rb, len(idx), *_hyper(t), upload, None, strm)
        nat.check(rc, "a8_fused_update_1d_multi_noalloc")
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            assert torch.equal(pa[i], pb[i]), f"call {t}: param {i}"
            for k in sa[i]:
                assert torch.equal(sa[i][k], sb[i][k]), f"call {t}: {k} of tensor {i}"
    # the tensors stepped every call moved; the others only on the first call
    for i in range(len(shapes)):
        assert not torch.equal(pa[i].cpu(), base[i])
