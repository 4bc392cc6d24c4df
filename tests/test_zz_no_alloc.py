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


@pytest.mark.gpu
@pytest.mark.filterwarnings("ignore:The CUDA Graph is empty")
def test_noalloc_refuses_stale_table_and_captured_upload():
    """upload == 0 with tensors other than those last uploaded, and upload != 0 on a
    capturing stream, are refused before any launch (A8_ERR_ARG)."""
    from adafactor8bit import _native as nat
    L = nat.lib()
    dev = torch.device("cuda", 0)
    strm = torch.cuda.current_stream(dev).cuda_stream
    shapes = [(3000,), (2048,)]
    ps = [make_param(s, i, 19).reshape(-1).to(dev) for i, s in enumerate(shapes)]
    gs = [make_grad((p.numel(),), i, 1, 19).to(dev) for i, p in enumerate(ps)]
    sts = [_state(p.numel(), dev) for p in ps]
    recs = _records(nat, ps, gs, sts)
    nat.check(L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, recs, 2, *_hyper(1), 1, None, strm), "upload")
    torch.cuda.synchronize()
    before = [p.clone() for p in ps]
    print("[noalloc] stale table refused", flush=True)
    one = _records(nat, ps[:1], gs[:1], sts[:1])          # fewer tensors than the uploaded table
    assert L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, one, 1, *_hyper(2), 0, None, strm) == -1
    assert b"differ" in L.a8_last_error()
    other = _records(nat, [ps[1], ps[0]], [gs[1], gs[0]], [sts[1], sts[0]])   # same tensors, other order
    assert L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, other, 2, *_hyper(2), 0, None, strm) == -1
    torch.cuda.synchronize()
    for p, b in zip(ps, before):
        assert torch.equal(p, b)   # nothing ran
    print("[noalloc] upload under capture refused", flush=True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            rc = L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, recs, 2, *_hyper(2), 1, None,
                                                    torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    assert rc == -1 and b"capturing" in L.a8_last_error(), rc


@pytest.mark.gpu
def test_noalloc_captured_replays_equal_eager_calls():
    """One eager call uploads the table; a8_fused_update_1d_multi_noalloc with upload
    == 0 captured in a HIP graph then replays as the same call: five replays (new
    gradients in the same buffers, eager work between them) leave parameters and
    states bit-identical to five eager a8_fused_update_1d_multi calls."""
    from adafactor8bit import _native as nat
    L = nat.lib()
    dev = torch.device("cuda", 0)
    strm = torch.cuda.current_stream(dev).cuda_stream
    shapes = [(700, 300), (5000,), (4096,), (3, 700)]
    base = [make_param(s, i, 23).reshape(-1) for i, s in enumerate(shapes)]
    pa = [b.clone().to(dev) for b in base]
    pb = [b.clone().to(dev) for b in base]
    sa = [_state(b.numel(), dev) for b in base]
    sb = [_state(b.numel(), dev) for b in base]
    ga = [torch.zeros_like(p) for p in pa]
    gb = [torch.zeros_like(p) for p in pb]
    table = torch.empty(int(L.a8_table_bytes_1d(len(shapes))), dtype=torch.uint8, device=dev)
    ra, rb = _records(nat, pa, ga, sa), _records(nat, pb, gb, sb)
    hyp = _hyper(1)   # host scalars: the captured call keeps those of its capture

    def load(t):
        for i in range(len(shapes)):
            g = make_grad((base[i].numel(),), i, t, 23).to(dev)
            ga[i].copy_(g)
            gb[i].copy_(g)

    load(1)
    nat.check(L.a8_fused_update_1d_multi(0, 0, nat.F32, ra, len(shapes), table.data_ptr(), table.numel(), *hyp, 1,
                                         None, strm), "multi")
    nat.check(L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, rb, len(shapes), *hyp, 1, None, strm), "noalloc")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph):
            rc = L.a8_fused_update_1d_multi_noalloc(0, 0, nat.F32, rb, len(shapes), *hyp, 0, None,
                                                    torch.cuda.current_stream().cuda_stream)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    nat.check(rc, "captured noalloc")
    for t in range(2, 7):
        print(f"[noalloc capture] replay {t - 1}", flush=True)
        load(t)
        nat.check(L.a8_fused_update_1d_multi(0, 0, nat.F32, ra, len(shapes), table.data_ptr(), table.numel(), *hyp,
                                             0, None, strm), "multi")
        graph.replay()
        junk = torch.randn(4096, device=dev).sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for i in range(len(shapes)):
            assert torch.equal(pa[i], pb[i]), f"replay {t - 1}: param {i}"
            for k in sa[i]:
                assert torch.equal(sa[i][k], sb[i][k]), f"replay {t - 1}: {k} of tensor {i}"
