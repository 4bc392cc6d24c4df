"""Edge-case parameter sets on the GPU.

* Empty parameters (numel 0: shapes (0,), (0, 8), (8, 0), (2, 0, 3)) sit in a
  group with ordinary ones under every update path -- quantised and fp32 1-D,
  factored Adafactor and CAME, SGD, APOLLO -- and take steps without a launch
  error, while the others step exactly as in an optimizer without them.
* One optimizer holding bf16 matrices beside fp32 vectors (a model cast to bf16
  with its norms kept in fp32) steps each parameter as an optimizer holding
  only parameters of its dtype would.
* A quantised 1-D tensor past 2^31 elements steps as its two halves do.
* lr and weight decay changed between steps reach the next launch.
* A group added with add_param_group mid-run steps on its own count and can be
  captured together with the first group.
* Parameters and gradients that are views into flat buffers starting off a 16-byte
  boundary step as aligned copies of them do, eagerly and captured.
"""
import pytest
import torch

from inputs import make_grad, make_param

PATHS = {
    "adamw_q1d": dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
                      scale_parameter=False, d=0.0, lr=1e-3, block_size=256, m_block_size=64),
    "adamw_fp32": dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
                       scale_parameter=False, d=1.0, lr=1e-3, quantize=False),
    "adafactor_factored": dict(beta1=None, beta2=None, beta2_decay=-0.8, factored=True, lr=1e-3, block_size=256),
    "came": dict(beta1=0.9, beta2=0.999, beta2_decay=None, beta3=0.9999, factored=True, relative_step=False,
                 lr=1e-3, block_size=256, d=1.0, enable_fira_for_adafactor=True),
    "sgd_clip": dict(beta1=0.9, beta2=None, beta2_decay=None, factored=False, relative_step=False,
                     scale_parameter=False, d=1.0, lr=1e-2, block_size=256, m_block_size=64),
    "apollo": dict(beta1=0.9, beta2=0.999, beta2_decay=None, factored=False, relative_step=False,
                   scale_parameter=False, d=0.0, lr=1e-3, apollo_rank=16, block_size=256, m_block_size=64),
}
SHAPES = [(300, 200), (1000,), (64, 96)]
EMPTY = [(0,), (0, 8), (8, 0), (2, 0, 3)]


def _params(shapes, seed, dtype=torch.float32):
    return [torch.nn.Parameter(make_param(s, i, seed).to("cuda", dtype)) if 0 not in s else
            torch.nn.Parameter(torch.zeros(s, device="cuda", dtype=dtype)) for i, s in enumerate(shapes)]


def _grads(ps, t, seed):
    for i, p in enumerate(ps):
        p.grad = (make_grad(tuple(p.shape), i, t, seed, zero_frac=0.0).to("cuda", p.dtype) if p.numel() else
                  torch.zeros_like(p))


@pytest.mark.gpu
@pytest.mark.parametrize("path", sorted(PATHS))
def test_empty_parameters_step_beside_ordinary_ones(path):
    from adafactor8bit import Adafactor8Bit
    print(f"[empty params] {path}", flush=True)
    kw = PATHS[path]
    pa = _params(SHAPES + EMPTY, 41)
    pb = _params(SHAPES, 41)
    oa = Adafactor8Bit(pa, **kw)
    ob = Adafactor8Bit(pb, **kw)
    for t in range(1, 4):
        _grads(pa, t, 41)
        _grads(pb, t, 41)
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pa[:len(SHAPES)], pb)):
        assert torch.equal(a, b), f"{path}: param {i}"
    for p in pa[len(SHAPES):]:
        assert p.numel() == 0 and oa.state[p]["step"] == 3
    # the state of the mixed set round-trips through a checkpoint and steps on
    sd = oa.state_dict()
    oc = Adafactor8Bit(pa, **kw)
    oc.load_state_dict(sd)
    _grads(pa, 4, 41)
    _grads(pb, 4, 41)
    oc.step()
    ob.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pa[:len(SHAPES)], pb)):
        assert torch.equal(a, b), f"{path}: param {i} after the checkpoint"


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["adamw_q1d", "adafactor_factored", "apollo"])
def test_bf16_matrices_beside_fp32_vectors(path):
    """Matrices in bf16 (stochastic rounding) and vectors in fp32 in one group; each
    steps as in an optimizer holding only its own dtype's parameters."""
    from adafactor8bit import Adafactor8Bit
    print(f"[mixed dtypes] {path}", flush=True)
    kw = dict(PATHS[path], stochastic_round_writeback=True)
    mats, vecs = [(300, 200), (64, 96)], [(1000,), (256,)]
    m1, v1 = _params(mats, 43, torch.bfloat16), _params(vecs, 44)
    m2, v2 = _params(mats, 43, torch.bfloat16), _params(vecs, 44)
    both = Adafactor8Bit(m1 + v1, **kw)
    only_m, only_v = Adafactor8Bit(m2, **kw), Adafactor8Bit(v2, **kw)
    for t in range(1, 4):
        _grads(m1, t, 43); _grads(v1, t, 44)
        _grads(m2, t, 43); _grads(v2, t, 44)
        both.step(); only_m.step(); only_v.step()
    torch.cuda.synchronize()
    for a, b in zip(m1 + v1, m2 + v2):
        assert a.dtype == b.dtype and torch.equal(a, b), tuple(a.shape)


@pytest.mark.gpu
def test_quantised_1d_step_past_2_31_elements():
    """A tensor of 2^31 + 8192 elements (AdamW UF8 / AL8, B_V 2048, B_M 256) steps as
    its two block-aligned halves stepped as separate tensors do: the update is
    elementwise inside blocks, so the bits must agree whatever the element index's
    width.  (About 40 GB of device memory.)"""
    from adafactor8bit import Adafactor8Bit
    n1 = 1 << 31
    n = n1 + 8192
    print(f"[2^31] one tensor of {n} elements against two halves", flush=True)
    kw = dict(PATHS["adamw_q1d"], block_size=2048, m_block_size=256)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    big = torch.nn.Parameter(torch.randn(n, device="cuda", generator=gen) * 0.02)
    halves = [torch.nn.Parameter(big.detach()[:n1].clone()), torch.nn.Parameter(big.detach()[n1:].clone())]
    oa = Adafactor8Bit([big], **kw)
    ob = Adafactor8Bit(halves, **kw)
    for t in range(2):
        g = torch.randn(n, device="cuda", generator=gen) * 1e-3
        big.grad = g
        halves[0].grad = g[:n1].clone()
        halves[1].grad = g[n1:].clone()
        del g
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        assert torch.equal(big.detach()[:n1], halves[0].detach()), f"step {t + 1}: first half"
        assert torch.equal(big.detach()[n1:], halves[1].detach()), f"step {t + 1}: second half"
    sa, sb0, sb1 = oa.state[big], ob.state[halves[0]], ob.state[halves[1]]
    for k in ("variance_q", "m_q"):   # codes, stored as [blocks, block] views
        assert torch.equal(sa[k].reshape(-1), torch.cat([sb0[k].reshape(-1), sb1[k].reshape(-1)])), k
    print("[2^31] equal after two steps", flush=True)


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["adamw_q1d", "adamw_fp32", "came", "sgd_clip", "apollo"])
def test_hyperparameter_changes_take_effect(path):
    """group["lr"] and group["weight_decay"] changed between steps reach the next
    launch (no cached table or batch keeps the old ones): the run equals one that
    resumes from the step-2 checkpoint in a new optimizer built with the new values."""
    from adafactor8bit import Adafactor8Bit
    print(f"[hyper change] {path}", flush=True)
    kw = dict(PATHS[path], weight_decay=0.01)
    new = dict(lr=kw["lr"] * 0.37, weight_decay=0.05)
    pa = _params(SHAPES, 45)
    pb = _params(SHAPES, 45)
    oa = Adafactor8Bit(pa, **kw)
    ob = Adafactor8Bit(pb, **kw)
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _grads(ps, t, 45)
            o.step()
    for g in oa.param_groups:
        g.update(new)
    sd = ob.state_dict()
    oc = Adafactor8Bit(pb, **dict(kw, **new))
    oc.load_state_dict(sd)
    for g in oc.param_groups:   # a loaded checkpoint brings its own group options back
        g.update(new)
    for t in (3, 4):
        for ps, o in ((pa, oa), (pb, oc)):
            _grads(ps, t, 45)
            o.step()
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), f"{path}: param {i}"


@pytest.mark.gpu
def test_group_added_mid_run_steps_and_captures():
    """add_param_group after two steps: the new group starts its own count and state,
    the old group is unaffected, and once both have taken an eager step a capturable
    optimizer's step (both groups) is captured and replays bit-identically to eager
    steps of a twin."""
    from adafactor8bit import Adafactor8Bit
    print("[add_param_group]", flush=True)
    kw = dict(PATHS["adamw_q1d"], capturable=True)
    runs = []
    for _ in range(2):
        p0 = _params([(300, 200), (1000,)], 47)
        p1 = _params([(64, 96), (2048,)], 48)
        for p in p0 + p1:
            p.grad = torch.zeros_like(p)
        o = Adafactor8Bit(p0, **kw)
        for t in (1, 2):
            _fill(p0, t, 47)
            o.step()
        o.add_param_group({"params": p1, "lr": 5e-4})
        _fill(p0, 3, 47)
        _fill(p1, 3, 48)
        o.step()
        runs.append((p0, p1, o))
    (a0, a1, oa), (b0, b1, ob) = runs
    assert {oa.state[p]["step"] for p in a0} == {3} and {oa.state[p]["step"] for p in a1} == {1}
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _fill(a0, 4, 47)
        _fill(a1, 4, 48)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    for t in range(4, 7):
        _fill(a0, t, 47)
        _fill(a1, t, 48)
        graph.replay()
        _fill(b0, t, 47)
        _fill(b1, t, 48)
        ob.step()
        torch.cuda.synchronize()
        for a, b in zip(a0 + a1, b0 + b1):
            assert torch.equal(a, b), (t, tuple(a.shape))
    sd = oa.state_dict()["state"]
    assert sorted({s["step"] for s in sd.values()}) == [4, 6]


def _fill(ps, t, seed):
    for i, p in enumerate(ps):
        p.grad.copy_(make_grad(tuple(p.shape), i, t, seed, zero_frac=0.0).to(p.dtype))


def _flat_views(shapes, dtype, seed=None):
    """Views into one flat buffer, each starting one element past a 16-byte boundary
    (element offsets 1 mod 8: off for fp32 and for bf16), with gaps between them."""
    offs, o = [], 1
    for s in shapes:
        offs.append(o)
        o += (torch.Size(s).numel() + 7) // 8 * 8 + 8
    flat = torch.zeros(o, device="cuda", dtype=dtype)
    views = [flat[a:a + torch.Size(s).numel()].view(s) for a, s in zip(offs, shapes)]
    if seed is not None:
        for i, (v, s) in enumerate(zip(views, shapes)):
            v.copy_(make_param(s, i, seed).to(v.dtype))
    return flat, views


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16_sr"])
@pytest.mark.parametrize("path", sorted(PATHS))
def test_parameters_off_16_byte_boundaries(path, dtype):
    """Parameters and gradients that are views into flat buffers starting off a 16-byte
    boundary step exactly as aligned copies of them do; the results land in the flat
    parameter buffer and its gaps stay untouched."""
    from adafactor8bit import Adafactor8Bit
    print(f"[misaligned] {path} {dtype}", flush=True)
    kw = dict(PATHS[path], stochastic_round_writeback=dtype == torch.bfloat16)
    pflat, views = _flat_views(SHAPES, dtype, seed=49)
    gflat, gviews = _flat_views(SHAPES, dtype)
    pa = [torch.nn.Parameter(v) for v in views]
    assert all(p.data_ptr() % 16 for p in pa) and all(p.data_ptr() == v.data_ptr() for p, v in zip(pa, views))
    pb = _params(SHAPES, 49, dtype)
    oa, ob = Adafactor8Bit(pa, **kw), Adafactor8Bit(pb, **kw)
    for t in range(1, 4):
        for i, (p, gv) in enumerate(zip(pa, gviews)):
            gv.copy_(make_grad(tuple(p.shape), i, t, 49, zero_frac=0.0).to(dtype))
            p.grad = gv
        _grads(pb, t, 49)
        oa.step()
        ob.step()
    torch.cuda.synchronize()
    gaps = torch.ones_like(pflat, dtype=torch.bool)
    for i, (a, b, v) in enumerate(zip(pa, pb, views)):
        assert torch.equal(a, b) and torch.equal(v, b), f"{path}: param {i}"
        for k, s in oa.state[a].items():
            if torch.is_tensor(s):
                assert torch.equal(s, ob.state[b][k]), f"{path}: param {i} {k}"
        a0 = (v.data_ptr() - pflat.data_ptr()) // pflat.element_size()
        gaps[a0:a0 + v.numel()] = False
    assert not pflat[gaps].any(), "a write outside the parameters"


@pytest.mark.gpu
@pytest.mark.parametrize("path", ["adamw_q1d", "came", "sgd_clip", "apollo"])
def test_parameters_off_16_byte_boundaries_capture(path):
    """Misaligned bf16 views (parameters and gradients) in a capturable optimizer: the
    aligned copies are kept per parameter, so the step is captured and its replays
    equal eager steps of a twin on the same views."""
    from adafactor8bit import Adafactor8Bit
    print(f"[misaligned capture] {path}", flush=True)
    kw = dict(PATHS[path], stochastic_round_writeback=True, capturable=True)
    sets = []
    for _ in range(2):
        _, views = _flat_views(SHAPES, torch.bfloat16, seed=51)
        _, gviews = _flat_views(SHAPES, torch.bfloat16)
        ps = [torch.nn.Parameter(v) for v in views]
        for p, gv in zip(ps, gviews):
            p.grad = gv
        sets.append((ps, Adafactor8Bit(ps, **kw)))
    (pa, oa), (pb, ob) = sets
    for t in (1, 2):
        for ps, o in sets:
            _fill(ps, t, 51)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _fill(pa, 3, 51)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    for t in range(3, 7):
        _fill(pa, t, 51)
        graph.replay()
        _fill(pb, t, 51)
        ob.step()
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(zip(pa, pb)):
            assert torch.equal(a, b), (path, t, i)
            for k, s in oa.state[a].items():
                if torch.is_tensor(s):
                    assert torch.equal(s, ob.state[b][k]), (path, t, i, k)
