"""A whole model's step captured in one HIP graph, for every preset.

build_param_groups puts a small Llama-shaped model (Hugging Face names: attention
and MLP projections, embedding, head, norm vectors) into the groups its preset
gives it -- factored and 1-D Adafactor, AdamW, RMSprop, CAME, SGD, APOLLO with its
full-rank fallback -- with the automatic quantisation profile (coded and fp32
states side by side).  One optimizer over all of them runs with capturable=True:
after two eager steps one step() is captured, and its replays must equal the
eager steps of a twin optimizer bit for bit, parameters and every state, across
APOLLO projection refreshes (apollo_update_proj_gap=3), for fp32 and for bf16
parameters with stochastic rounding.  The same model also shows that parameters
without a gradient take no step and leave the others' steps unchanged.
"""
import pytest
import torch
import torch.nn as nn

from inputs import make_grad, make_param

H, F, KV, V, L = 256, 512, 64, 1000, 2


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(H, H, bias=False)
        self.k_proj = nn.Linear(H, KV, bias=False)
        self.v_proj = nn.Linear(H, KV, bias=False)
        self.o_proj = nn.Linear(H, H, bias=False)


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(H, F, bias=False)
        self.up_proj = nn.Linear(H, F, bias=False)
        self.down_proj = nn.Linear(F, H, bias=False)


class _Norm(nn.Module):
    def __init__(self):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(H))


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Attn()
        self.mlp = _Mlp()
        self.input_layernorm = _Norm()
        self.post_attention_layernorm = _Norm()


class _Model(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(V, H)
        self.layers = nn.ModuleList([_Layer() for _ in range(L)])
        self.norm = _Norm()
        self.lm_head = nn.Linear(H, V, bias=False)


def _build(preset, capturable, dtype=torch.float32, grads=True):
    """The model in dtype (bf16: stochastic rounding on), its groups and the optimizer."""
    from adafactor8bit import Adafactor8Bit, build_param_groups
    model = _Model()
    with torch.no_grad():
        for i, p in enumerate(model.parameters()):
            p.copy_(make_param(tuple(p.shape), i, 37))
    model = model.to("cuda", dtype)
    params = list(model.parameters())
    if grads:
        for p in params:
            p.grad = torch.zeros_like(p)   # static gradient buffers: the graph reads these addresses
    over = {"apollo_update_proj_gap": 3} if preset == "apollo" else {}
    groups = build_param_groups(model, preset, **over)
    return params, Adafactor8Bit(groups, lr=1e-3, capturable=capturable,
                                 stochastic_round_writeback=dtype == torch.bfloat16)


def _load(params, t):
    for i, p in enumerate(params):
        p.grad.copy_(make_grad(tuple(p.shape), i, t, 37, zero_frac=0.0).to(p.dtype))


def _same(oa, ob, pa, pb, what):
    for i, (a, b) in enumerate(zip(pa, pb)):
        assert torch.equal(a, b), f"{what}: param {i} {tuple(a.shape)}"
        sa, sb = oa.state[a], ob.state[b]
        assert sorted(sa) == sorted(sb), (what, i)
        for k, v in sa.items():
            if torch.is_tensor(v):
                assert torch.equal(v, sb[k]), f"{what}: param {i} {k}"


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16_sr"])
@pytest.mark.parametrize("preset", ["adafactor", "adamw", "rmsprop", "came", "sgd", "apollo"])
def test_model_step_captured_for_every_preset(preset, dtype):
    print(f"[capture preset] {preset} {dtype}", flush=True)
    pa, oa = _build(preset, True, dtype)   # replayed
    pb, ob = _build(preset, True, dtype)   # eager
    routes = sorted({tuple(sorted((k, str(v)) for k, v in g.items() if k != "params")) for g in oa.param_groups})
    print(f"  {len(oa.param_groups)} groups, {len(routes)} distinct option sets", flush=True)
    for t in (1, 2):
        for ps, o in ((pa, oa), (pb, ob)):
            _load(ps, t)
            o.step()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _load(pa, 3)
        with torch.cuda.graph(graph):
            oa.step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    _same(oa, ob, pa, pb, f"{preset}: after capture (nothing ran)")
    for t in range(3, 9):
        _load(pa, t)
        graph.replay()
        _load(pb, t)
        ob.step()
        junk = torch.randn(1024, device="cuda").sum()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        _same(oa, ob, pa, pb, f"{preset}: step {t}")
    sd = oa.state_dict()
    assert {st["step"] for st in sd["state"].values()} == {8}


@pytest.mark.gpu
@pytest.mark.parametrize("preset", ["adafactor", "came", "apollo"])
def test_parameters_without_gradients_are_skipped(preset):
    """A parameter whose .grad is None takes no step: its value and state stay as
    they were, its step count included.  The others step exactly as in a run where
    every parameter has its gradient (each parameter's update depends only on its
    own state).  Here the layer-1 MLP has no gradient at steps 2 and 3."""
    print(f"[no grad] {preset}", flush=True)
    pa, oa = _build(preset, False, grads=False)   # layer-1 MLP skipped at steps 2, 3
    pb, ob = _build(preset, False, grads=False)   # every parameter, every step
    names = [n for n, _ in _Model().named_parameters()]
    skip = {i for i, n in enumerate(names) if n.startswith("layers.1.mlp.")}
    assert len(skip) == 3
    for t in range(1, 5):
        drop = t in (2, 3)
        for ps, d in ((pa, drop), (pb, False)):
            for i, p in enumerate(ps):
                p.grad = None if (d and i in skip) else make_grad(tuple(p.shape), i, t, 37, zero_frac=0.0).cuda()
        if drop:
            before = {i: (pa[i].detach().clone(), oa.state[pa[i]]["step"],
                          {k: v.clone() for k, v in oa.state[pa[i]].items() if torch.is_tensor(v)}) for i in skip}
        oa.step()
        ob.step()
        torch.cuda.synchronize()
        if drop:
            for i, (pv, stp, sv) in before.items():
                assert torch.equal(pa[i], pv), (t, i)
                assert oa.state[pa[i]]["step"] == stp, (t, i)
                for k, v in sv.items():
                    assert torch.equal(oa.state[pa[i]][k], v), (t, i, k)
    for i, (a, b) in enumerate(zip(pa, pb)):
        if i in skip:
            assert oa.state[a]["step"] == 2 and ob.state[b]["step"] == 4, i
            continue
        assert torch.equal(a, b), f"param {i} {names[i]}"
        for k, v in oa.state[a].items():
            if torch.is_tensor(v):
                assert torch.equal(v, ob.state[b][k]), (i, k)
