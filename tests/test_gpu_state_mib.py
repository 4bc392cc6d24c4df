"""The README's APOLLO 'State' figure for TinyLlama-1.1B (README.md:77: UF8 M, AL8 V, B_V 2048,
756.3 MiB of optimizer-owned tensors), on the GPU.

The other rows of that table are pinned on the CPU (tests/test_oracle_codecs.py): their state
exists once the group is initialised.  APOLLO's low-rank slots and its cached projection P^T
are created by the first step (their shapes depend on the matrix side), so this row needs a
step.  The model is TinyLlama-1.1B's parameter set under Hugging Face's names (so the apollo
preset's targets "attn" and "mlp" find the projections; embeddings, the head and the norms
take the preset's full-rank fallback), grouped by build_param_groups(model, "apollo", "G0")
as the README's G0 row was.  What the figure fixes: rank-256 low-rank UF8/AL8 codes and block
metadata for the 154 attention / MLP matrices, their fp32 P^T (K x 256 each, cached), full-rank
UF8/AL8 state for the embedding and head, and fp32 state for the 45 norm vectors.
"""
import pytest
import torch
import torch.nn as nn

H, F, KV, V, L = 2048, 5632, 256, 32000, 22


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj = nn.Linear(H, H, bias=False, device="meta")
        self.k_proj = nn.Linear(H, KV, bias=False, device="meta")
        self.v_proj = nn.Linear(H, KV, bias=False, device="meta")
        self.o_proj = nn.Linear(H, H, bias=False, device="meta")


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj = nn.Linear(H, F, bias=False, device="meta")
        self.up_proj = nn.Linear(H, F, bias=False, device="meta")
        self.down_proj = nn.Linear(F, H, bias=False, device="meta")


class _Norm(nn.Module):
    def __init__(self):
        super().__init__()
        self.weight = nn.Parameter(torch.empty(H, device="meta"))


class _Layer(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn = _Attn()
        self.mlp = _Mlp()
        self.input_layernorm = _Norm()
        self.post_attention_layernorm = _Norm()


class _TinyLlama(nn.Module):
    def __init__(self):
        super().__init__()
        self.embed_tokens = nn.Embedding(V, H, device="meta")
        self.layers = nn.ModuleList([_Layer() for _ in range(L)])
        self.norm = _Norm()
        self.lm_head = nn.Linear(H, V, bias=False, device="meta")


@pytest.mark.gpu
def test_apollo_state_mib_matches_readme():
    from adafactor8bit import Adafactor8Bit, build_param_groups
    from adafactor8bit import _state as S
    print("[state MiB] APOLLO TinyLlama-1.1B, apollo preset, G0", flush=True)
    model = _TinyLlama().to_empty(device="cuda")
    params = list(model.parameters())
    assert sum(p.numel() for p in params) == 1_100_048_384
    with torch.no_grad():
        for p in params:
            p.fill_(0.01)
            p.grad = torch.full_like(p, 1e-3)
    groups = build_param_groups(model, "apollo", "G0")
    opt = Adafactor8Bit(groups)
    opt.step()
    torch.cuda.synchronize()
    routes = {}
    for p in params:
        st = opt.state[p]
        routes["apollo" if "apollo_seed" in st else "full"] = routes.get(
            "apollo" if "apollo_seed" in st else "full", 0) + 1
    mib = sum(S.state_bytes(opt.state[p]) for p in params) / 2 ** 20
    print(f"  routes {routes}, state {mib:.2f} MiB", flush=True)
    assert routes == {"apollo": 7 * L, "full": 2 * L + 3}
    assert round(mib, 1) == 756.3
