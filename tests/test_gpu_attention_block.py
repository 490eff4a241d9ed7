"""GPU parity of the whole attention block (harp_amd.RingZAttention: q/k/v
projections, QK RMSNorm + RoPE, ring attention over sp_size chunks, output
projection; src/models/z_image/module/attn.py:51-105) against an fp64 CPU
restatement of the same block on the same bf16 parameters and inputs.

Bar (relative Frobenius error): output <= 2e-2, every gradient (hidden
states, the four projection weights, the two RMSNorm weights) <= 3e-2.  The
GPU path rounds to bf16 after each projection, the norm, RoPE and the
attention, so its error sits near 1e-2 of the fp64 result."""

import math

import pytest
import torch
from torch import nn

import harp_amd

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


class _Norm(nn.Module):
    def __init__(self, d, eps):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(d))


class _Attn(nn.Module):
    """The attribute set Z_Attention reads from the model's attention module
    (standalone_transformer.py:210-225)."""

    def __init__(self, dim, heads, d, qk_norm, eps=1e-5):
        super().__init__()
        self.heads = heads
        self.to_q = nn.Linear(dim, heads * d, bias=False)
        self.to_k = nn.Linear(dim, heads * d, bias=False)
        self.to_v = nn.Linear(dim, heads * d, bias=False)
        self.to_out = nn.ModuleList([nn.Linear(heads * d, dim, bias=False), nn.Identity()])
        self.norm_q = _Norm(d, eps) if qk_norm else None
        self.norm_k = _Norm(d, eps) if qk_norm else None


def _params(attn):
    names = ["to_q.weight", "to_k.weight", "to_v.weight", "to_out.0.weight"]
    if attn.norm_q is not None:
        names += ["norm_q.weight", "norm_k.weight"]
    return names


def _reference(p, x, freqs, heads, eps, rope):
    """fp64 restatement of the block: x @ W^T projections, RMSNorm
    x / sqrt(mean(x^2) + eps) * w, RoPE as complex multiplication, softmax
    attention with scale 1/sqrt(D), output projection."""
    B, S, _ = x.shape

    def split(t):
        return t.reshape(B, S, heads, -1).transpose(1, 2)  # [B, H, S, D]

    q, k, v = split(x @ p["to_q.weight"].T), split(x @ p["to_k.weight"].T), split(x @ p["to_v.weight"].T)
    if "norm_q.weight" in p:
        def norm(t, w):
            return t / torch.sqrt(t.pow(2).mean(-1, keepdim=True) + eps) * w

        q, k = norm(q, p["norm_q.weight"]), norm(k, p["norm_k.weight"])
    if rope:
        def rot(t):
            c = torch.view_as_complex(t.reshape(*t.shape[:-1], -1, 2).contiguous())
            return torch.view_as_real(c * freqs).flatten(-2)

        q, k = rot(q), rot(k)
    D = q.shape[-1]
    a = torch.softmax((q @ k.transpose(-1, -2)) / math.sqrt(D), dim=-1) @ v
    return a.transpose(1, 2).reshape(B, S, -1) @ p["to_out.0.weight"].T


def _rel(a, b):
    a = a.detach().double().cpu()
    return ((a - b).norm() / b.norm()).item()


@pytest.mark.parametrize("qk_norm,rope", [(True, True), (True, False), (False, True)])
def test_block_matches_fp64_reference(qk_norm, rope):
    B, S, dim, heads, D, sp = 1, 256, 192, 3, 64, 2
    eps = 1e-5
    torch.manual_seed(3407)
    attn = _Attn(dim, heads, D, qk_norm, eps)
    with torch.no_grad():
        for mod in (attn.norm_q, attn.norm_k):
            if mod is not None:
                mod.weight.copy_(1 + 0.2 * torch.randn(D))
    attn = attn.to(torch.bfloat16)
    x = torch.randn(B, S, dim).to(torch.bfloat16)
    dy = torch.randn(B, S, dim).to(torch.bfloat16)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(D // 2) / D))[None, :]
    freqs = torch.polar(torch.ones_like(ang), ang)  # complex128 [S, D/2]

    # GPU block on bf16 parameters
    gattn = _Attn(dim, heads, D, qk_norm, eps).to(torch.bfloat16)
    gattn.load_state_dict(attn.state_dict())
    gattn = gattn.to(DEV)
    block = harp_amd.RingZAttention(gattn, sp)
    xg = x.to(DEV).requires_grad_(True)
    yg = block(xg, freqs.to(torch.complex64).to(DEV) if rope else None, attn_mask=None)
    yg.backward(dy.to(DEV))
    torch.cuda.synchronize()

    # fp64 reference on the same bf16 values
    p = {n: t.detach().double().requires_grad_(True) for n, t in attn.state_dict().items() if n in _params(attn)}
    xr = x.double().requires_grad_(True)
    yr = _reference(p, xr, freqs, heads, eps, rope)
    yr.backward(dy.double())

    errs = {"out": _rel(yg, yr.detach()), "d_hidden": _rel(xg.grad, xr.grad)}
    gparams = dict(gattn.named_parameters())
    for n in _params(attn):
        errs["d_" + n] = _rel(gparams[n].grad, p[n].grad)
    print({k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["out"] <= 2e-2, errs
    assert max(v for k, v in errs.items() if k != "out") <= 3e-2, errs


def test_block_at_model_width():
    """The model's own width (standalone_transformer.py:423-440: dim 3840,
    30 heads x 128) over a 2048-token sequence in 2 ring chunks, with norm and
    RoPE; the fp64 reference runs on the GPU."""
    B, S, dim, heads, D, sp = 1, 2048, 3840, 30, 128, 2
    eps = 1e-5
    torch.manual_seed(30)
    attn = _Attn(dim, heads, D, True, eps)
    with torch.no_grad():
        for mod in (attn.norm_q, attn.norm_k):
            mod.weight.copy_(1 + 0.2 * torch.randn(D))
    attn = attn.to(torch.bfloat16)
    x = torch.randn(B, S, dim).to(torch.bfloat16)
    dy = torch.randn(B, S, dim).to(torch.bfloat16)
    ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(D // 2) / D))[None, :]
    freqs = torch.polar(torch.ones_like(ang), ang)

    gattn = _Attn(dim, heads, D, True, eps).to(torch.bfloat16)
    gattn.load_state_dict(attn.state_dict())
    gattn = gattn.to(DEV)
    xg = x.to(DEV).requires_grad_(True)
    yg = harp_amd.RingZAttention(gattn, sp)(xg, freqs.to(torch.complex64).to(DEV))
    yg.backward(dy.to(DEV))

    p = {n: t.detach().to(DEV).double().requires_grad_(True) for n, t in attn.state_dict().items()
         if n in _params(attn)}
    xr = x.to(DEV).double().requires_grad_(True)
    yr = _reference(p, xr, freqs.to(DEV), heads, eps, True)
    yr.backward(dy.to(DEV).double())
    torch.cuda.synchronize()

    def rel(a, b):
        return ((a.detach().double() - b.detach()).norm() / b.detach().norm()).item()

    errs = {"out": rel(yg, yr), "d_hidden": rel(xg.grad, xr.grad)}
    gparams = dict(gattn.named_parameters())
    for n in _params(attn):
        errs["d_" + n] = rel(gparams[n].grad, p[n].grad)
    print({k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    assert errs["out"] <= 2e-2, errs
    assert max(v for k, v in errs.items() if k != "out") <= 3e-2, errs


def test_block_rejects_a_sequence_not_split_into_chunks():
    attn = _Attn(64, 1, 64, True).to(torch.bfloat16).to(DEV)
    with pytest.raises(ValueError, match="multiple of sp_size"):
        harp_amd.RingZAttention(attn, 3)(torch.zeros(1, 64, 64, dtype=torch.bfloat16, device=DEV), None)
