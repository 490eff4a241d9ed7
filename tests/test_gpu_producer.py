"""GPU parity of the producer of q, k, v (harp_amd.project_qkv: the q/k/v
projections, then QK-RMSNorm and RoPE; src/models/z_image/module/attn.py:69-89)
at the ring-attention headline shape [1, 8192, 3072] (24 heads) and at the
model's own width, 3840 = 30 heads x 128 (standalone_transformer.py:423-440).

Each stage is checked on its own inputs:
* the projections (library GEMMs) against the fp64 product of the same bf16
  hidden states and weights, within one bf16 rounding;
* the fused norm + RoPE of q and k against the CPU oracle
  (oracle/qk_norm_rope_oracle.py) applied to the GPU's own projection output,
  to the bar of tests/test_gpu_qk.py (two units of the pair magnitude on at
  most 0.5% of the elements);
* v passes through unchanged;
* the backward through QKNormRopeFn at the model width against the oracle."""

from types import SimpleNamespace

import numpy as np
import pytest
import torch

import harp_amd
from oracle import qk_norm_rope_oracle as qo
from tests.test_gpu_qk import assert_grad_close, assert_pairs_close, bits, freqs_cis

pytestmark = pytest.mark.gpu


def _module(dim, heads, seed):
    g = torch.Generator().manual_seed(seed)
    lin = []
    for _ in range(3):
        m = torch.nn.Linear(dim, dim, bias=False)
        with torch.no_grad():
            m.weight.copy_(torch.randn((dim, dim), generator=g) / dim ** 0.5)
        lin.append(m.to("cuda", torch.bfloat16))
    norms = []
    for _ in range(2):
        w = (1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).cuda()
        norms.append(SimpleNamespace(weight=w, eps=1e-6))
    return SimpleNamespace(heads=heads, to_q=lin[0], to_k=lin[1], to_v=lin[2], norm_q=norms[0], norm_k=norms[1])


def _check_projection(lin, hid, got):
    ref = hid.double() @ lin.weight.double().t()
    rel = ((got.double() - ref).norm() / ref.norm()).item()
    assert rel <= 4e-3, rel


@pytest.mark.parametrize("dim,heads,S", [(3072, 24, 8192), (3840, 30, 4096)])
def test_project_qkv_matches_oracle(dim, heads, S):
    print(f"[producer dim={dim} heads={heads} S={S}]", flush=True)
    attn = _module(dim, heads, seed=dim)
    g = torch.Generator().manual_seed(S)
    hid = torch.randn((1, S, dim), generator=g).to(torch.bfloat16).cuda()
    fc, f_np = freqs_cis(S, 128)
    with torch.no_grad():
        q, k, v = harp_amd.project_qkv(attn, hid, fc)
        q_lin = attn.to_q(hid)
        k_lin = attn.to_k(hid)
        v_lin = attn.to_v(hid)
    for lin, got in ((attn.to_q, q_lin), (attn.to_k, k_lin), (attn.to_v, v_lin)):
        _check_projection(lin, hid[0], got[0])
    assert torch.equal(v, v_lin.unflatten(-1, (heads, -1)).transpose(1, 2))
    for name, lin_out, out, norm in (("q", q_lin, q, attn.norm_q), ("k", k_lin, k, attn.norm_k)):
        x_bits = bits(lin_out.unflatten(-1, (heads, -1)).transpose(1, 2))
        want, _ = qo.norm_rope_forward(x_bits, bits(norm.weight), norm.eps, f_np)
        assert_pairs_close(bits(out), want, what=f"{name} norm+RoPE dim {dim}")


def test_norm_rope_backward_at_model_width():
    B, heads, S, D = 1, 30, 4096, 128
    g = torch.Generator().manual_seed(30)
    x = torch.randn((B, S, heads * D), generator=g).to(torch.bfloat16).cuda().unflatten(-1, (heads, -1)).transpose(1, 2)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    dy = torch.randn((B, S, heads * D), generator=g).to(torch.bfloat16).cuda().unflatten(-1, (heads, -1)).transpose(1, 2)
    fc, f_np = freqs_cis(S, D)
    xr = x.detach().clone().requires_grad_(True)
    wr = w.detach().clone().requires_grad_(True)
    y = harp_amd.QKNormRopeFn.apply(xr, wr, fc, 1e-6)
    y.backward(dy)
    want_y, want_rms = qo.norm_rope_forward(bits(x), bits(w), 1e-6, f_np)
    assert_pairs_close(bits(y), want_y, what="model-width fwd")
    want_dx, want_gw = qo.norm_rope_backward(bits(x), bits(dy), bits(w), want_rms, f_np)
    assert_grad_close(bits(xr.grad), want_dx, what="model-width bwd dx")
    gw = wr.grad.float().cpu().numpy()
    # grad_weight is bf16 here (the weight's dtype): one truncation of the sum
    np.testing.assert_allclose(gw, want_gw, rtol=2.0 ** -7, atol=1e-4 * np.abs(want_gw).max())
