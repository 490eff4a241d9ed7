"""GPU parity of the fused q/k/v producer (harp_amd.qkv: the kernel of
harp_amd/csrc/proj_kernels.hip through the C ABI harp_qkv_project), the
projections + QK RMSNorm + RoPE of src/models/z_image/module/attn.py:69-89
in one launch.

* The bf16 products the kernel keeps for the backward (y_lin) and the plain
  projection v: against the fp64 product of the same bf16 inputs (on the
  GPU), elementwise within one bf16 rounding (to nearest) plus an fp32
  accumulation term.
* The normalised and rotated q, k: against the CPU oracle
  (oracle/qk_norm_rope_oracle.py) applied to the kernel's own products, to
  the bar of tests/test_gpu_qk.py (two units of the pair magnitude, on at
  most 0.5% of the elements), and the rms within 1e-5 relative; and against
  the separate norm + RoPE kernel applied to the same products, to the same
  bar (the sum of squares is reduced in another order).
* ProjectQKVFn's gradients: against the unfused autograd path (torch Linear
  and QKNormRopeFn) on the same inputs.
Shapes: the headline producer [1, 8192, 3072] (24 heads), the model's width
[1, 4096, 3840] (30 heads), and small ones covering 1 to 5 k-tiles (the
kernel's loop is unrolled over three stages), token counts that are not a
multiple of the 256-token tile, batches with per-batch RoPE tables, fp32
norm weights, plain projections and RMSNorm without RoPE."""

import math

import numpy as np
import pytest
import torch

from harp_amd import qkv
from harp_amd.attention import project_qkv
from oracle import qk_norm_rope_oracle as qo
from tests.test_gpu_qk import assert_pairs_close, bits, freqs_cis, ops

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def _inputs(B, S, dim, heads, nw_kind, rope, batched, seed):
    g = torch.Generator().manual_seed(seed)
    n_out = heads * 128
    x = torch.randn((B, S, dim), generator=g).to(torch.bfloat16).to(DEV)
    ws = [(torch.randn((n_out, dim), generator=g) / math.sqrt(dim)).to(torch.bfloat16).to(DEV) for _ in range(3)]
    norms = []
    for _ in range(2):
        if nw_kind is None:
            norms.append((None, 0.0))
            continue
        w = 1.0 + 0.2 * torch.randn(128, generator=g)
        w = w.to(torch.bfloat16) if nw_kind == "bf16" else w
        norms.append((w.to(DEV), 1e-6))
    fc, f_np = freqs_cis(S, 128, batched_B=B if batched else 0) if rope else (None, None)
    return x, ws, norms, fc, f_np


def _check_product(x, w, got, what):
    """got [B, S, n_out] (or a [B, H, S, 128] view of it) against the fp64
    product, elementwise."""
    M = x.shape[0] * x.shape[1]
    xd = x.reshape(M, -1).double()
    wd = w.double()
    ref = xd @ wd.t()
    bound = 2.0 ** -8 * ref.abs() + 1e-5 * (xd.abs() @ wd.abs().t())
    got2 = got.transpose(1, 2).reshape(M, -1) if got.dim() == 4 else got.reshape(M, -1)
    err = (got2.double() - ref).abs()
    rel = (err.norm() / ref.norm()).item()
    print(f"{what}: rel {rel:.2e}, max err / bound {(err / bound).max().item():.3f}", flush=True)
    assert bool((err <= bound).all()), what
    assert rel <= 4e-3, (what, rel)
    del ref, bound, err


CASES = [
    # B, S, dim, heads, norm weight, rope, batched freqs
    (1, 8192, 3072, 24, "bf16", True, False),   # headline producer: 48 k-tiles
    (1, 4096, 3840, 30, "bf16", True, False),   # model width: 60 k-tiles
    (2, 300, 192, 2, "f32", True, True),        # 3 k-tiles, 600 tokens (ragged last tile)
    (1, 77, 64, 1, "bf16", True, False),        # 1 k-tile, one partial token tile
    (3, 100, 128, 3, "bf16", True, True),       # 2 k-tiles, batched RoPE table
    (1, 513, 256, 2, "f32", True, False),       # 4 k-tiles
    (1, 256, 320, 1, "bf16", True, False),      # 5 k-tiles
    (1, 300, 256, 2, "bf16", False, False),     # RMSNorm without RoPE
    (2, 200, 128, 2, None, False, False),       # three plain projections
]


@pytest.mark.parametrize("B,S,dim,heads,nwk,rope,batched", CASES)
def test_fused_producer_matches_oracle(B, S, dim, heads, nwk, rope, batched):
    print(f"[qkv B={B} S={S} dim={dim} heads={heads} norm={nwk} rope={rope}]", flush=True)
    x, ws, norms, fc, f_np = _inputs(B, S, dim, heads, nwk, rope, batched, seed=dim + S)
    (q, k, v), lins, rmss = qkv.qkv_project(x, ws, norms + [(None, 0.0)], fc, keep_for_backward=True)
    torch.cuda.synchronize()
    assert q.shape == (B, heads, S, 128) and q.stride() == (S * heads * 128, 128, heads * 128, 1)
    _check_product(x, ws[2], v, "v")
    for name, out, lin, rms, (nw, eps), w in (("q", q, lins[0], rmss[0], norms[0], ws[0]),
                                            ("k", k, lins[1], rmss[1], norms[1], ws[1])):
        if nw is None:
            assert lin is None and rms is None
            _check_product(x, w, out, name)
            continue
        _check_product(x, w, lin, f"{name} product")
        lin4 = lin.unflatten(-1, (heads, 128)).transpose(1, 2)
        w_ref = bits(nw) if nw.dtype == torch.bfloat16 else nw.cpu().numpy().astype(np.float32)
        if rope:
            want, want_rms = qo.norm_rope_forward(bits(lin4), w_ref, eps, f_np)
        else:
            want, want_rms = qo.rmsnorm_forward(bits(lin4), w_ref, eps)
        assert_pairs_close(bits(out), want, what=f"{name} vs oracle")
        np.testing.assert_allclose(rms.cpu().numpy().reshape(want_rms.shape), want_rms, rtol=1e-5)
        # the separate kernel on the same products
        sep = torch.empty_like(out)
        sep_rms = torch.empty_like(rms)
        if rope:
            ops().qk_norm_rope_forward(lin4, nw, fc, sep, sep_rms, eps)
        else:
            ops().rmsnorm_forward_out(lin4, nw, sep, sep_rms, eps)
        assert_pairs_close(bits(out), bits(sep), what=f"{name} vs separate kernel")


@pytest.mark.parametrize("S,heads,n_outs", [(140 * 256 - 50, 2, 2), (90 * 256 - 200, 3, 3)])
def test_tail_launch_matches_oracle(S, heads, n_outs):
    """Shapes whose work units fill at most half of the CUs' last round: the
    launcher runs those units as 128-token halves in a second launch.  The
    tail then covers the last output's final units, including the partial
    last token tile (and, with 3 heads, the half-empty last head pair)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    units = n_outs * ((heads + 1) // 2) * math.ceil(S / 256)
    r = units % cus
    assert units > cus and 0 < r <= cus // 2, (units, cus)  # the case under test
    print(f"[qkv tail S={S} heads={heads} outs={n_outs}: {r} units in the tail launch]", flush=True)
    x, ws, norms, fc, f_np = _inputs(1, S, 128, heads, "bf16", True, False, seed=S)
    norms = norms + [(None, 0.0)]
    outs, lins, rmss = qkv.qkv_project(x, ws[:n_outs], norms[:n_outs], fc, keep_for_backward=True)
    torch.cuda.synchronize()
    for i in range(n_outs):
        nw, eps = norms[i]
        if nw is None:
            _check_product(x, ws[i], outs[i], f"out {i}")
            continue
        _check_product(x, ws[i], lins[i], f"out {i} product")
        lin4 = lins[i].unflatten(-1, (heads, 128)).transpose(1, 2)
        want, want_rms = qo.norm_rope_forward(bits(lin4), bits(nw), eps, f_np)
        assert_pairs_close(bits(outs[i]), want, what=f"out {i} vs oracle")
        np.testing.assert_allclose(rmss[i].cpu().numpy().reshape(want_rms.shape), want_rms, rtol=1e-5)


def _module(dim, heads, seed, bias=False):
    from types import SimpleNamespace

    g = torch.Generator().manual_seed(seed)
    lin = []
    for _ in range(3):
        m = torch.nn.Linear(dim, heads * 128, bias=bias)
        with torch.no_grad():
            m.weight.copy_(torch.randn((heads * 128, dim), generator=g) / dim ** 0.5)
        lin.append(m.to(DEV, torch.bfloat16))
    norms = []
    for _ in range(2):
        w = torch.nn.Parameter((1 + 0.1 * torch.randn(128, generator=g)).to(torch.bfloat16).to(DEV))
        norms.append(SimpleNamespace(weight=w, eps=1e-6))
    return SimpleNamespace(heads=heads, to_q=lin[0], to_k=lin[1], to_v=lin[2], norm_q=norms[0], norm_k=norms[1])


def test_project_qkv_takes_the_fused_path_only_where_it_applies():
    attn = _module(256, 2, seed=1)
    x = torch.randn((1, 64, 256)).to(torch.bfloat16).to(DEV)
    fc, _ = freqs_cis(64, 128)
    assert qkv.fused_supported(attn, x, fc)
    assert not qkv.fused_supported(attn, x.cpu(), fc)
    assert not qkv.fused_supported(_module(256, 2, seed=1, bias=True), x, fc)
    assert not qkv.fused_supported(attn, x[..., :200].contiguous(), fc)  # dim not a multiple of 64
    with torch.no_grad():
        fused = project_qkv(attn, x, fc)
        unfused = project_qkv(attn, x, fc, fused=False)
    assert all(t.grad_fn is None for t in fused)  # no gradient possible: the kernel alone
    for a, b, name in zip(fused, unfused, "qkv"):
        rel = ((a.double() - b.double()).norm() / b.double().norm()).item()
        assert rel <= 4e-3, (name, rel)
    q, k, v = project_qkv(attn, x, fc)  # weights require grad: the autograd Function
    assert all(t.grad_fn is not None for t in (q, k, v))
    assert torch.equal(q, fused[0]) and torch.equal(k, fused[1]) and torch.equal(v, fused[2])


@pytest.mark.parametrize("B,S,dim,heads,rope", [(2, 256, 256, 2, True), (1, 300, 192, 3, False)])
def test_fused_backward_matches_unfused_autograd(B, S, dim, heads, rope):
    attn = _module(dim, heads, seed=dim)
    g = torch.Generator().manual_seed(S)
    x0 = torch.randn((B, S, dim), generator=g).to(torch.bfloat16).to(DEV)
    fc = freqs_cis(S, 128, batched_B=B if B > 1 else 0)[0] if rope else None
    ups = [torch.randn((B, heads, S, 128), generator=g).to(torch.bfloat16).to(DEV) for _ in range(3)]
    params = [attn.to_q.weight, attn.to_k.weight, attn.to_v.weight, attn.norm_q.weight, attn.norm_k.weight]
    grads = {}
    for fused in (True, False):
        x = x0.detach().clone().requires_grad_(True)
        for p in params:
            p.grad = None
        q, k, v = project_qkv(attn, x, fc, fused=fused)
        loss = sum((t.float() * u.float()).sum() for t, u in zip((q, k, v), ups))
        loss.backward()
        grads[fused] = [x.grad.detach().clone()] + [p.grad.detach().clone() for p in params]
    names = ["hidden", "wq", "wk", "wv", "norm_q", "norm_k"]
    for name, a, b in zip(names, grads[True], grads[False]):
        rel = ((a.double() - b.double()).norm() / b.double().norm()).item()
        print(f"grad {name}: rel {rel:.2e}", flush=True)
        assert rel <= 1e-2, (name, rel)


def test_qkv_project_refuses_mismatched_weights():
    """Shapes the kernel cannot check (a weight's row count, the norm
    weight's length) are refused on the host before any launch."""
    x = torch.zeros((1, 64, 128), dtype=torch.bfloat16, device=DEV)
    w = torch.zeros((256, 128), dtype=torch.bfloat16, device=DEV)
    nw = torch.ones(128, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError, match="every weight"):
        qkv.qkv_project(x, [w, w, w[:128]], [(nw, 1e-6), (nw, 1e-6), (None, 0.0)], None)
    with pytest.raises(ValueError, match="every weight"):
        qkv.qkv_project(x, [w, w.float(), w], [(nw, 1e-6), (nw, 1e-6), (None, 0.0)], None)
    with pytest.raises(ValueError, match="RMSNorm weights"):
        qkv.qkv_project(x, [w, w, w], [(nw[:64], 1e-6), (nw, 1e-6), (None, 0.0)], None)
    with pytest.raises(ValueError, match="multiple of 64"):
        qkv.qkv_project(x[..., :96].contiguous(), [w[:, :96].contiguous()] * 3, [(None, 0.0)] * 3, None)
