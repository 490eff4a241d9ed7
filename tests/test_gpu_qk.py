"""GPU parity of the QK-RMSNorm / RoPE kernels (kernels/libharp_ra.so through
torch.ops.async_op) against the CPU oracle (oracle/qk_norm_rope_oracle.py) on
the same bf16 inputs.

Bar: bf16 outputs agree with the oracle bit for bit except where a value sits
on a truncation boundary and the sum of squares or dot product (reduced in a
different order on the GPU, the reference and the oracle) moves it, on at
most 0.5% of the elements: RMSNorm forward at most one bf16 unit apart; after
RoPE at most two units of the complex pair's magnitude; RMSNorm gradients,
which cancel, at most one unit plus 2^-14 of the row's largest gradient.
RoPE alone has no reduction and must match exactly.  fp32 outputs (rms,
grad_weight) within 1e-5 relative (1e-4 for grad_weight summed over 196 608
rows).  The fused operators must equal the composition of the separate ones
on the GPU bit for bit."""

import math

import numpy as np
import pytest
import torch

import harp_amd
from oracle import qk_norm_rope_oracle as qo

pytestmark = pytest.mark.gpu

DEV = "cuda:0"


def ops():
    harp_amd.load_async_ops()
    return torch.ops.async_op


def bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def ordered(u: np.ndarray) -> np.ndarray:
    i = u.astype(np.int64)
    return np.where(i & 0x8000, -(i & 0x7FFF), i)


def assert_bf16_close(got_bits, want_bits, max_frac=5e-3, what=""):
    d = np.abs(ordered(got_bits) - ordered(want_bits))
    frac = float((d != 0).mean())
    print(f"{what}: {frac:.2e} of elements differ, max {int(d.max())} ulp", flush=True)
    assert d.max() <= 1, (what, int(d.max()))
    assert frac <= max_frac, (what, frac)


def assert_pairs_close(got_bits, want_bits, max_frac=5e-3, what=""):
    """For results that went through RoPE after a step that may differ by one
    unit (RMSNorm): a unit of the complex pair's magnitude moves each part by
    at most that much, plus the output truncation, so allow two units of the
    pair's larger part."""
    g = qo.bf16_to_f32(got_bits).astype(np.float64)
    w = qo.bf16_to_f32(want_bits).astype(np.float64)
    mag = np.maximum(np.abs(w[..., 0::2]), np.abs(w[..., 1::2]))
    unit = np.where(mag > 0, 2.0 ** (np.floor(np.log2(np.where(mag > 0, mag, 1.0))) - 7), 2.0 ** -133)
    unit = np.repeat(unit, 2, axis=-1)
    d = np.abs(g - w)
    frac = float((d != 0).mean())
    print(f"{what}: {frac:.2e} of elements differ, max {float((d / unit).max()):.2f} pair units", flush=True)
    assert np.all(d <= 2 * unit), what
    assert frac <= max_frac, (what, frac)


def assert_grad_close(got_bits, want_bits, max_frac=5e-3, what=""):
    """RMSNorm gradients: dx = (g - xn * coeff) / rms cancels in places, so a
    reduction-order difference in coeff (a few fp32 units of the row's dot
    product) moves a near-zero result by more than its own unit.  Allow one
    unit of the value plus 2^-14 of the row's largest gradient."""
    g = qo.bf16_to_f32(got_bits).astype(np.float64)
    w = qo.bf16_to_f32(want_bits).astype(np.float64)
    a = np.abs(w)
    unit = np.where(a > 0, 2.0 ** (np.floor(np.log2(np.where(a > 0, a, 1.0))) - 7), 0.0)
    tol = unit + 2.0 ** -14 * a.max(-1, keepdims=True)
    d = np.abs(g - w)
    frac = float((d != 0).mean())
    print(f"{what}: {frac:.2e} of elements differ, max {float((d / np.maximum(tol, 1e-30)).max()):.2f} of the bound",
          flush=True)
    assert np.all(d <= tol), what
    assert frac <= max_frac, (what, frac)


def make_x(B, H, S, D, layout, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    if layout == "token":  # [B, S, H, D] storage seen as [B, H, S, D]
        base = (torch.randn((B, S, H, D), generator=g) * scale).to(torch.bfloat16)
        dev = base.to(DEV).transpose(1, 2)
        host = base.transpose(1, 2).contiguous()
    else:
        host = (torch.randn((B, H, S, D), generator=g) * scale).to(torch.bfloat16)
        dev = host.to(DEV)
    return dev, bits(host)


def freqs_cis(S, D, batched_B=0):
    f = qo.rope_table(S, D)
    if batched_B:
        f = np.stack([qo.rope_table(S, D, offset=17 * b) for b in range(batched_B)])
    fc = torch.view_as_complex(torch.from_numpy(np.ascontiguousarray(f.reshape(*f.shape[:-1], D // 2, 2))))
    return fc.to(DEV), (f[:, None] if batched_B else f)


def make_w(D, kind, seed):
    if kind is None:
        return None, None
    g = torch.Generator().manual_seed(seed)
    w = 1.0 + 0.3 * torch.randn(D, generator=g)
    if kind == "bf16":
        wd = w.to(torch.bfloat16)
        return wd.to(DEV), bits(wd)
    return w.to(DEV), w.numpy().astype(np.float32)


CASES = [
    # B, H, S, D, layout, weight kind, batched freqs
    (1, 24, 512, 128, "token", "bf16", False),
    (2, 4, 300, 72, "head", "f32", True),
    (1, 3, 65, 64, "token", None, False),
    (1, 2, 33, 256, "head", "bf16", False),
]


@pytest.mark.parametrize("B,H,S,D,layout,wk,batched", CASES)
def test_separate_ops_match_oracle(B, H, S, D, layout, wk, batched):
    o = ops()
    x, xb = make_x(B, H, S, D, layout, seed=3407, scale=2.0)
    w, wb = make_w(D, wk, seed=1)
    fc, f_np = freqs_cis(S, D, B if batched else 0)
    eps = 1e-6
    wt = w if w is not None else torch.empty(0, device=DEV)

    y = torch.empty_like(x)
    rms = torch.empty(B * H * S, device=DEV, dtype=torch.float32)
    o.rmsnorm_forward_out(x, wt, y, rms, eps)
    want_y, want_rms = qo.rmsnorm_forward(xb, wb, eps)
    assert_bf16_close(bits(y), want_y, what="rmsnorm fwd")
    np.testing.assert_allclose(rms.cpu().numpy(), want_rms.reshape(-1), rtol=1e-6)

    r = torch.empty_like(x)
    o.rope_forward_impl(y, fc, r)
    np.testing.assert_array_equal(bits(r), qo.rope_forward(bits(y), f_np))

    dy, dyb = make_x(B, H, S, D, layout, seed=7)
    g1 = torch.empty_like(x)
    o.rope_backward_impl(dy, fc, g1)
    np.testing.assert_array_equal(bits(g1), qo.rope_backward(dyb, f_np))

    dx = torch.empty_like(x)
    gw = torch.empty(D, device=DEV, dtype=torch.float32) if wk is not None else torch.empty(0, device=DEV)
    o.rmsnorm_backward_out(x, g1, wt, rms, dx, gw)
    want_dx, want_gw = qo.rmsnorm_backward(xb, bits(g1), wb, rms.cpu().numpy().reshape(B, H, S))
    assert_grad_close(bits(dx), want_dx, what="rmsnorm bwd")
    if wk is not None:
        np.testing.assert_allclose(gw.cpu().numpy(), want_gw, rtol=1e-5, atol=1e-5 * np.abs(want_gw).max())


@pytest.mark.parametrize("B,H,S,D,layout,wk,batched", CASES)
def test_fused_ops_equal_the_composition(B, H, S, D, layout, wk, batched):
    o = ops()
    x, xb = make_x(B, H, S, D, layout, seed=11, scale=0.7)
    w, wb = make_w(D, wk, seed=2)
    wt = w if w is not None else torch.empty(0, device=DEV)
    fc, f_np = freqs_cis(S, D, B if batched else 0)
    eps = 1e-5
    y = torch.empty_like(x)
    rms = torch.empty(B * H * S, device=DEV, dtype=torch.float32)
    o.qk_norm_rope_forward(x, wt, fc, y, rms, eps)
    y1 = torch.empty_like(x)
    rms1 = torch.empty_like(rms)
    o.rmsnorm_forward_out(x, wt, y1, rms1, eps)
    y2 = torch.empty_like(x)
    o.rope_forward_impl(y1, fc, y2)
    np.testing.assert_array_equal(bits(y), bits(y2))
    assert torch.equal(rms, rms1)
    np.testing.assert_array_equal(bits(y), qo.rope_forward(bits(y1), f_np))
    want, _ = qo.norm_rope_forward(xb, wb, eps, f_np)
    assert_pairs_close(bits(y), want, what="fused fwd")

    dy, dyb = make_x(B, H, S, D, layout, seed=12)
    dx = torch.empty_like(x)
    gw = torch.empty(D, device=DEV, dtype=torch.bfloat16) if wk is not None else torch.empty(0, device=DEV)
    o.qk_norm_rope_backward(x, dy, wt, rms, fc, dx, gw)
    g1 = torch.empty_like(x)
    o.rope_backward_impl(dy, fc, g1)
    dx2 = torch.empty_like(x)
    gw2 = torch.empty_like(gw)
    o.rmsnorm_backward_out(x, g1, wt, rms, dx2, gw2)
    np.testing.assert_array_equal(bits(dx), bits(dx2))
    assert torch.equal(gw, gw2)
    want_dx, want_gw = qo.norm_rope_backward(xb, dyb, wb, rms.cpu().numpy().reshape(B, H, S), f_np)
    assert_grad_close(bits(dx), want_dx, what="fused bwd")
    if wk is not None:
        assert_bf16_close(bits(gw), qo.f32_to_bf16_trunc(want_gw), max_frac=0.05, what="grad_weight bf16")


@pytest.mark.parametrize("D", [8, 16, 24, 40, 72, 120, 136, 200, 248])
def test_head_dim_sweep(D):
    """Every head dim class of the kernels: one 16-byte chunk per lane, a
    partial first chunk set (D < 128), and a partial second one (D > 128)."""
    B, H, S = 1, 3, 40
    o = ops()
    x, xb = make_x(B, H, S, D, "token", seed=D, scale=1.5)
    w, wb = make_w(D, "f32", seed=D + 1)
    fc, f_np = freqs_cis(S, D)
    eps = 1e-6
    y = torch.empty_like(x)
    rms = torch.empty(B * H * S, device=DEV, dtype=torch.float32)
    o.qk_norm_rope_forward(x, w, fc, y, rms, eps)
    want, want_rms = qo.norm_rope_forward(xb, wb, eps, f_np)
    assert_pairs_close(bits(y), want, what=f"D={D} fused fwd")
    np.testing.assert_allclose(rms.cpu().numpy(), want_rms.reshape(-1), rtol=1e-6)
    dy, dyb = make_x(B, H, S, D, "token", seed=D + 2)
    dx = torch.empty_like(x)
    gw = torch.empty(D, device=DEV, dtype=torch.float32)
    o.qk_norm_rope_backward(x, dy, w, rms, fc, dx, gw)
    want_dx, want_gw = qo.norm_rope_backward(xb, dyb, wb, rms.cpu().numpy().reshape(B, H, S), f_np)
    assert_grad_close(bits(dx), want_dx, what=f"D={D} fused bwd")
    np.testing.assert_allclose(gw.cpu().numpy(), want_gw, rtol=1e-5, atol=1e-5 * np.abs(want_gw).max())


def test_in_place_and_head_major_output():
    o = ops()
    B, H, S, D = 1, 6, 130, 128
    x, xb = make_x(B, H, S, D, "token", seed=5)
    w, wb = make_w(D, "bf16", seed=6)
    fc, f_np = freqs_cis(S, D)
    rms = torch.empty(B * H * S, device=DEV, dtype=torch.float32)
    out = torch.empty((B, H, S, D), device=DEV, dtype=torch.bfloat16)  # head-major output of a token-major input
    o.qk_norm_rope_forward(x, w, fc, out, rms, 1e-6)
    want, _ = qo.norm_rope_forward(xb, wb, 1e-6, f_np)
    assert_pairs_close(bits(out), want, what="head-major out")
    o.qk_norm_rope_forward(x, w, fc, x, rms, 1e-6)  # in place
    np.testing.assert_array_equal(bits(x), bits(out))


def test_autograd_functions_match_oracle():
    B, H, S, D = 1, 4, 96, 128
    x, xb = make_x(B, H, S, D, "token", seed=21)
    w, wb = make_w(D, "bf16", seed=22)
    fc, f_np = freqs_cis(S, D)
    xg = x.detach().clone().requires_grad_(True)
    wg = w.detach().clone().requires_grad_(True)
    y = harp_amd.QKNormRopeFn.apply(xg, wg, fc, 1e-6)
    dy, dyb = make_x(B, H, S, D, "token", seed=23)
    y.backward(dy)
    want_y, want_rms = qo.norm_rope_forward(xb, wb, 1e-6, f_np)
    assert_pairs_close(bits(y), want_y, what="QKNormRopeFn fwd")
    want_dx, want_gw = qo.norm_rope_backward(xb, dyb, wb, want_rms, f_np)
    assert_grad_close(bits(xg.grad), want_dx, what="QKNormRopeFn dx")
    assert_bf16_close(bits(wg.grad), qo.f32_to_bf16_trunc(want_gw), max_frac=0.05, what="QKNormRopeFn dw")
    # the separate Functions in the model's order give the same gradients
    xs = x.detach().clone().requires_grad_(True)
    ws = w.detach().clone().requires_grad_(True)
    ys = harp_amd.ApplyRotaryComplexFn.apply(harp_amd.RMSNormFn.apply(xs, ws, 1e-6), fc)
    ys.backward(dy)
    assert torch.equal(ys, y) and torch.equal(xs.grad, xg.grad) and torch.equal(ws.grad, wg.grad)


def test_config4_shape_full_size():
    """Q at the ring-attention headline shape (B1 H24 S8192 D128, token-major)."""
    o = ops()
    B, H, S, D = 1, 24, 8192, 128
    x, xb = make_x(B, H, S, D, "token", seed=3407)
    w, wb = make_w(D, "bf16", seed=3)
    fc, f_np = freqs_cis(S, D)
    y = torch.empty_like(x)
    rms = torch.empty(B * H * S, device=DEV, dtype=torch.float32)
    o.qk_norm_rope_forward(x, w, fc, y, rms, 1e-6)
    want, want_rms = qo.norm_rope_forward(xb, wb, 1e-6, f_np)
    assert_pairs_close(bits(y), want, what="config-4 fused fwd")
    dy, dyb = make_x(B, H, S, D, "token", seed=4)
    dx = torch.empty_like(x)
    gw = torch.empty(D, device=DEV, dtype=torch.float32)
    o.qk_norm_rope_backward(x, dy, w, rms, fc, dx, gw)
    want_dx, want_gw = qo.norm_rope_backward(xb, dyb, wb, rms.cpu().numpy().reshape(B, H, S), f_np)
    assert_grad_close(bits(dx), want_dx, what="config-4 fused bwd")
    np.testing.assert_allclose(gw.cpu().numpy(), want_gw, rtol=1e-4, atol=1e-5 * np.abs(want_gw).max())
    # invariant: without the weight, RMSNorm rows have unit rms and RoPE keeps
    # pair norms; each of the two truncations toward zero shrinks a value by
    # less than 2^-7 of itself
    o.qk_norm_rope_forward(x, torch.empty(0, device=DEV), fc, y, rms, 0.0)
    r = torch.sqrt(y.float().pow(2).mean(-1))
    assert (r - 1).min().item() > -2 * 2.0 ** -7 and (r - 1).max().item() < 1e-3
    assert math.isfinite(float(gw.abs().sum()))
