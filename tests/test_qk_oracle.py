"""Pins the QK-RMSNorm / RoPE oracle (oracle/qk_norm_rope_oracle.py) to
closed forms, library routines and invariants, independently of the oracle's
own formulas, and shows that plausible mistakes in copies of the math fail
the same checks (CPU only)."""

import numpy as np
import pytest
import torch

from oracle import qk_norm_rope_oracle as qo

RNG = np.random.default_rng(3407)


def bf16_input(shape, scale=1.0):
    return qo.f32_to_bf16_rne((RNG.standard_normal(shape) * scale).astype(np.float32))


def f64(u16):
    return qo.bf16_to_f32(u16).astype(np.float64)


def ulp_bound(ref):
    """Truncation to bf16 removes less than one unit of the 8-bit mantissa."""
    a = np.abs(ref)
    return np.where(a > 0, 2.0 ** (np.floor(np.log2(np.where(a > 0, a, 1.0))) - 7), 0.0)


def torch_rmsnorm64(x, w, eps):
    """The model's RMSNorm (standalone_transformer.py:141-153) in float64."""
    xt = torch.from_numpy(x)
    var = xt.pow(2).mean(-1, keepdim=True)
    return (xt * torch.rsqrt(var + eps) * torch.from_numpy(w)).numpy()


@pytest.mark.parametrize("D", [64, 72, 128])
def test_rmsnorm_forward_matches_fp64_formula_within_truncation(D):
    x = bf16_input((3, 5, 17, D), 2.0)
    w = bf16_input((D,), 0.5)
    out, rms = qo.rmsnorm_forward(x, w, 1e-6)
    ref = torch_rmsnorm64(f64(x), f64(w), 1e-6)
    got = f64(out)
    # truncation: |got| <= |ref| (toward zero), gap < 1 ulp plus fp32 noise
    slack = 4e-7 * np.abs(ref) + 1e-30
    assert np.all(np.abs(got) <= np.abs(ref) + slack)
    assert np.all(np.abs(ref) - np.abs(got) <= ulp_bound(ref) + slack)
    assert np.all((got == 0) | (np.sign(got) == np.sign(ref)))
    np.testing.assert_allclose(rms, np.sqrt((f64(x) ** 2).mean(-1) + 1e-6), rtol=2e-7)


def test_rmsnorm_output_has_unit_rms_without_weight():
    x = bf16_input((4, 3, 64, 128), 3.0)
    out, _ = qo.rmsnorm_forward(x, None, 0.0)
    r = np.sqrt((f64(out) ** 2).mean(-1))
    assert np.all(np.abs(r - 1.0) < 8e-3)  # truncation biases toward zero by < 2^-7


def test_rmsnorm_backward_matches_autograd():
    D = 128
    x = bf16_input((2, 3, 9, D))
    w = bf16_input((D,), 0.7)
    dy = bf16_input((2, 3, 9, D))
    _, rms = qo.rmsnorm_forward(x, w, 1e-5)
    dx, gw = qo.rmsnorm_backward(x, dy, w, rms)
    xt = torch.from_numpy(f64(x)).requires_grad_(True)
    wt = torch.from_numpy(f64(w)).requires_grad_(True)
    y = xt * torch.rsqrt(xt.pow(2).mean(-1, keepdim=True) + 1e-5) * wt
    y.backward(torch.from_numpy(f64(dy)))
    ref = xt.grad.numpy()
    assert np.all(np.abs(f64(dx) - ref) <= ulp_bound(ref) + 1e-5 * np.abs(ref).max())
    np.testing.assert_allclose(gw, wt.grad.numpy(), rtol=2e-5, atol=1e-5)


def complex_rope64(x, f, conj=False):
    xc = torch.view_as_complex(torch.from_numpy(np.ascontiguousarray(x.reshape(*x.shape[:-1], -1, 2))))
    fb = np.broadcast_to(f, x.shape)
    fc = torch.view_as_complex(torch.from_numpy(np.ascontiguousarray(fb.reshape(*fb.shape[:-1], -1, 2))))
    if conj:
        fc = fc.conj()
    return torch.view_as_real(xc * fc).reshape(x.shape).numpy()


@pytest.mark.parametrize("D", [64, 72, 128])
def test_rope_matches_complex_multiplication(D):
    x = bf16_input((2, 4, 33, D), 1.5)
    f32 = qo.rope_table(33, D)
    f = f32.astype(np.float64)  # the same fp32 table, exactly
    # the oracle rounds one product to fp32 before its fused add: an absolute
    # error below 2^-23 of the row's largest input, on top of truncation
    slack = 2.0 ** -23 * np.abs(f64(x)).max(-1, keepdims=True)
    ref = complex_rope64(f64(x), f)
    got = f64(qo.rope_forward(x, f32))
    assert np.all(np.abs(got) <= np.abs(ref) + slack)
    assert np.all(np.abs(ref) - np.abs(got) <= ulp_bound(ref) + slack)
    assert np.all((got == 0) | (np.sign(got) == np.sign(ref)) | (np.abs(ref) <= slack))
    refb = complex_rope64(f64(x), f, conj=True)
    gotb = f64(qo.rope_backward(x, f32))
    assert np.all(np.abs(gotb) <= np.abs(refb) + slack)
    assert np.all(np.abs(refb) - np.abs(gotb) <= ulp_bound(refb) + slack)


def test_rope_preserves_pair_norms_and_backward_undoes_forward():
    D = 128
    x = bf16_input((3, 2, 40, D))
    f = qo.rope_table(40, D)
    y = qo.rope_forward(x, f)
    nx = np.hypot(f64(x)[..., 0::2], f64(x)[..., 1::2])
    ny = np.hypot(f64(y)[..., 0::2], f64(y)[..., 1::2])
    assert np.all(np.abs(nx - ny) <= 2 * 2.0 ** -7 * nx + 1e-6)
    z = qo.rope_backward(y, f)
    assert np.abs(f64(z) - f64(x)).max() <= 4 * 2.0 ** -7 * np.abs(f64(x)).max()


def test_rope_backward_is_the_adjoint():
    D = 64
    x = bf16_input((1, 2, 11, D))
    dy = bf16_input((1, 2, 11, D))
    f = qo.rope_table(11, D)
    xt = torch.from_numpy(f64(x)).requires_grad_(True)
    xc = torch.view_as_complex(xt.reshape(1, 2, 11, D // 2, 2))
    fc = torch.view_as_complex(torch.from_numpy(f.astype(np.float64).reshape(11, D // 2, 2)))
    torch.view_as_real(xc * fc).reshape(1, 2, 11, D).backward(torch.from_numpy(f64(dy)))
    ref = xt.grad.numpy()
    got = f64(qo.rope_backward(dy, f))
    slack = 2.0 ** -23 * np.abs(f64(dy)).max(-1, keepdims=True)
    assert np.all(np.abs(got) <= np.abs(ref) + slack)
    assert np.all(np.abs(ref) - np.abs(got) <= ulp_bound(ref) + slack)


def test_batched_freqs_broadcast():
    D = 64
    x = bf16_input((2, 3, 5, D))
    f = np.stack([qo.rope_table(5, D), qo.rope_table(5, D, offset=7)])  # [B, S, D]
    got = qo.rope_forward(x, f[:, None])
    for b in range(2):
        np.testing.assert_array_equal(got[b], qo.rope_forward(x[b], f[b]))


def test_planted_mistakes_fail_the_checks():
    D = 128
    x = bf16_input((2, 3, 7, D), 2.0)
    w = bf16_input((D,), 0.5)
    ref = torch_rmsnorm64(f64(x), f64(w), 1e-6)
    # sum instead of mean in the variance
    xf = f64(x)
    wrong = xf / np.sqrt((xf ** 2).sum(-1, keepdims=True) + 1e-6) * f64(w)
    assert np.abs(wrong - ref).max() > 10 * ulp_bound(ref).max()
    # RoPE with the conjugate dropped from the backward, or the pair order rotated
    f = qo.rope_table(7, D)
    refb = complex_rope64(xf, f.astype(np.float64), conj=True)
    wrong_b = f64(qo.rope_forward(x, f))
    assert np.abs(wrong_b - refb).max() > 0.1
    fr = f.copy()
    fr[..., 0::2], fr[..., 1::2] = f[..., 1::2], f[..., 0::2]
    assert np.abs(f64(qo.rope_forward(x, fr)) - complex_rope64(xf, f.astype(np.float64))).max() > 0.1


def test_fused_equals_the_two_operators():
    D = 128
    x = bf16_input((1, 4, 19, D))
    w = bf16_input((D,))
    f = qo.rope_table(19, D)
    y, rms = qo.norm_rope_forward(x, w, 1e-6, f)
    y2, rms2 = qo.rmsnorm_forward(x, w, 1e-6)
    np.testing.assert_array_equal(y, qo.rope_forward(y2, f))
    np.testing.assert_array_equal(rms, rms2)
