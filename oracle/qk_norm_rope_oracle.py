"""CPU oracle for the QK-RMSNorm and RoPE operators (HARP's async runtime).

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` may import this module, and only as
the checker (or, for the baseline, as the timed CPU restatement).  The product
path (``harp_amd``) never imports it and has no CPU fallback.

What it restates
----------------
The reference kernels are ARM SVE C++ (``async_rt/csrc/rms_norm.cc`` and
``async_rt/csrc/rope.cc``; not buildable on x86: they need ``arm_sve.h``).
Their arithmetic, row by row over the last dimension D:

* RMSNorm forward (``rmsnormForwardKernelBF16``, rms_norm.cc:20-105):
  ``sum_sq = sum(x*x)`` (fused multiply-adds, :54-55), ``variance = sum_sq / D``
  (:65), ``rms = sqrt(variance + eps)`` (:67), ``inv = 1 / rms`` (:68),
  ``out = (x * inv) * w`` (two rounded products, :83-96), ``rms`` saved (:69).
* RMSNorm backward (``rmsnormBackwardKernelBF16``, rms_norm.cc:107-240):
  ``inv = 1 / rms`` (:146), ``gn = dy * w``, ``xn = x * inv``,
  ``dot = sum(gn * xn)`` (:170-185), ``coeff = dot / D`` (:189),
  ``dx = (gn - xn * coeff) * inv`` (:210-218), ``grad_w += dy * xn``
  (:222-229).  The reference's binding passes a NULL weight-gradient pointer
  (rms_norm.cc:500-512), so its operator returns zeros for grad_weight; the
  oracle returns the sum the kernel accumulates.
* RoPE forward (``rope_row``, rope.cc:9-44): pairs (x[2i], x[2i+1]) times
  (f[2i], f[2i+1]) as complex numbers with two FCMLA steps:
  ``re = fma(-xi, fi, xr*fr)``, ``im = fma(xi, fr, xr*fi)``.
* RoPE backward (``rope_backward_row``, rope.cc:88-141): times the
  conjugate, ``re = fma(gi, fi, gr*fr)``, ``im = fma(-gr, fi, gi*fr)``.
* Every bf16 store keeps the high 16 bits of the fp32 value (truncation,
  ``fp32x2_store_as_bf16``, async_rt/csrc/async_op_math.h:24-35); loads
  widen exactly (:12-22).

The oracle follows that order of fp32 roundings with numpy float32 values.
Reductions (sums of squares and dot products) are formed in float64 and
rounded once: the reference's SVE lane order is not reproducible, so a
result may differ from the reference or the GPU by one bf16 unit where a
value sits on a truncation boundary.  Fused multiply-adds are formed exactly
in float64 (the product of two fp32 values is exact there) and rounded once.

How each function is pinned (tests/test_qk_oracle.py):
* rmsnorm_forward: vs an fp64 restatement of x / sqrt(mean(x^2) + eps) * w
  (the model's RMSNorm module, src/models/z_image/standalone_transformer.py:
  123-153); truncation bounds |out| <= |exact| < |out| + 1 ulp; the rms of
  out / w is 1 for eps = 0.
* rmsnorm_backward: vs fp64 autograd of that formula (dx and grad_w).
* rope_forward / rope_backward: vs complex multiplication with
  torch.view_as_complex (fp64); norm preservation for unit |f|; backward is
  the adjoint (fp64 autograd) and undoes the forward for unit |f|.
* Planted mistakes in copies of the math (sum instead of mean, conjugate
  dropped, rotated pair order) fail these checks.
"""

from __future__ import annotations

import numpy as np

F32 = np.float32


def bf16_to_f32(u16: np.ndarray) -> np.ndarray:
    """Exact widening of bf16 bits (uint16) to float32 (async_op_math.h:12-22)."""
    return (u16.astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_trunc(x: np.ndarray) -> np.ndarray:
    """bf16 bits of float32 values by truncation (async_op_math.h:24-35)."""
    return (np.ascontiguousarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def f32_to_bf16_rne(x: np.ndarray) -> np.ndarray:
    """bf16 bits by round-to-nearest-even (how torch casts fp32 inputs)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def _fma(a, b, c):
    """fp32 fused multiply-add: the product of two fp32 values is exact in
    float64; the sum is rounded once to float32."""
    return (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(F32)


def _weight(w, D):
    if w is None:
        return np.ones(D, dtype=F32)
    w = np.asarray(w)
    return bf16_to_f32(w) if w.dtype == np.uint16 else w.astype(F32)


def rmsnorm_forward(x_bf16: np.ndarray, w=None, eps: float = 1e-6):
    """RMSNorm over the last axis (rms_norm.cc:39-103).  x_bf16: uint16 bf16
    bits [..., D]; w: bf16 bits (uint16) or float32 [D], or None.  Returns
    (out bf16 bits, rms float32 [...])."""
    x = bf16_to_f32(x_bf16)
    D = x.shape[-1]
    wf = _weight(w, D)
    ss = (x.astype(np.float64) ** 2).sum(-1).astype(F32)
    var = (ss / F32(D)).astype(F32)
    rms = np.sqrt((var + F32(eps)).astype(F32)).astype(F32)
    inv = (F32(1.0) / rms).astype(F32)
    y = ((x * inv[..., None]).astype(F32) * wf).astype(F32)
    return f32_to_bf16_trunc(y), rms


def rmsnorm_backward(x_bf16: np.ndarray, dy_bf16: np.ndarray, w, rms: np.ndarray):
    """RMSNorm backward (rms_norm.cc:139-230).  Returns (dx bf16 bits,
    grad_w float32 [D] = sum over rows of dy * xn)."""
    x = bf16_to_f32(x_bf16)
    dy = bf16_to_f32(dy_bf16)
    D = x.shape[-1]
    wf = _weight(w, D)
    inv = (F32(1.0) / rms.astype(F32)).astype(F32)[..., None]
    gn = (dy * wf).astype(F32)
    xn = (x * inv).astype(F32)
    dot = (gn.astype(np.float64) * xn.astype(np.float64)).sum(-1).astype(F32)
    coeff = (dot / F32(D)).astype(F32)[..., None]
    dx = ((gn - (xn * coeff).astype(F32)).astype(F32) * inv).astype(F32)
    gw = (dy.astype(np.float64) * xn.astype(np.float64)).reshape(-1, D).sum(0).astype(F32)
    return f32_to_bf16_trunc(dx), gw


def rope_forward(x_bf16: np.ndarray, freqs: np.ndarray):
    """RoPE (rope.cc:9-44): freqs float32 [..., D] of (cos, sin) pairs,
    broadcast against x [..., D].  Returns bf16 bits."""
    x = bf16_to_f32(x_bf16)
    f = np.broadcast_to(freqs.astype(F32), x.shape)
    xr, xi = x[..., 0::2], x[..., 1::2]
    fr, fi = f[..., 0::2], f[..., 1::2]
    re = _fma(-xi, fi, (xr * fr).astype(F32))
    im = _fma(xi, fr, (xr * fi).astype(F32))
    out = np.empty_like(x)
    out[..., 0::2] = re
    out[..., 1::2] = im
    return f32_to_bf16_trunc(out)


def rope_backward(dy_bf16: np.ndarray, freqs: np.ndarray):
    """RoPE backward (rope.cc:115-134): times the conjugate.  Returns bf16 bits."""
    g = bf16_to_f32(dy_bf16)
    f = np.broadcast_to(freqs.astype(F32), g.shape)
    gr, gi = g[..., 0::2], g[..., 1::2]
    fr, fi = f[..., 0::2], f[..., 1::2]
    re = _fma(gi, fi, (gr * fr).astype(F32))
    im = _fma(-gr, fi, (gi * fr).astype(F32))
    out = np.empty_like(g)
    out[..., 0::2] = re
    out[..., 1::2] = im
    return f32_to_bf16_trunc(out)


def norm_rope_forward(x_bf16, w, eps, freqs):
    """RMSNorm then RoPE, as the model applies them (attn.py:78-89)."""
    y, rms = rmsnorm_forward(x_bf16, w, eps)
    return rope_forward(y, freqs), rms


def norm_rope_backward(x_bf16, dy_bf16, w, rms, freqs):
    """RoPE backward then RMSNorm backward."""
    g = rope_backward(dy_bf16, freqs)
    return rmsnorm_backward(x_bf16, g, w, rms)


def rope_table(S: int, D: int, theta: float = 10000.0, offset: int = 0) -> np.ndarray:
    """A standard rotary table, float32 [S, D] of (cos, sin) pairs: angle
    (s + offset) * theta^(-2i/D) for pair i (test input; the model builds its
    own freqs_cis)."""
    i = np.arange(D // 2, dtype=np.float64)
    inv_freq = theta ** (-2.0 * i / D)
    ang = (np.arange(S, dtype=np.float64) + offset)[:, None] * inv_freq[None, :]
    out = np.empty((S, D), dtype=F32)
    out[:, 0::2] = np.cos(ang)
    out[:, 1::2] = np.sin(ang)
    return out
