"""Autograd Functions over torch.ops.async_op for the step before ring
attention: QK RMSNorm and the rotary embedding, on the GPU.

* ``ApplyRotaryComplexFn`` mirrors the reference's Function of the same name
  (async_rt/async_ops.py:156-178): output allocated with the input's strides,
  ``rope_forward_impl`` / ``rope_backward_impl``, freqs_cis saved.
* ``RMSNormFn`` runs ``rmsnorm_forward_out`` / ``rmsnorm_backward_out``
  (async_rt/csrc/async_op_api.cc:54-55) and returns the weight gradient.
* ``QKNormRopeFn`` is the fused pair the model applies back to back
  (src/models/z_image/module/attn.py:78-89): one pass forward, one backward.

Every op runs on the current HIP stream through kernels/libharp_async_op.so;
there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _lib


def _ops():
    _lib.load_async_ops()
    return torch.ops.async_op


def _weight(weight, x):
    """The op schemas take a Tensor: an empty one stands for 'no weight'."""
    return weight if weight is not None else torch.empty(0, dtype=x.dtype, device=x.device)


def _rms_buffer(x: torch.Tensor) -> torch.Tensor:
    rows = x.numel() // x.size(-1)
    return torch.empty(rows, dtype=torch.float32, device=x.device)


class ApplyRotaryComplexFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, freqs_cis):
        y = torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=x.device)
        _ops().rope_forward_impl(x, freqs_cis, y)
        ctx.save_for_backward(freqs_cis)
        ctx.x_shape = x.shape
        return y

    @staticmethod
    def backward(ctx, grad_output):
        (freqs_cis,) = ctx.saved_tensors
        grad_x = torch.empty_strided(ctx.x_shape, grad_output.stride(), dtype=grad_output.dtype,
                                     device=grad_output.device)
        _ops().rope_backward_impl(grad_output, freqs_cis, grad_x)
        return grad_x, None


class RMSNormFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, eps):
        y = torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=x.device)
        rms = _rms_buffer(x)
        weight = _weight(weight, x)
        _ops().rmsnorm_forward_out(x, weight, y, rms, float(eps))
        ctx.save_for_backward(x, weight, rms)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, weight, rms = ctx.saved_tensors
        grad_output = grad_output.contiguous() if grad_output.stride(-1) != 1 else grad_output
        grad_x = torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=x.device)
        grad_w = torch.empty_like(weight) if weight.numel() else torch.empty(0, device=x.device)
        _ops().rmsnorm_backward_out(x, grad_output, weight, rms, grad_x, grad_w)
        return grad_x, (grad_w if grad_w.numel() else None), None


class QKNormRopeFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, freqs_cis, eps):
        y = torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=x.device)
        rms = _rms_buffer(x)
        weight = _weight(weight, x)
        _ops().qk_norm_rope_forward(x, weight, freqs_cis, y, rms, float(eps))
        ctx.save_for_backward(x, weight, rms, freqs_cis)
        return y

    @staticmethod
    def backward(ctx, grad_output):
        x, weight, rms, freqs_cis = ctx.saved_tensors
        grad_output = grad_output.contiguous() if grad_output.stride(-1) != 1 else grad_output
        grad_x = torch.empty_strided(x.size(), x.stride(), dtype=x.dtype, device=x.device)
        grad_w = torch.empty_like(weight) if weight.numel() else torch.empty(0, device=x.device)
        _ops().qk_norm_rope_backward(x, grad_output, weight, rms, freqs_cis, grad_x, grad_w)
        return grad_x, (grad_w if grad_w.numel() else None), None, None
