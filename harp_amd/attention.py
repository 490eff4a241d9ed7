"""The attention block around the ring-attention operator, on the GPU.

:class:`RingZAttention` mirrors ``Z_Attention`` (src/models/z_image/module/
attn.py:51-105): it wraps the model's pretrained attention module (``to_q``,
``to_k``, ``to_v``, ``norm_q``, ``norm_k``, ``to_out``, ``heads``; the
``ZAttention`` of src/models/z_image/standalone_transformer.py:197-225) and
runs, for ``hidden_states`` [B, S, dim]:

1. the three projections, viewed as token-major [B, H, S, D] (attn.py:69-76);
2. QK RMSNorm and RoPE (attn.py:78-89), writing the token-major layout the
   ring kernel reads.  Steps 1-2 are one launch of the fused projection
   kernel (:mod:`harp_amd.qkv`) where it applies (head dim 128, no bias);
   otherwise plain library GEMMs (``nn.Linear``, hipBLASLt) and one fused
   norm + RoPE pass per tensor (:class:`QKNormRopeFn`), or the separate
   operator when only one of the two applies;
3. :class:`RingAttention` over ``sp_size`` KV chunks of the sequence (all on
   this GPU), then ``transpose(1, 2).flatten(2, 3)`` and ``to_out``
   (attn.py:99-103).

``attn_mask`` is accepted and ignored, as in the reference (attn.py:91-97).
:func:`project_qkv` is steps 1-2 on their own (the producer of q, k, v).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch
from torch import nn

from .ops import RingAttention
from .qk import ApplyRotaryComplexFn, QKNormRopeFn, RMSNormFn
from .qkv import ProjectQKVFn, fused_supported, qkv_project


def _norm_rope(x: torch.Tensor, norm: Optional[nn.Module], freqs_cis: Optional[torch.Tensor]) -> torch.Tensor:
    """RMSNorm (when ``norm`` is set) then RoPE (when ``freqs_cis`` is set) of a
    [B, H, S, D] view, on the async_op kernels."""
    if norm is not None:
        weight = getattr(norm, "weight", None)
        eps = float(norm.eps)
        if freqs_cis is not None:
            return QKNormRopeFn.apply(x, weight, freqs_cis, eps)
        return RMSNormFn.apply(x, weight, eps)
    if freqs_cis is not None:
        return ApplyRotaryComplexFn.apply(x, freqs_cis)
    return x


def project_qkv(attn: nn.Module, hidden_states: torch.Tensor, freqs_cis: Optional[torch.Tensor],
                fused: bool = True) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """q, k, v as token-major [B, H, S, D] views: projections, then QK RMSNorm
    and RoPE (attn.py:69-89).  With ``fused`` (default) and a module and input
    the fused kernel takes (:func:`harp_amd.qkv.fused_supported`: head dim
    128, no bias), all of it is one launch (:class:`ProjectQKVFn`); otherwise
    three library GEMMs and the separate norm + RoPE kernels."""
    if fused and fused_supported(attn, hidden_states, freqs_cis):
        nq, nk = getattr(attn, "norm_q", None), getattr(attn, "norm_k", None)
        args = (hidden_states, attn.to_q.weight, attn.to_k.weight, attn.to_v.weight,
                None if nq is None else nq.weight, None if nk is None else nk.weight, freqs_cis,
                0.0 if nq is None else float(nq.eps), 0.0 if nk is None else float(nk.eps))
        if torch.is_grad_enabled() and any(isinstance(a, torch.Tensor) and a.requires_grad for a in args):
            return ProjectQKVFn.apply(*args)
        # no gradient can be taken: the kernel alone, without the pre-norm
        # products and rms a backward would need
        (q, k, v), _, _ = qkv_project(args[0], args[1:4], [(args[4], args[7]), (args[5], args[8]), (None, 0.0)],
                                      freqs_cis)
        return q, k, v
    heads = attn.heads
    query = attn.to_q(hidden_states).unflatten(-1, (heads, -1)).transpose(1, 2)
    key = attn.to_k(hidden_states).unflatten(-1, (heads, -1)).transpose(1, 2)
    value = attn.to_v(hidden_states).unflatten(-1, (heads, -1)).transpose(1, 2)
    query = _norm_rope(query, getattr(attn, "norm_q", None), freqs_cis)
    key = _norm_rope(key, getattr(attn, "norm_k", None), freqs_cis)
    return query, key, value


class RingZAttention(nn.Module):
    """GPU drop-in for ``Z_Attention(pretrained_attn, sp_size)`` (attn.py:51-105).

    All ``sp_size`` ring chunks of the sequence are on this GPU: the sequence
    length S must be a multiple of ``sp_size``, and chunk c holds tokens
    c*S/sp_size .. (c+1)*S/sp_size - 1.  The result equals the reference's
    per-rank outputs concatenated over the ranks.
    """

    def __init__(self, pretrained_attn: nn.Module, sp_size: int):
        super().__init__()
        self.attn = pretrained_attn
        self.sp_size = sp_size

    def forward(self, hidden_states: torch.Tensor, RoPE_embeds: Optional[torch.Tensor],
                attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        attn = self.attn
        if hidden_states.size(1) % self.sp_size:
            raise ValueError(f"sequence length {hidden_states.size(1)} is not a multiple of sp_size {self.sp_size}")
        query, key, value = project_qkv(attn, hidden_states, RoPE_embeds)
        out = RingAttention.apply(query, key, value, self.sp_size).transpose(1, 2).flatten(2, 3)
        out = attn.to_out[0](out)
        if len(attn.to_out) > 1:  # dropout / identity
            out = attn.to_out[1](out)
        return out
