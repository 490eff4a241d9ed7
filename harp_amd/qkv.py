"""The fused producer of the ring-attention block's q, k and v on the GPU.

``Z_Attention.forward`` (src/models/z_image/module/attn.py:69-89) projects
the hidden states with ``to_q``, ``to_k``, ``to_v`` (``nn.Linear`` without
bias, src/models/z_image/standalone_transformer.py:214-216), applies
``norm_q`` / ``norm_k`` (RMSNorm over each head's 128 features) and then RoPE
to q and k.  :func:`qkv_project` does all of it in one launch of the
hand-written kernel behind ``harp_qkv_project`` (include/harp_qk_norm_rope.h,
harp_amd/csrc/proj_kernels.hip): every 256-token x 128-feature tile of q, k
and v is computed once, and the tiles of q and k are normalised and rotated
in registers before their only store.

:class:`ProjectQKVFn` makes it differentiable: its forward also keeps the
pre-norm products and rms of q and k, and its backward runs the separate
norm + RoPE backward kernel (``async_op.qk_norm_rope_backward``) and the
projections' backward GEMMs (library GEMMs, as ``nn.Linear``'s own backward).

There is no CPU path: CPU tensors, or shapes the kernel does not take (head
dim other than 128, a bias, hidden size not a multiple of 64, RoPE without
RMSNorm), are reported by :func:`fused_supported` and left to the unfused
path of :func:`harp_amd.project_qkv`.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple

import torch

from . import _lib

HEAD_DIM = 128
K_TILE = 64


def _freqs_table(freqs_cis: torch.Tensor, B: int, S: int) -> Tuple[torch.Tensor, int, int]:
    """complex [S, 64] or [B or 1, S, 64] -> fp32 (cos, sin) pairs [.., S, 128]
    and its batch / row strides in floats (batch stride 0 when shared), as
    the async_op operators read it."""
    r = torch.view_as_real(freqs_cis).flatten(-2) if freqs_cis.is_complex() else freqs_cis
    if r.dtype != torch.float32:
        raise ValueError("freqs_cis must be complex64 (or its float32 view_as_real)")
    r = r.contiguous()
    if r.dim() not in (2, 3) or r.size(-1) != HEAD_DIM or r.size(-2) != S:
        raise ValueError(f"freqs_cis must be [S, 64] or [B, S, 64] complex with S={S}, got {tuple(freqs_cis.shape)}")
    if r.dim() == 3 and r.size(0) not in (1, B):
        raise ValueError(f"freqs_cis batch must be 1 or {B}")
    sb = r.stride(0) if (r.dim() == 3 and r.size(0) > 1) else 0
    return r, sb, r.stride(-2)


MAX_LD = 1 << 22  # harp_qkv_project: a 256-row tile of x or W spans < 2^32 bytes


def _aligned16(t: torch.Tensor) -> bool:
    return t.data_ptr() % 16 == 0


def fused_supported(attn, hidden_states: torch.Tensor, freqs_cis: Optional[torch.Tensor]) -> bool:
    """True when :func:`qkv_project` takes this attention module and input:
    the checks harp_qkv_project makes (shapes, dtypes, leading dimensions
    multiples of 8 up to 2^22, 16-byte aligned x / weight / norm-weight /
    RoPE-table pointers), made on what qkv_project would pass it, so that
    anything the kernel refuses takes the unfused path instead of raising."""
    x = hidden_states
    if not (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3 and x.stride(-1) == 1):
        return False
    K = x.size(-1)
    if K % K_TILE or K == 0 or K > MAX_LD:
        return False
    if x.is_contiguous() and not _aligned16(x):  # qkv_project passes x itself (a copy only when strided)
        return False
    lins = [getattr(attn, n, None) for n in ("to_q", "to_k", "to_v")]
    if any(m is None or getattr(m, "bias", None) is not None or not hasattr(m, "weight") for m in lins):
        return False
    n_out = lins[0].weight.size(0)
    if n_out % HEAD_DIM or n_out != attn.heads * HEAD_DIM:
        return False
    for m in lins:
        w = m.weight
        if w.dtype != torch.bfloat16 or w.device != x.device or tuple(w.shape) != (n_out, K) or w.stride(-1) != 1:
            return False
        if w.stride(0) % 8 or not K <= w.stride(0) <= MAX_LD or not _aligned16(w):
            return False
    norms = [getattr(attn, "norm_q", None), getattr(attn, "norm_k", None)]
    for nm in norms:
        if nm is None:
            continue
        w = getattr(nm, "weight", None)
        if w is None or w.dtype not in (torch.bfloat16, torch.float32) or w.device != x.device or w.numel() != HEAD_DIM:
            return False
        if not w.is_contiguous() or not _aligned16(w):
            return False
    if freqs_cis is not None:
        if any(nm is None for nm in norms) or not freqs_cis.is_cuda or freqs_cis.device != x.device:
            return False  # RoPE without RMSNorm runs on the separate operator
        try:
            table, _, _ = _freqs_table(freqs_cis, x.size(0), x.size(1))
        except ValueError:
            return False
        if not _aligned16(table):
            return False
    return x.size(0) * x.size(1) < (1 << 31)


def qkv_project(hidden_states: torch.Tensor, weights: Sequence[torch.Tensor],
                norms: Sequence[Tuple[Optional[torch.Tensor], float]], freqs_cis: Optional[torch.Tensor],
                keep_for_backward: bool = False):
    """([q, k, v], pre-norm products, rms) for hidden_states [B, S, dim], the
    Linear weights [H*128, dim] (one to three) and the (weight, eps) RMSNorm
    of each output (weight None: plain projection), then RoPE of the
    normalised outputs when freqs_cis is given.  The outputs are [B, H, S, 128]
    tensors with the token-major strides of the Linear output.  With
    keep_for_backward the normalised outputs' bf16 products ([B, S, H*128])
    and rms ([B*H*S] fp32) are written too (else None)."""
    x = hidden_states
    if not (x.is_cuda and x.dtype == torch.bfloat16 and x.dim() == 3):
        raise ValueError("hidden_states must be a [B, S, dim] bf16 tensor on a HIP device (there is no CPU path)")
    B, S, K = x.shape
    if not 1 <= len(weights) <= 3:
        raise ValueError(f"one to three weights, got {len(weights)}")
    n_out = weights[0].size(0)
    if n_out % HEAD_DIM or K % K_TILE or K == 0:
        raise ValueError(f"weights must be [heads*128, dim] with dim a multiple of {K_TILE}, got {tuple(weights[0].shape)}")
    for w in weights:
        if (w.dtype != torch.bfloat16 or w.device != x.device or tuple(w.shape) != (n_out, K) or w.stride(-1) != 1):
            raise ValueError(f"every weight must be a bf16 [{n_out}, {K}] tensor with unit column stride on "
                             f"{x.device}, got {w.dtype} {tuple(w.shape)} on {w.device}")
    for nw, _ in norms:
        if nw is not None and (nw.dtype not in (torch.bfloat16, torch.float32) or nw.device != x.device
                               or nw.numel() != HEAD_DIM or not nw.is_contiguous()):
            raise ValueError(f"RMSNorm weights must be contiguous [128] bf16 or fp32 tensors on {x.device}")
    x2 = x if x.is_contiguous() else x.contiguous()
    H = n_out // HEAD_DIM
    M = B * S
    f = None
    fsb = fss = 0
    if freqs_cis is not None:
        f, fsb, fss = _freqs_table(freqs_cis, B, S)
    outs = (_lib.QkvOut * 3)()
    ys, lins, rmss = [], [], []
    for i, w in enumerate(weights):
        # [B, H, S, 128] with the token-major strides of the Linear output
        y = torch.empty_strided((B, H, S, HEAD_DIM), (S * n_out, HEAD_DIM, n_out, 1), dtype=torch.bfloat16,
                                device=x.device)
        nw, eps = norms[i] if i < len(norms) else (None, 0.0)
        y_lin = rms = None
        if nw is not None and keep_for_backward:
            y_lin = torch.empty((B, S, n_out), dtype=torch.bfloat16, device=x.device)
            rms = torch.empty(B * H * S, dtype=torch.float32, device=x.device)
        o = outs[i]
        o.weight = w.data_ptr()
        o.ld_weight = w.stride(0)
        o.y = y.data_ptr()
        o.ld_y = n_out
        o.y_lin = y_lin.data_ptr() if y_lin is not None else None
        o.norm_weight = nw.data_ptr() if nw is not None else None
        o.norm_weight_dtype = _lib.HARP_QK_F32 if (nw is not None and nw.dtype == torch.float32) else _lib.HARP_QK_BF16
        o.eps = eps
        o.rms = rms.data_ptr() if rms is not None else None
        ys.append(y)
        lins.append(y_lin)
        rmss.append(rms)
    stream = torch.cuda.current_stream(x.device).cuda_stream
    rc = _lib.load_abi().harp_qkv_project(x2.data_ptr(), x2.stride(1), B, S, K, n_out,
                                         f.data_ptr() if f is not None else None, fsb, fss, outs, len(weights),
                                         ctypes.c_void_p(stream))
    _lib.qk_check(rc, "harp_qkv_project")
    return ys, lins, rmss


class ProjectQKVFn(torch.autograd.Function):
    """Differentiable :func:`qkv_project`: the three projections, and the
    RMSNorm (+ RoPE) of q and k where their norm weight is given."""

    @staticmethod
    def forward(ctx, hidden, wq, wk, wv, nwq, nwk, freqs_cis, eps_q, eps_k):
        norms = [(nwq, eps_q), (nwk, eps_k), (None, 0.0)]
        # the pre-norm products and rms are written only when a gradient can be
        # asked for (needs_input_grad follows requires_grad, also under no_grad:
        # callers that take no gradient call qkv_project directly)
        keep = any(ctx.needs_input_grad)
        (q, k, v), lins, rmss = qkv_project(hidden, [wq, wk, wv], norms, freqs_cis, keep_for_backward=keep)
        ctx.save_for_backward(hidden, wq, wk, wv, nwq, nwk, freqs_cis, lins[0], lins[1], rmss[0], rmss[1])
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        hidden, wq, wk, wv, nwq, nwk, freqs_cis, q_lin, k_lin, rms_q, rms_k = ctx.saved_tensors
        _lib.load_async_ops()
        ops = torch.ops.async_op
        B, S, K = hidden.shape
        n_out = wq.size(0)
        H = n_out // HEAD_DIM
        M = B * S
        x2 = hidden.reshape(M, K)

        def lin_grad(d, lin, nw, rms):
            """dL/d(product) as [M, n_out] from d ([B, H, S, 128]): through the
            RMSNorm (+ RoPE) backward kernel where the output was normalised."""
            if d is None:
                return None, None
            if nw is None:
                return d.transpose(1, 2).reshape(M, n_out), None
            d = d if d.stride(-1) == 1 else d.contiguous()
            x4 = lin.unflatten(-1, (H, HEAD_DIM)).transpose(1, 2)
            gx = torch.empty_like(lin)
            gx4 = gx.unflatten(-1, (H, HEAD_DIM)).transpose(1, 2)
            gw = torch.empty_like(nw)
            if freqs_cis is None:
                ops.rmsnorm_backward_out(x4, d, nw, rms, gx4, gw)
            else:
                ops.qk_norm_rope_backward(x4, d, nw, rms, freqs_cis, gx4, gw)
            return gx.reshape(M, n_out), gw

        gq, gnq = lin_grad(dq, q_lin, nwq, rms_q)
        gk, gnk = lin_grad(dk, k_lin, nwk, rms_k)
        gv, _ = lin_grad(dv, None, None, None)
        need = ctx.needs_input_grad
        dx = None
        if need[0]:
            for g, w in ((gq, wq), (gk, wk), (gv, wv)):
                if g is not None:
                    dx = g @ w if dx is None else dx.addmm_(g, w)
            dx = dx.view(B, S, K) if dx is not None else None
        dws = [g.t() @ x2 if (g is not None and need[n]) else None for g, n in ((gq, 1), (gk, 2), (gv, 3))]
        return (dx, dws[0], dws[1], dws[2], gnq if need[4] else None, gnk if need[5] else None, None, None, None)
