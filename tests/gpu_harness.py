"""Drive the HIP path for parity tests: token-major device copies, calls
through the C ABI (per-chunk pointers) or through torch.ops, results back on
the CPU.  Imports no oracle code."""

from __future__ import annotations

import math
from typing import Dict, List, Optional, Sequence

import torch

import harp_amd
from harp_amd import ops as hops


def token_major_dev(x: torch.Tensor, device="cuda") -> torch.Tensor:
    """[B,H,T,D] (any layout, CPU) -> device [B,H,T,D] view over [B,T,H,D] storage."""
    return x.transpose(1, 2).contiguous().to(device).transpose(1, 2)


def head_major_dev(x: torch.Tensor, device="cuda") -> torch.Tensor:
    return x.contiguous().to(device)


def run_hip(
    q: torch.Tensor,
    ks: Sequence[torch.Tensor],
    vs: Sequence[torch.Tensor],
    do: torch.Tensor,
    scale: Optional[float] = None,
    ring_rank: int = 0,
    kv_lens: Optional[Sequence[int]] = None,
    via: str = "abi",
    m_dtype: torch.dtype = torch.bfloat16,
    out_layout: str = "token",
    do_layout: str = "token",
    grad_dtype: torch.dtype = torch.bfloat16,
    backward: bool = True,
    dkv_view: Optional[tuple] = None,
    dq_view: Optional[tuple] = None,
) -> Dict[str, torch.Tensor]:
    """Run forward (+ delta + backward) on the GPU; return CPU tensors:
    o (fp32), lse (fp64), m, l, delta, dq, dk, dv (dk/dv concatenated over chunks).
    dkv_view = (pad, offset) (C ABI only): each dK / dV chunk is the view
    [..., offset:offset + D] of a token-major buffer whose rows hold D + pad
    elements per head, so the view's row stride is H (D + pad) and its base
    sits `offset` elements into the buffer.  dq_view = (pad, offset): the same
    for dQ (C ABI only)."""
    dev = torch.device("cuda")
    B, H, T, D = q.shape
    n = len(ks)
    tc = ks[0].shape[2]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    qd = token_major_dev(q)
    if via == "abi":
        kd = [token_major_dev(k) for k in ks]
        vd = [token_major_dev(v) for v in vs]
    else:
        kd = [token_major_dev(torch.cat(list(ks), dim=2))]
        vd = [token_major_dev(torch.cat(list(vs), dim=2))]
    if out_layout == "token":
        out = torch.empty((B, T, H, D), device=dev, dtype=torch.float32).transpose(1, 2)
    else:
        out = torch.empty((B, H, T, D), device=dev, dtype=torch.float32)
    out.fill_(float("nan"))
    m_i = torch.full((B, H, T, 1), float("nan"), device=dev, dtype=m_dtype)
    l_i = torch.full((B, H, T, 1), float("nan"), device=dev, dtype=torch.float32)
    if via == "abi":
        hops.abi_forward(qd, kd, vd, out, m_i, l_i, scale, ring_rank=ring_rank, kv_lens=kv_lens)
    else:
        harp_amd.load_ops()
        torch.ops.ring_attention_ops.ring_attention_forward(
            qd, kd[0], vd[0], out, m_i, l_i, n, scale, ring_rank, None if kv_lens is None else list(kv_lens), tc)
    res = {"o": out, "m": m_i, "l": l_i}
    if backward:
        dod = token_major_dev(do) if do_layout == "token" else head_major_dev(do)
        if via == "abi":
            delta = torch.empty((B, H, T, 1), device=dev, dtype=torch.float32)
            hops.abi_delta(dod, out, delta)
            if dq_view is not None:
                pad, off = dq_view
                dq = torch.full((B, T, H, D + pad), float("nan"), device=dev, dtype=grad_dtype)[..., off:off + D]
                dq = dq.transpose(1, 2)
            else:
                dq = torch.full((B, T, H, D), float("nan"), device=dev, dtype=grad_dtype).transpose(1, 2)

            def grad_chunk():
                if dkv_view is not None:
                    pad, off = dkv_view
                    buf = torch.full((B, tc, H, D + pad), float("nan"), device=dev, dtype=grad_dtype)
                    return buf[..., off:off + D].transpose(1, 2)
                return torch.full((B, tc, H, D), float("nan"), device=dev, dtype=grad_dtype).transpose(1, 2)

            dk = [grad_chunk() for _ in range(n)]
            dv = [grad_chunk() for _ in range(n)]
            hops.abi_backward(qd, dq, kd, vd, dk, dv, dod, m_i, l_i, delta, scale, ring_rank=ring_rank,
                              kv_lens=kv_lens)
            dk_all = torch.cat(dk, dim=2)
            dv_all = torch.cat(dv, dim=2)
        else:
            assert dkv_view is None and dq_view is None, "dkv_view / dq_view go through the C ABI"
            delta = torch.ops.ring_attention_ops.ring_attention_delta(dod, out)
            dq = torch.full((B, T, H, D), float("nan"), device=dev, dtype=grad_dtype).transpose(1, 2)
            dk_all = torch.full((B, n * tc, H, D), float("nan"), device=dev, dtype=grad_dtype).transpose(1, 2)
            dv_all = torch.full((B, n * tc, H, D), float("nan"), device=dev, dtype=grad_dtype).transpose(1, 2)
            torch.ops.ring_attention_ops.ring_attention_backward(
                qd, dq, kd[0], dk_all, vd[0], dv_all, dod, m_i, l_i, delta, n, scale, ring_rank,
                None if kv_lens is None else list(kv_lens), tc)
        res.update(delta=delta, dq=dq, dk=dk_all, dv=dv_all)
    torch.cuda.synchronize()
    cpu = {k: v.cpu() for k, v in res.items()}
    cpu["lse"] = cpu["m"].double() + torch.log(cpu["l"].double())
    return cpu
