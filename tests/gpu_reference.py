"""A plain PyTorch fp32 reference of the ring-attention block on the GPU,
for full-size parity checks (the CPU oracle covers every element only at
small sizes).  Same math as the oracle (oracle/ring_attn_oracle.py): softmax
attention of q against the concatenated valid keys of every chunk, fp32
arithmetic on the bf16 inputs, exact scale; backward with D = rowsum(dO*O),
P = exp(S - LSE), dS = P (dP - D), dQ = scale dS K, dK = scale dS^T Q,
dV = P^T dO.  Processed per (b, h) and per block of keys, so no T x L matrix
is held whole.  tests/test_gpu_fullsize.py pins it against the oracle."""

from __future__ import annotations

from typing import Dict, Optional, Sequence

import torch


@torch.no_grad()
def attention_fp32(q: torch.Tensor, ks: Sequence[torch.Tensor], vs: Sequence[torch.Tensor], do: torch.Tensor,
                   scale: float, lens: Optional[Sequence[int]] = None, key_block: int = 8192) -> Dict[str, torch.Tensor]:
    """q, do [B,H,T,D] and chunk lists ks, vs ([B,H,Tc,D]) on the GPU, bf16.
    Returns fp32 o, lse, delta ([B,H,T,1]), dq, and dk, dv over the
    concatenated chunks ([B,H,N*Tc,D], pad rows 0)."""
    B, H, T, D = q.shape
    tcs = [k.shape[2] for k in ks]
    lens = list(tcs) if lens is None else list(lens)
    dev = q.device
    o = torch.empty((B, H, T, D), device=dev, dtype=torch.float32)
    lse = torch.empty((B, H, T, 1), device=dev, dtype=torch.float32)
    delta = torch.empty_like(lse)
    dq = torch.zeros((B, H, T, D), device=dev, dtype=torch.float32)
    dk = torch.zeros((B, H, sum(tcs), D), device=dev, dtype=torch.float32)
    dv = torch.zeros_like(dk)
    offs = [sum(tcs[:c]) for c in range(len(tcs))]
    for b in range(B):
        for h in range(H):
            qh = q[b, h].float()
            doh = do[b, h].float()
            blocks = []  # (chunk offset of the block, K block, V block)
            for c, (k, v, n) in enumerate(zip(ks, vs, lens)):
                for k0 in range(0, n, key_block):
                    k1 = min(n, k0 + key_block)
                    blocks.append((offs[c] + k0, k[b, h, k0:k1].float(), v[b, h, k0:k1].float()))
            m = torch.full((T, 1), float("-inf"), device=dev)
            l = torch.zeros((T, 1), device=dev)
            for _, kb, _ in blocks:
                s = (qh @ kb.t()) * scale
                m_new = torch.maximum(m, s.amax(-1, keepdim=True))
                l = l * torch.exp(m - m_new) + torch.exp(s - m_new).sum(-1, keepdim=True)
                m = m_new
            lse_h = m + torch.log(l)
            oh = torch.zeros((T, D), device=dev)
            for _, kb, vb in blocks:
                oh += torch.exp((qh @ kb.t()) * scale - lse_h) @ vb
            dl = (doh * oh).sum(-1, keepdim=True)
            for r0, kb, vb in blocks:
                p = torch.exp((qh @ kb.t()) * scale - lse_h)
                ds = p * (doh @ vb.t() - dl)
                dq[b, h] += (ds @ kb) * scale
                dk[b, h, r0:r0 + kb.shape[0]] = (ds.t() @ qh) * scale
                dv[b, h, r0:r0 + kb.shape[0]] = p.t() @ doh
            o[b, h] = oh
            lse[b, h] = lse_h
            delta[b, h] = dl
    return {"o": o, "lse": lse, "delta": delta, "dq": dq, "dk": dk, "dv": dv}
