"""Write tests/golden/ra_tiny.npz: small ring-attention cases with fp64
oracle outputs.

The reference ships no golden vectors for this path, so these fixtures come
from the build's own oracle (oracle/ring_attn_oracle.py), which
tests/test_oracle.py pins against fp64 SDPA, fp64 autograd, brute force and
finite differences.  Inputs are stored as bf16 bit patterns (uint16);
outputs as float32 rounded from fp64.  Rerun:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import ring_attn_oracle as orc  # noqa: E402

# name: (B, H, T, D, N, chunk_len, valid_lens or None, value_scale, ring_rank, seed)
CASES = {
    "d64_n1": (1, 2, 48, 64, 1, 48, None, 1.0, 0, 3407),
    "d64_n4": (1, 2, 40, 64, 4, 40, None, 1.0, 1, 3407),
    "d72_n2": (2, 1, 48, 72, 2, 48, None, 0.5, 0, 3407),
    "d128_n3": (1, 2, 33, 128, 3, 33, None, 1.0, 2, 3407),
    "d64_masked": (1, 2, 37, 64, 2, 40, [40, 29], 1.0, 0, 3407),
}


def build_case(B, H, T, D, N, tc, lens, vscale, rank, seed):
    q, ks, vs, do = orc.make_inputs(B, H, T, D, N, seed=seed, value_scale=vscale, chunk_len=tc)
    scale = 1.0 / math.sqrt(D)
    o, m, l = orc.ring_forward(q, ks, vs, scale, ring_rank=rank, kv_valid_lens=lens)
    Dl = orc.delta(do, o)
    dq, dks, dvs = orc.ring_backward(q, ks, vs, do, m, l, Dl, scale, ring_rank=rank, kv_valid_lens=lens)
    f32 = lambda t: t.detach().to(torch.float32).contiguous().numpy()  # noqa: E731
    bits = lambda t: t.detach().to(torch.bfloat16).contiguous().view(torch.int16).numpy().view(np.uint16)  # noqa: E731
    return {
        "meta": np.array([B, H, T, D, N, tc, rank], dtype=np.int64),
        "lens": np.array(lens if lens is not None else [tc] * N, dtype=np.int64),
        "scale": np.array([scale], dtype=np.float64),
        "q": bits(q),
        "k": bits(torch.cat(ks, dim=2)),
        "v": bits(torch.cat(vs, dim=2)),
        "do": bits(do),
        "o": f32(o),
        "lse": f32(orc.lse_from_ml(m, l)),
        "delta": f32(Dl),
        "dq": f32(dq),
        "dk": f32(torch.cat(dks, dim=2)),
        "dv": f32(torch.cat(dvs, dim=2)),
    }


def main() -> None:
    arrays = {}
    for name, spec in CASES.items():
        for key, val in build_case(*spec).items():
            arrays[f"{name}/{key}"] = val
    path = os.path.join(HERE, "ra_tiny.npz")
    np.savez_compressed(path, **arrays)
    print(f"wrote {path} ({os.path.getsize(path)} bytes, {len(CASES)} cases)")


if __name__ == "__main__":
    main()
