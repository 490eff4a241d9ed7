#!/usr/bin/env python
"""Benchmark: ring-attention block fwd+bwd on one MI355X.

Metric: ring-attn fwd+bwd TFLOP/s and % of bf16 MFMA peak at
S_local=8192, D=128 — config 4: B=1, H=24, D=128, T=8192 local queries, KV
streamed as 8 chunks of 8192 (8 ring steps, 65536 keys), bf16 N(0,1) inputs
from seed 3407, non-causal.

One step = the hot path once: ring_attention_forward (fused forward kernel),
ring_attention_delta (D = rowsum(dO*O)), and ring_attention_backward (dK/dV
kernel + dQ kernel), called through torch.ops.ring_attention_ops with every
input and output resident in HBM.  FLOP_total = 14*B*H*T*L*D (fwd 4, bwd 10;
L = valid keys).

Prints ONE JSON line.  --gpus N with N > 1 is refused: this build measures one
GPU (multi-GPU sharding is a design, not a measured path).  After the headline
(config 4) it adds, as context: BASELINE configs 2, 3 and 5 (`other_configs`)
and HARP's own call shapes, 30 heads of 128 with 256 or 768 local rows over 8
ring steps (`harp_call_shapes`).
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

PEAK_BF16_TFLOPS = 2516.6  # 256 CU x 2.4 GHz x 4096 FLOP/clk/CU (dense)
PEAK_HBM_GBS = 8000.0

# HBM bytes per launch (read + write) of each kernel at config 4, measured
# with rocprofv3 --pmc FETCH_SIZE and WRITE_SIZE, each scaled by what the same
# counter reads for a 1 GiB device copy in the same run (FETCH x2.0, WRITE
# x1.0).  Source: profiles/ring_attn_config4_counters.md.
MEASURED_TRAFFIC_BYTES = {4: {"fwd": 960.3e6, "dkdv": 2429.0e6, "dq": 961.8e6, "delta": 151.8e6}}

CONFIGS = {
    1: dict(B=1, H=8, T=512, D=64, N=1, tc=512, lens=None, vscale=1.0),
    2: dict(B=1, H=16, T=2048, D=64, N=4, tc=2048, lens=None, vscale=1.0),
    3: dict(B=2, H=16, T=4096, D=72, N=8, tc=4096, lens=None, vscale=0.5),
    4: dict(B=1, H=24, T=8192, D=128, N=8, tc=8192, lens=None, vscale=1.0),
    5: dict(B=1, H=24, T=4429, D=128, N=4, tc=4480, lens=[4429] * 4, vscale=1.0),
}
# HARP's own per-rank call shapes (30 heads of 128, 256 / 768 local rows, an
# 8-rank ring): context beside the BASELINE configs, not a bench line
HARP_SHAPES = {
    "T256": dict(B=1, H=30, T=256, D=128, N=8, tc=256, lens=None, vscale=1.0),
    "T768": dict(B=1, H=30, T=768, D=128, N=8, tc=768, lens=None, vscale=1.0),
}


def make_inputs_dev(cfg, seed, device):
    """Seeded inputs (draw order Q, K chunks, V chunks, dO; fp32 randn -> bf16)
    laid out token-major on the device; k/v hold all chunks along T."""
    import torch

    B, H, T, D, N, tc = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["N"], cfg["tc"]
    g = torch.Generator().manual_seed(seed)

    def draw(rows):
        x = torch.randn((B, rows, H, D), generator=g, dtype=torch.float32)
        if cfg["vscale"] != 1.0:
            x = x * cfg["vscale"]
        return x.to(torch.bfloat16)

    q = draw(T).to(device).transpose(1, 2)
    k = torch.empty((B, N * tc, H, D), dtype=torch.bfloat16, device=device)
    v = torch.empty_like(k)
    for c in range(N):
        k[:, c * tc:(c + 1) * tc] = draw(tc).to(device)
    for c in range(N):
        v[:, c * tc:(c + 1) * tc] = draw(tc).to(device)
    do = draw(T).to(device).transpose(1, 2)
    return q, k.transpose(1, 2), v.transpose(1, 2), do


def cpu_threads() -> int:
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count() or 1
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit():
        n = min(n, int(cap))
    return max(1, n)


def cpu_info() -> dict:
    """Host CPU as lscpu reports it: model, physical cores (sockets x cores per
    socket), hardware threads, and the bf16 / matrix extensions the CPU
    baseline's matmuls could use."""
    info = {"model": "unknown", "physical_cores": None, "hw_threads": os.cpu_count(), "bf16_flags": []}
    fields = {}
    try:
        import subprocess

        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            if ":" in line:
                k, v = line.split(":", 1)
                fields[k.strip()] = v.strip()
    except (OSError, ValueError):
        pass
    flags = fields.get("Flags", "").split()
    if not flags:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("flags"):
                        flags = line.split(":", 1)[1].split()
                        break
        except OSError:
            pass
    info["model"] = fields.get("Model name", info["model"])
    try:
        info["physical_cores"] = int(fields["Socket(s)"]) * int(fields["Core(s) per socket"])
        info["hw_threads"] = int(fields.get("CPU(s)", info["hw_threads"]))
    except (KeyError, ValueError):
        pass
    info["bf16_flags"] = sorted(f for f in flags if f in ("avx512f", "avx512_bf16", "amx_bf16", "amx_tile", "avx_vnni"))
    return info


def cpu_model() -> str:
    return cpu_info()["model"]


def cpu_baseline(cfg, target_s: float):
    """The reference algorithm as PyTorch CPU ops (oracle.cpu_baseline_fwd_bwd)
    on a bounded sample of the workload: query rows of one head (then whole
    heads, one at a time) against the full KV length, sized from a short probe
    so that one repetition takes about target_s / 4.  One warm-up and three
    timed repetitions of that sample; the median is reported, with the three
    times and the host's model, cores and bf16 / matrix flags.  Returns the
    cpu_baseline JSON object."""
    import statistics

    import torch

    from oracle import ring_attn_oracle as orc

    threads = cpu_threads()
    torch.set_num_threads(threads)
    B, D, N, T, tc, H = 1, cfg["D"], cfg["N"], cfg["T"], cfg["tc"], cfg["H"]
    lens = cfg["lens"] or [tc] * N
    L = sum(lens)
    scale = 1.0 / math.sqrt(D)

    def run(tq, seed):
        q, ks, vs, do = orc.make_inputs(B, 1, tq, D, N, seed=seed, chunk_len=tc, value_scale=cfg["vscale"])
        ks = [k[:, :, :n] for k, n in zip(ks, lens)]
        vs = [v[:, :, :n] for v, n in zip(vs, lens)]
        t0 = time.perf_counter()
        orc.cpu_baseline_fwd_bwd(q, ks, vs, do, scale)
        return time.perf_counter() - t0

    run(64, 1)  # warm up oneDNN / thread pool
    rep_s = target_s / 4
    rows_target = 128 * rep_s / max(run(128, 1), 1e-3)
    if rows_target <= T:
        tq, nh = max(128, int(rows_target) // 128 * 128), 1
    else:
        tq, nh = T, int(min(H, max(1, rows_target // T)))

    def sample():
        return sum(run(tq, 1 + i) for i in range(nh))

    sample()  # warm-up repetition
    reps = [sample() for _ in range(3)]
    dt = statistics.median(reps)
    flops = 14.0 * nh * tq * L * D
    ci = cpu_info()
    return {
        "value": round(flops / dt / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "cpu_model": ci["model"],
        "physical_cores": ci["physical_cores"],
        "hw_threads": ci["hw_threads"],
        "bf16_flags": ci["bf16_flags"],
        "reps_s": [round(r, 2) for r in reps],
        "sample": (f"{nh} of {H} heads x {tq} of {T} query rows against all {L} keys ({N} chunks), fwd+bwd; "
                   f"median of 3 repetitions ({dt:.1f} s each) after 1 warm-up, {threads} threads"),
    }


def producer_bench(cfg, seed: int, iters: int = 20):
    """The step before the ring-attention block: fused QK RMSNorm + RoPE
    forward and backward (torch.ops.async_op.qk_norm_rope_{forward,backward})
    on one Q-shaped tensor of the workload ([B, H, T, D] token-major view),
    timed with HIP events on the current stream.  HBM-bound: algorithmic
    bytes per call are x in + out (bf16) + rms (fp32) + the RoPE table once per
    token (forward); dy + x in + dx out (bf16) + rms + table + the
    weight-gradient partials written and read (backward)."""
    import torch

    import harp_amd
    from harp_amd import _lib

    harp_amd.load_async_ops()
    ops = torch.ops.async_op
    dev = torch.device("cuda:0")
    B, H, T, D = cfg["B"], cfg["H"], cfg["T"], cfg["D"]
    g = torch.Generator().manual_seed(seed)
    x = torch.randn((B, T, H, D), generator=g).to(torch.bfloat16).to(dev).transpose(1, 2)
    dy = torch.randn((B, T, H, D), generator=g).to(torch.bfloat16).to(dev).transpose(1, 2)
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).to(dev)
    ang = torch.arange(T, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(D // 2) / D))[None, :]
    freqs = torch.polar(torch.ones_like(ang), ang).to(torch.complex64).to(dev)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    rms = torch.empty(B * H * T, device=dev, dtype=torch.float32)
    gw = torch.empty(D, device=dev, dtype=torch.bfloat16)
    rows = B * H * T
    ws_bytes = _lib.load_abi().harp_qk_backward_workspace_bytes(B, H, T, D)
    fwd_bytes = rows * D * 2 * 2 + rows * 4 + T * D * 4
    bwd_bytes = rows * D * 2 * 3 + rows * 4 + T * D * 4 + 2 * ws_bytes
    res = {}
    for name, fn, nbytes in (
        ("forward", lambda: ops.qk_norm_rope_forward(x, w, freqs, y, rms, 1e-6), fwd_bytes),
        ("backward", lambda: ops.qk_norm_rope_backward(x, dy, w, rms, freqs, dx, gw), bwd_bytes),
    ):
        for _ in range(3):
            fn()
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(iters):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        us = ev[0].elapsed_time(ev[1]) * 1e3 / iters
        gbs = nbytes / (us * 1e-6) / 1e9
        res[name] = {"avg_us": round(us, 2), "bytes": int(nbytes), "GB_s": round(gbs, 1),
                     "frac_hbm_peak": round(gbs / PEAK_HBM_GBS, 4)}
    res["shape"] = f"[B,H,T,D]=[{B},{H},{T},{D}] token-major bf16, weight bf16 [D], freqs complex64 [T, D/2]"
    res["ops"] = "async_op.qk_norm_rope_forward / qk_norm_rope_backward (one of Q, K)"

    # The whole producer of one rank's q, k, v (harp_amd.project_qkv): three
    # projections of hidden [B, T, H*D] (plain library GEMMs, hipBLASLt) and
    # the fused norm + RoPE of q and k, forward only.
    from types import SimpleNamespace

    dim = H * D
    lin = [torch.nn.Linear(dim, dim, bias=False).to(dev, torch.bfloat16) for _ in range(3)]
    norm = SimpleNamespace(weight=w, eps=1e-6)
    attn = SimpleNamespace(heads=H, to_q=lin[0], to_k=lin[1], to_v=lin[2], norm_q=norm, norm_k=norm)
    hid = torch.randn((B, T, dim), generator=g).to(torch.bfloat16).to(dev)
    gemm_flop = 3 * 2 * B * T * dim * dim

    def timed(fn, n=iters, warm=10):
        for _ in range(warm):
            fn()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
        torch.cuda.synchronize()
        e[0].record()
        for _ in range(n):
            fn()
        e[1].record()
        torch.cuda.synchronize()
        return e[0].elapsed_time(e[1]) / n

    # the producer as harp_amd.project_qkv runs it (fused kernel: projections
    # with norm + RoPE in the epilogue), and the unfused path beside it
    with torch.no_grad():
        # the two paths alternated twice after a warm-up of both (the board's
        # clock settles over the first calls), mean of the two measurements each
        timed(lambda: harp_amd.project_qkv(attn, hid, freqs), n=20)
        runs = [(timed(lambda: harp_amd.project_qkv(attn, hid, freqs)),
                 timed(lambda: harp_amd.project_qkv(attn, hid, freqs, fused=False))) for _ in range(2)]
        ms = sum(r[0] for r in runs) / 2
        ms_unfused = sum(r[1] for r in runs) / 2
    res["project_qkv_forward"] = {
        "avg_ms": round(ms, 4),
        "gemm_flop": gemm_flop,
        "tflops_incl_norm_rope": round(gemm_flop / (ms * 1e-3) / 1e12, 1),
        "what": f"3 projections [{B},{T},{dim}] x [{dim},{dim}] with norm+RoPE of q and k in the epilogue "
                "(one launch of the fused projection kernel)",
        "unfused_avg_ms": round(ms_unfused, 4),
        "unfused_what": "torch Linear (hipBLASLt) x 3, then the fused norm+RoPE kernel on q and k",
    }
    # the fused kernel alone, HIP events on the launch stream, and as the
    # training forward runs it (pre-norm products and rms also written)
    from harp_amd import qkv as _qkv

    ws3 = [m.weight for m in lin]
    nrm = [(w, 1e-6), (w, 1e-6), (None, 0.0)]
    with torch.no_grad():
        ms_k = timed(lambda: _qkv.qkv_project(hid, ws3, nrm, freqs))
        ms_kt = timed(lambda: _qkv.qkv_project(hid, ws3, nrm, freqs, keep_for_backward=True))
    res["project_qkv_forward"]["kernel_ms"] = round(ms_k, 4)
    res["project_qkv_forward"]["kernel_tflops"] = round(gemm_flop / (ms_k * 1e-3) / 1e12, 1)
    res["project_qkv_forward"]["kernel_frac_bf16_peak"] = round(gemm_flop / (ms_k * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 4)
    res["project_qkv_forward"]["kernel_keep_for_backward_ms"] = round(ms_kt, 4)

    w_cat = torch.cat([m.weight for m in lin], 0)
    qkv = torch.empty((B, T, 3 * dim), device=dev, dtype=torch.bfloat16)
    q_out = torch.empty((B, T, dim), device=dev, dtype=torch.bfloat16).unflatten(-1, (H, D)).transpose(1, 2)
    k_out = torch.empty_like(q_out)
    rms_q = torch.empty(B * H * T, device=dev, dtype=torch.float32)
    with torch.no_grad():
        ms_3 = timed(lambda: [m(hid) for m in lin])
        ms_cat = timed(lambda: torch.matmul(hid, w_cat.t(), out=qkv))
        qv = qkv[..., :dim].unflatten(-1, (H, D)).transpose(1, 2)
        kv = qkv[..., dim:2 * dim].unflatten(-1, (H, D)).transpose(1, 2)
        ms_nr = timed(lambda: (ops.qk_norm_rope_forward(qv, w, freqs, q_out, rms_q, 1e-6),
                               ops.qk_norm_rope_forward(kv, w, freqs, k_out, rms_q, 1e-6)))
    res["producer_parts"] = {
        "three_gemms_ms": round(ms_3, 4),
        "three_gemms_tflops": round(gemm_flop / (ms_3 * 1e-3) / 1e12, 1),
        "one_concatenated_gemm_ms": round(ms_cat, 4),
        "one_concatenated_gemm_tflops": round(gemm_flop / (ms_cat * 1e-3) / 1e12, 1),
        "norm_rope_q_and_k_ms": round(ms_nr, 4),
        "norm_rope_q_and_k_bytes": int(2 * fwd_bytes),
        "norm_rope_q_and_k_frac_hbm_peak": round(2 * fwd_bytes / (ms_nr * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
    }

    # The producer's backward as training runs it (ProjectQKVFn): the fused
    # RMSNorm + RoPE backward of q and k, then dX (three GEMMs into one
    # accumulator) and dW (three GEMMs); gradients of all inputs, none
    # accumulated into .grad.
    hid_g = hid.clone().requires_grad_(True)
    wts = [m.weight.detach().clone().requires_grad_(True) for m in lin]
    nw_g = w.detach().clone().requires_grad_(True)
    q_o, k_o, v_o = _qkv.ProjectQKVFn.apply(hid_g, wts[0], wts[1], wts[2], nw_g, nw_g, freqs, 1e-6, 1e-6)
    grads = [torch.randn(t.shape, generator=g).to(torch.bfloat16).to(dev).as_strided(t.shape, t.stride())
             for t in (q_o, k_o, v_o)]
    ins = [hid_g, *wts, nw_g]
    ms_b = timed(lambda: torch.autograd.grad([q_o, k_o, v_o], ins, grads, retain_graph=True), n=iters, warm=5)
    gq = torch.empty((B, T, dim), device=dev, dtype=torch.bfloat16)
    gq4 = gq.unflatten(-1, (H, D)).transpose(1, 2)
    lin4 = torch.randn((B, T, dim), generator=g).to(torch.bfloat16).to(dev).unflatten(-1, (H, D)).transpose(1, 2)
    gwt = torch.empty(D, device=dev, dtype=torch.bfloat16)
    with torch.no_grad():
        ms_nrb = timed(lambda: (ops.qk_norm_rope_backward(lin4, grads[0], w, rms_q, freqs, gq4, gwt),
                                ops.qk_norm_rope_backward(lin4, grads[1], w, rms_q, freqs, gq4, gwt)))
    bwd_flop = 2 * gemm_flop  # dX and dW: each the forward's three products
    res["project_qkv_backward"] = {
        "avg_ms": round(ms_b, 4),
        "gemm_flop": bwd_flop,
        "tflops_gemms": round(bwd_flop / (ms_b * 1e-3) / 1e12, 1),
        "norm_rope_backward_q_and_k_ms": round(ms_nrb, 4),
        "norm_rope_backward_q_and_k_bytes": int(2 * bwd_bytes),
        "norm_rope_backward_q_and_k_frac_hbm_peak": round(2 * bwd_bytes / (ms_nrb * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "what": "ProjectQKVFn backward through autograd: fused RMSNorm + RoPE backward of q and k "
                "(async_op.qk_norm_rope_backward), then dX = sum of three products and dW of each weight "
                "(hipBLASLt); gradients of hidden, the three weights and the norm weight",
    }
    return res


def producer_cpu_baseline(cfg, seed: int, target_s: float = 4.0):
    """The reference's producer math as a CPU restatement (oracle, numpy) on
    a bounded sample of Q rows: fused forward + backward per row, rows/s."""
    import numpy as np

    from oracle import qk_norm_rope_oracle as qo

    D, T = cfg["D"], cfg["T"]
    rng = np.random.default_rng(seed)
    f = qo.rope_table(T, D)
    w = qo.f32_to_bf16_rne((1 + 0.1 * rng.standard_normal(D)).astype(np.float32))

    def run(rows):
        s_len = min(rows, T)
        x = qo.f32_to_bf16_rne(rng.standard_normal((rows // s_len, s_len, D)).astype(np.float32))
        dy = qo.f32_to_bf16_rne(rng.standard_normal((rows // s_len, s_len, D)).astype(np.float32))
        t0 = time.perf_counter()
        y, rms = qo.norm_rope_forward(x, w, 1e-6, f[:s_len])
        qo.norm_rope_backward(x, dy, w, rms, f[:s_len])
        return time.perf_counter() - t0

    run(1024)
    probe = run(8192)
    rows = int(max(8192, min(cfg["B"] * cfg["H"] * T, 8192 * target_s / max(probe, 1e-3))) // 8192 * 8192)
    dt = run(rows)
    return {"rows_per_s": round(rows / dt, 1), "cores": 1, "kind": "port",
            "sample": f"{rows} rows of D={D} (fused forward + backward, numpy), {dt:.1f} s on {cpu_model()}"}


PROBE_LIB = os.path.join(os.path.dirname(os.path.abspath(__file__)), "kernels", "libharp_bench_probe.so")
_probe_lib = None


def probe_rate(lds_fed: bool, iters: int, seed: int) -> tuple:
    """(TFLOP/s, shader GHz) of a dense bf16 MFMA stream on random operands
    (bench_probe.hip): register-fed at 32 waves per CU, or (lds_fed) with
    one operand of every MFMA read from LDS at the kernels' 8 waves per CU."""
    import ctypes

    global _probe_lib
    if _probe_lib is None:
        if not os.path.exists(PROBE_LIB):
            raise FileNotFoundError(f"{PROBE_LIB} is not built: run __graft_entry__.build()")
        lib = ctypes.CDLL(PROBE_LIB)
        for fn in (lib.harp_probe_mfma_rate, lib.harp_probe_mfma_lds_rate):
            fn.restype = ctypes.c_int
            fn.argtypes = [ctypes.c_int, ctypes.c_uint32, ctypes.POINTER(ctypes.c_double),
                           ctypes.POINTER(ctypes.c_double)]
        lib.harp_probe_last_error.restype = ctypes.c_char_p
        _probe_lib = lib
    tf, ghz = ctypes.c_double(), ctypes.c_double()
    fn = _probe_lib.harp_probe_mfma_lds_rate if lds_fed else _probe_lib.harp_probe_mfma_rate
    rc = fn(int(iters), int(seed) & 0xFFFFFFFF, ctypes.byref(tf), ctypes.byref(ghz))
    if rc != 0:
        raise RuntimeError(f"MFMA probe failed (status {rc}): {_probe_lib.harp_probe_last_error().decode()}")
    return tf.value, ghz.value


class BoardTelemetry:
    """The board's own power, shader-clock and power-limit readings (SMU
    metrics through amdsmi), taken while one piece of work runs in a loop:
    socket power and GFX clock sampled every few milliseconds, the average
    power from the energy counter, and the share of the interval the SMU
    spent limiting the clock for package power (PPT residency counters).
    Read-only; every field is None where this board or driver does not
    report it."""

    def __init__(self, torch_mod):
        import amdsmi

        self.smi = amdsmi
        amdsmi.amdsmi_init()
        handles = amdsmi.amdsmi_get_processor_handles()
        if not handles:
            raise RuntimeError("amdsmi sees no GPU")
        self.h = handles[0]
        props = torch_mod.cuda.get_device_properties(0)
        bus = getattr(props, "pci_bus_id", None)
        if bus is not None and len(handles) > 1:
            for h in handles:
                try:
                    bdf = amdsmi.amdsmi_get_gpu_device_bdf(h)
                    if int(bdf.split(":")[1], 16) == int(bus):
                        self.h = h
                        break
                except Exception:  # noqa: BLE001 - best effort matching
                    pass
        self.cap_w = None
        try:
            cap = amdsmi.amdsmi_get_power_cap_info(self.h).get("power_cap")
            if isinstance(cap, (int, float)) and cap > 0:
                self.cap_w = cap / 1e6 if cap > 1e5 else float(cap)  # reported in microwatts
        except Exception:  # noqa: BLE001
            pass

    def _metrics(self):
        return self.smi.amdsmi_get_gpu_metrics_info(self.h)

    @staticmethod
    def _num(x):
        return x if isinstance(x, (int, float)) and not isinstance(x, bool) else None

    def measure(self, fn, seconds: float, sync) -> dict:
        import statistics
        import threading

        samples = []
        stop = threading.Event()

        def sampler():
            while not stop.is_set():
                try:
                    m = self._metrics()
                    clks = m.get("current_gfxclks")
                    clk = None
                    if isinstance(clks, (list, tuple)):
                        v = [c for c in clks if self._num(c) and 0 < c < 10000]
                        clk = sum(v) / len(v) if v else None
                    if clk is None:
                        clk = self._num(m.get("current_gfxclk"))
                    samples.append((self._num(m.get("current_socket_power")), clk))
                except Exception:  # noqa: BLE001
                    pass
                stop.wait(0.005)

        m0 = self._metrics()
        t0 = time.perf_counter()
        th = threading.Thread(target=sampler, daemon=True)
        th.start()
        n = 0
        while time.perf_counter() - t0 < seconds:
            fn()
            n += 1
            sync()
        stop.set()
        th.join()
        t1 = time.perf_counter()
        m1 = self._metrics()

        def delta(key):
            a, b = self._num(m0.get(key)), self._num(m1.get(key))
            return None if a is None or b is None else b - a

        acc = delta("accumulation_counter")
        ppt = delta("ppt_residency_acc")
        thm = delta("socket_thm_residency_acc")
        pw = [p for p, _ in samples if p]
        ck = [c for _, c in samples if c]
        return {
            "seconds": round(t1 - t0, 3),
            "calls": n,
            "samples": len(samples),
            "socket_power_w_median": round(statistics.median(pw), 1) if pw else None,
            "socket_power_w_max": round(max(pw), 1) if pw else None,
            "power_cap_w": round(self.cap_w, 1) if self.cap_w else None,
            "gfxclk_mhz_median": round(statistics.median(ck), 1) if ck else None,
            "gfxclk_mhz_min": round(min(ck), 1) if ck else None,
            "ppt_limited_frac": round(min(1.0, max(0.0, ppt / acc)), 4) if acc and ppt is not None else None,
            "thermal_limited_frac": round(min(1.0, max(0.0, thm / acc)), 4) if acc and thm is not None else None,
        }


def bhtld_of(cfg) -> float:
    lens = cfg["lens"]
    L = sum(lens) if lens else cfg["N"] * cfg["tc"]
    return float(cfg["B"]) * cfg["H"] * cfg["T"] * L * cfg["D"]


class Workload:
    """One BASELINE config resident on the device, with the step of the hot
    path (forward, delta, backward through torch.ops.ring_attention_ops)."""

    def __init__(self, cfg, seed, dev):
        import torch

        self.cfg = cfg
        B, H, T, D, N, tc = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["N"], cfg["tc"]
        self.lens, self.N, self.tc = cfg["lens"], N, tc
        self.scale = 1.0 / math.sqrt(D)
        self.q, self.k, self.v, self.do = make_inputs_dev(cfg, seed, dev)
        self.out = torch.empty((B, T, H, D), device=dev, dtype=torch.float32).transpose(1, 2)
        self.m_i = torch.empty((B, H, T, 1), device=dev, dtype=torch.bfloat16)
        self.l_i = torch.empty((B, H, T, 1), device=dev, dtype=torch.float32)
        self.dq = torch.empty_like(self.q)
        self.dk = torch.empty_like(self.k)
        self.dv = torch.empty_like(self.v)
        self.delta = None
        self.ops = torch.ops.ring_attention_ops

    def forward(self):
        self.ops.ring_attention_forward(self.q, self.k, self.v, self.out, self.m_i, self.l_i, self.N, self.scale, 0,
                                        self.lens, self.tc)

    def backward(self):
        self.delta = self.ops.ring_attention_delta(self.do, self.out)
        self.ops.ring_attention_backward(self.q, self.dq, self.k, self.dk, self.v, self.dv, self.do, self.m_i,
                                         self.l_i, self.delta, self.N, self.scale, 0, self.lens, self.tc)

    def step(self):
        self.forward()
        self.backward()

    def timed(self, steps: int, warmup: int) -> dict:
        """warmup untimed steps, then `steps` timed ones between one pair of
        HIP events on the current stream (nothing else recorded in between:
        the step time is the operators' own), then `steps` more with an event
        after each (their median; an event between steps costs a few µs at
        the smallest shapes, so those steps do not give the mean), then
        `steps` more with the library's per-kernel launch timing on (its event
        pairs around every launch add gaps to the stream, so those steps only
        give the per-kernel breakdown).  Returns ms per step (mean over the
        first timed steps, median of the second), per-kernel (ms, launches) of
        the third, and the host wall time of the first."""
        import torch

        from harp_amd import _lib

        for _ in range(warmup):
            self.step()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t_wall = time.perf_counter()
        e0.record()
        for _ in range(steps):
            self.step()
        e1.record()
        torch.cuda.synchronize()
        wall_s = time.perf_counter() - t_wall
        ms = e0.elapsed_time(e1) / steps
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 1)]
        ev[0].record()
        for i in range(steps):
            self.step()
            ev[i + 1].record()
        torch.cuda.synchronize()
        step_ms = sorted(ev[i].elapsed_time(ev[i + 1]) for i in range(steps))
        med = step_ms[len(step_ms) // 2] if len(step_ms) % 2 else 0.5 * (
            step_ms[len(step_ms) // 2 - 1] + step_ms[len(step_ms) // 2])
        _lib.timing_read()  # discard
        _lib.timing_enable(True)
        for _ in range(steps):
            self.step()
        torch.cuda.synchronize()
        _lib.timing_enable(False)
        kt = _lib.timing_read()
        return {"ms": ms, "median_ms": med, "kernels": kt, "wall_s": wall_s}


def other_configs(ids, seed, dev, min_steps: int = 10, table=None) -> dict:
    """The other BASELINE configs that run on the GPU (parity cases, not the
    headline), or other named shapes (`table`): ms per fwd+bwd step, counted
    TFLOP/s and % of the bf16 peak, and each kernel's ms per step.  Each
    shape warms up for about 30 ms of its own steps (a few steps of a small
    shape end before the board's clocks settle under the load) and times at
    least `min_steps` steps and about 20 ms."""
    import torch

    res = {}
    for cid in ids:
        cfg = (table or CONFIGS)[cid]
        w = Workload(cfg, seed, dev)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(3):
            w.step()
        torch.cuda.synchronize()
        est = max((time.perf_counter() - t0) / 3, 1e-5)
        warmup = max(3, int(0.03 / est))
        steps = max(min_steps, int(0.02 / est))
        r = w.timed(steps, warmup)
        tf = 14.0 * bhtld_of(cfg) / (r["ms"] * 1e-3) / 1e12
        res[str(cid)] = {
            "shape": f"B{cfg['B']} H{cfg['H']} D{cfg['D']} T{cfg['T']}, {cfg['N']} chunks of {cfg['tc']}"
                     + (f" ({cfg['lens'][0]} valid, pad keys masked)" if cfg["lens"] else ""),
            "ms_per_step": round(r["ms"], 4),
            "tflops": round(tf, 1),
            "pct_bf16_peak": round(100.0 * tf / PEAK_BF16_TFLOPS, 2),
            "kernel_ms_per_step": {k: round(ms / steps, 4) for k, (ms, n) in r["kernels"].items() if n},
            "steps": steps,
        }
        del w
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
    return res


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", type=int, default=4, choices=sorted(CONFIGS))
    ap.add_argument("--seed", type=int, default=3407)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="target CPU-baseline sample time")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-producer", action="store_true",
                    help="skip the QK RMSNorm + RoPE (producer step) measurement")
    ap.add_argument("--no-telemetry", action="store_true", help="skip the board power / clock readings")
    ap.add_argument("--no-other-configs", action="store_true",
                    help="skip BASELINE configs 2, 3 and 5 after the headline (config 4) run")
    ap.add_argument("--no-harp-shapes", action="store_true",
                    help="skip HARP's own call shapes (H 30, D 128, T 256 / 768, 8 ring steps) after the headline")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="before the timed steps, run one plain device copy of this many MiB "
                         "(a known-size reference for rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    args = ap.parse_args()

    if args.gpus != 1:
        print(f"bench.py: --gpus {args.gpus} is not supported; this build measures the ring-attention "
              "block on exactly one GPU (all ring steps of one rank's share on that GPU).", file=sys.stderr)
        return 2

    import torch

    import harp_amd

    assert torch.cuda.is_available(), "bench.py needs a HIP device"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    harp_amd.load_ops()

    cfg = CONFIGS[args.config]
    B, H, T, D, N, tc = cfg["B"], cfg["H"], cfg["T"], cfg["D"], cfg["N"], cfg["tc"]
    lens = cfg["lens"]
    L = sum(lens) if lens else N * tc
    work = Workload(cfg, args.seed, dev)

    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib * (1 << 20) // 4
        src = torch.ones(n, device=dev, dtype=torch.float32)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    r = work.timed(args.steps, args.warmup)
    kt, wall_s, ms_per_step, ms_median = r["kernels"], r["wall_s"], r["ms"], r["median_ms"]
    print(f"bench: config {args.config} timed, {ms_per_step:.4f} ms per step", file=sys.stderr, flush=True)

    bhtld = bhtld_of(cfg)
    flop_total = 14.0 * bhtld
    tflops = flop_total / (ms_per_step * 1e-3) / 1e12
    # algorithmic MFMA work per launch in this design's accounting
    kernel_flops = {"fwd": 4.0 * bhtld, "dkdv": 8.0 * bhtld, "dq": 2.0 * bhtld}
    # MFMA work each kernel performs (dq recomputes S and dP: 4 more units)
    kernel_mfma = {"fwd": 4.0 * bhtld, "dkdv": 8.0 * bhtld, "dq": 6.0 * bhtld}
    # sustained MFMA rate of this board (register-fed bf16 MFMA stream on
    # random operands), and the same at the kernels' operand path (one
    # operand of every MFMA from LDS, 1 KB per MFMA per wave, 8 waves per CU)
    probe_tf, probe_ghz = probe_rate(False, 4096, args.seed)
    lds_tf, lds_ghz = probe_rate(True, 32768, args.seed)
    kernels = {}
    for name, (ms, n) in kt.items():
        if n:
            avg = ms / n
            entry = {"avg_ms": round(avg, 4), "launches_per_step": n / args.steps}
            if name in kernel_flops:
                entry["tflops_algorithmic"] = round(kernel_flops[name] / (avg * 1e-3) / 1e12, 1)
                performed = kernel_mfma[name] / (avg * 1e-3) / 1e12
                entry["tflops_mfma_performed"] = round(performed, 1)
                entry["frac_of_sustained"] = round(performed / probe_tf, 4) if probe_tf > 0 else None
                entry["frac_of_lds_fed"] = round(performed / lds_tf, 4) if lds_tf > 0 else None
            kernels[name] = entry
    dom = max((n for n in kernel_flops if n in kernels), key=lambda n: kt[n][0])
    dom_tf = kernels[dom]["tflops_algorithmic"]
    fwd_ms = kt["fwd"][0] / args.steps
    bwd_ms = (kt["stats"][0] + kt["dkdv"][0] + kt["dq"][0] + kt["delta"][0]) / args.steps

    result = {
        "metric": "ring-attn fwd+bwd TFLOP/s and % bf16 MFMA peak, S_local=8192 D=128",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "ms_per_step_median": round(ms_median, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) bf16, draw order Q, K chunks, V chunks, dO)",
        "config": {
            "workload": f"BASELINE config {args.config}: ring attention fwd+bwd, one rank's share on one GPU",
            "B": B, "H": H, "D": D, "S_local": T, "kv_chunks": N, "chunk_len": tc, "L_valid": L,
            "causal": False, "parallelism": "single GPU, ring steps streamed from HBM",
        },
        "pct_bf16_peak": round(100.0 * tflops / PEAK_BF16_TFLOPS, 2),
        "fwd_ms": round(fwd_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "kernels": kernels,
        "wall_s_timed": round(wall_s, 3),
        "roofline": {
            "bound": "mfma",
            "kernel": dom,
            "achieved": dom_tf,
            "peak": PEAK_BF16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(dom_tf / PEAK_BF16_TFLOPS, 4),
            "traffic": MEASURED_TRAFFIC_BYTES.get(args.config, {}).get(dom),
            "sustained_mfma_tflops": round(probe_tf, 1),
            "sustained_mfma_shader_ghz": round(probe_ghz, 3),
            "frac_of_sustained": round(dom_tf / probe_tf, 4) if probe_tf > 0 else None,
            "lds_fed_mfma_tflops": round(lds_tf, 1),
            "lds_fed_mfma_shader_ghz": round(lds_ghz, 3),
            "frac_of_lds_fed": round(dom_tf / lds_tf, 4) if lds_tf > 0 else None,
        },
        "cpu_baseline": None,
        "gpu": torch.cuda.get_device_name(0),
        "clock_policy": "default power mode (not pinned)",
    }
    if not args.no_telemetry:
        # the board's power / clock / power-limit readings while each piece
        # of work runs alone in a loop (after the timed steps, outside them)
        try:
            tel = BoardTelemetry(torch)
            sync = torch.cuda.synchronize
            result["telemetry"] = {
                "probe_register_fed": tel.measure(lambda: probe_rate(False, 65536, args.seed), 1.5, sync),
                "probe_lds_fed": tel.measure(lambda: probe_rate(True, 262144, args.seed), 1.5, sync),
                "forward": tel.measure(work.forward, 1.5, sync),
                "backward_dkdv_dq": tel.measure(work.backward, 1.5, sync),
                "what": "amdsmi SMU metrics while the work runs in a loop: socket power and GFX clock sampled "
                        "every ~5 ms (median, max / min), ppt_limited_frac = share of the interval the SMU held "
                        "the clock down for package power (ppt_residency_acc / accumulation_counter deltas)",
            }
        except Exception as e:  # noqa: BLE001 - telemetry is context, never the measurement
            result["telemetry"] = {"unavailable": f"{type(e).__name__}: {e}"}
        print("bench: telemetry done", file=sys.stderr, flush=True)
    if args.config == 4 and not args.no_other_configs:
        del work
        torch.cuda.synchronize()
        torch.cuda.empty_cache()
        result["other_configs"] = other_configs((2, 3, 5), args.seed, dev)
        print("bench: other configs done", file=sys.stderr, flush=True)
    if args.config == 4 and not args.no_harp_shapes:
        result["harp_call_shapes"] = other_configs(tuple(HARP_SHAPES), args.seed, dev, table=HARP_SHAPES)
        print("bench: HARP call shapes done", file=sys.stderr, flush=True)
    if not args.no_producer:
        prod = producer_bench(cfg, args.seed)
        rows = B * H * T
        prod["gpu_rows_per_s"] = round(rows / ((prod["forward"]["avg_us"] + prod["backward"]["avg_us"]) * 1e-6), 1)
        if not args.no_cpu_baseline:
            prod["cpu_baseline"] = producer_cpu_baseline(cfg, args.seed)
        result["producer_qk_norm_rope"] = prod
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(result), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
