"""GPU test of the sustained-MFMA probes in the bench-only libharp_probe.so (a
measurement aid with no reference counterpart, outside the drop-in libraries):
each mix runs, reports a rate between a tenth of and the published dense bf16
peak, and a plausible shader clock."""

import pytest
import torch

from harp_amd import _lib

PEAK_BF16_TFLOPS = 2516.6


@pytest.mark.gpu
def test_probe_mfma_rate_is_plausible():
    torch.cuda.init()
    tf, ghz = _lib.probe_mfma_rate(1024, 3407)
    print(f"sustained bf16 MFMA {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0


@pytest.mark.gpu
def test_probe_rejects_bad_arguments():
    with pytest.raises(RuntimeError, match="iters"):
        _lib.probe_mfma_rate(3, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("softmax", [False, True])
def test_probe_mfma_lds_rate_is_plausible(softmax):
    torch.cuda.init()
    tf, ghz = _lib.probe_mfma_lds_rate(softmax, 2048, 3407)
    print(f"LDS-fed bf16 MFMA (softmax={softmax}) {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0


@pytest.mark.gpu
def test_probe_lds_rejects_bad_arguments():
    with pytest.raises(RuntimeError, match="iters"):
        _lib.probe_mfma_lds_rate(False, 17, 1)


@pytest.mark.gpu
@pytest.mark.parametrize("kernel", ["fwd", "dkdv", "dq"])
def test_probe_kernel_mix_is_plausible(kernel):
    torch.cuda.init()
    tf, ghz = _lib.probe_kernel_mix(kernel, 2052, 3407)
    print(f"{kernel} instruction mix {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0


@pytest.mark.gpu
def test_probe_kernel_mix_rejects_bad_arguments():
    lib = _lib.load_probe()
    import ctypes
    tf, ghz = ctypes.c_double(), ctypes.c_double()
    assert lib.harp_probe_kernel_mix(3, 2052, 1, ctypes.byref(tf), ctypes.byref(ghz)) == 1
    assert b"kernel" in lib.harp_probe_last_error()
    with pytest.raises(RuntimeError, match="iters"):
        _lib.probe_kernel_mix("dq", 15, 1)


@pytest.mark.gpu
def test_probe_fwd_asm_loop_is_plausible():
    """The D = 128 forward's generated loop on synthetic keys."""
    torch.cuda.init()
    tf, ghz = _lib.probe_fwd_asm_loop(256, 3407)
    print(f"forward loop {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0


@pytest.mark.gpu
def test_probe_dq_asm_loop_is_plausible():
    """The D = 128 dQ kernel's generated loop on synthetic keys."""
    torch.cuda.init()
    tf, ghz = _lib.probe_dq_asm_loop(256, 3407)
    print(f"dQ loop {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0


@pytest.mark.gpu
def test_probe_dkdv_asm_loop_is_plausible():
    """The D = 128 dK/dV kernel's generated loop on one synthetic query block."""
    torch.cuda.init()
    tf, ghz = _lib.probe_dkdv_asm_loop(256, 3407)
    print(f"dK/dV loop {tf:.1f} TFLOP/s at {ghz:.3f} GHz", flush=True)
    assert 0.1 * PEAK_BF16_TFLOPS < tf <= 1.02 * PEAK_BF16_TFLOPS
    assert 0.5 < ghz < 3.0
