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
