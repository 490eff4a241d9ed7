"""GPU test of harp_qk_norm_rope_backward_noalloc, the allocation-free variant
of harp_qk_norm_rope_backward (weight-gradient partials in the library's
static device scratch instead of a workspace).  Both are called through the C
ABI on the same inputs, twice in a row, the second call smaller than the
first (the scratch keeps the first call's partials): dx and grad_weight must
equal the workspace entry point's bit for bit, since both run the same
kernels and the same fixed-order reduction."""

import ctypes

import numpy as np
import pytest
import torch

from harp_amd import _lib

pytestmark = pytest.mark.gpu


def _i64(t):
    return _lib.i64_array(t.stride())


def _inputs(B, H, S, D, seed):
    g = torch.Generator().manual_seed(seed)
    tok = lambda: torch.randn((B, S, H, D), generator=g).to(torch.bfloat16).cuda().transpose(1, 2)  # noqa: E731
    x, dy = tok(), tok()
    w = (1 + 0.1 * torch.randn(D, generator=g)).to(torch.bfloat16).cuda()
    rms = (0.5 + torch.rand(B * H * S, generator=g)).cuda()
    ang = torch.arange(S, dtype=torch.float64)[:, None] * (10000.0 ** (-2.0 * torch.arange(D // 2) / D))[None, :]
    freqs = torch.view_as_real(torch.polar(torch.ones_like(ang), ang).to(torch.complex64)).reshape(S, D).cuda()
    return x, dy, w, rms, freqs


def _call(noalloc, x, dy, w, rms, freqs, gw_dtype):
    lib = _lib.load_abi()
    B, H, S, D = x.shape
    dx = torch.full_like(x, float("nan")).transpose(1, 2).contiguous().transpose(1, 2)
    gw = torch.full((D,), float("nan"), device="cuda", dtype=gw_dtype)
    gwt = _lib.HARP_QK_F32 if gw_dtype == torch.float32 else _lib.HARP_QK_BF16
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    common = (dy.data_ptr(), _i64(dy), x.data_ptr(), _i64(x), w.data_ptr(), _lib.HARP_QK_BF16, rms.data_ptr(),
              freqs.data_ptr(), 0, D, dx.data_ptr(), _i64(dx), gw.data_ptr(), gwt, B, H, S, D)
    if noalloc:
        rc = lib.harp_qk_norm_rope_backward_noalloc(*common, stream)
    else:
        nbytes = lib.harp_qk_backward_workspace_bytes(B, H, S, D)
        ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
        rc = lib.harp_qk_norm_rope_backward(*common, ws.data_ptr(), nbytes, stream)
    _lib.qk_check(rc, "harp_qk_norm_rope_backward" + ("_noalloc" if noalloc else ""))
    return dx, gw


def _bits(t):
    return t.detach().contiguous().cpu().view(torch.int16 if t.dtype == torch.bfloat16 else torch.int32).numpy()


@pytest.mark.parametrize("gw_dtype", [torch.float32, torch.bfloat16])
def test_noalloc_backward_equals_workspace_backward(gw_dtype):
    # first call: 2048 row blocks (the scratch's maximum) at D = 128; second:
    # a smaller problem at another D, which reads fewer partial rows
    for (B, H, S, D), seed in (((1, 24, 8192, 128), 1), ((2, 3, 100, 72), 2)):
        print(f"[noalloc backward B={B} H={H} S={S} D={D} grad_weight {gw_dtype}]", flush=True)
        args = _inputs(B, H, S, D, seed)
        want_dx, want_gw = _call(False, *args, gw_dtype)
        got_dx, got_gw = _call(True, *args, gw_dtype)
        torch.cuda.synchronize()
        assert torch.isfinite(got_dx.float()).all() and torch.isfinite(got_gw.float()).all()
        np.testing.assert_array_equal(_bits(got_dx), _bits(want_dx))
        np.testing.assert_array_equal(_bits(got_gw), _bits(want_gw))


def test_noalloc_backward_rejects_bad_sizes_on_the_host():
    lib = _lib.load_abi()
    st = _lib.i64_array([8 * 64 * 512, 512, 8 * 512, 1])
    fake = 1 << 20  # never dereferenced: validation fails first
    rc = lib.harp_qk_norm_rope_backward_noalloc(fake, st, fake, st, None, 1, fake, fake, 0, 512, fake, st, None, 1,
                                                1, 8, 64, 512, None)
    assert rc == 2 and "D=512" in lib.harp_qk_last_error().decode()
