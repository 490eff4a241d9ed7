"""CPU tests of the QK-RMSNorm / RoPE boundary: libharp_ra.so exports exactly
the functions include/harp_qk_norm_rope.h declares, validates arguments on the
host before touching a device, sizes its workspace, and the async_op operator
library registers the reference's schemas (no GPU needed)."""

import os
import re
import subprocess

import pytest
import torch

import harp_amd
from harp_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "harp_qk_norm_rope.h")

# async_rt/csrc/async_op_api.cc:54-57
REF_SCHEMAS = {
    "rmsnorm_forward_out": "rmsnorm_forward_out(Tensor input, Tensor weight, Tensor(a!) output, Tensor(b!) rms, "
                           "float eps) -> ()",
    "rmsnorm_backward_out": "rmsnorm_backward_out(Tensor input, Tensor grad_output, Tensor weight, Tensor rms, "
                            "Tensor(a!) grad_input, Tensor(b!) grad_weight) -> ()",
    "rope_forward_impl": "rope_forward_impl(Tensor x, Tensor freqs_cis, Tensor(a!) output) -> ()",
    "rope_backward_impl": "rope_backward_impl(Tensor grad_output, Tensor freqs_cis, Tensor(b!) grad_x) -> ()",
}


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"HARP_QK_API\s+[\w\s\*]+?\b(harp_qkv?_\w+)\s*\(", text)))


def test_header_and_prototypes_agree():
    fns = header_functions()
    assert len(fns) == 10
    assert set(fns) == set(_lib.QK_PROTOTYPES)


def test_library_exports_every_declared_symbol():
    lib = harp_amd.load_abi()
    for name in header_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.ABI_LIB)], capture_output=True, text=True)
    exported = {ln.split()[-1] for ln in nm.stdout.splitlines() if " T " in ln}
    assert {s for s in exported if s.startswith(("harp_qk_", "harp_qkv_"))} == set(header_functions())


def _strides(b, h, s, d=1):
    return _lib.i64_array([b, h, s, d])


FAKE = 1 << 20  # 16-byte aligned, never dereferenced: validation fails first


def _fwd(**over):
    lib = harp_amd.load_abi()
    st = _strides(8 * 64 * 128, 64, 8 * 64)
    a = dict(x=FAKE, xs=st, w=None, wdt=_lib.HARP_QK_BF16, eps=1e-6, f=FAKE, fsb=0, fss=128, out=FAKE, os=st,
             rms=FAKE, B=1, H=8, S=64, D=128)
    a.update(over)
    return lib.harp_qk_norm_rope_forward(a["x"], a["xs"], a["w"], a["wdt"], a["eps"], a["f"], a["fsb"], a["fss"],
                                         a["out"], a["os"], a["rms"], a["B"], a["H"], a["S"], a["D"], None)


@pytest.mark.parametrize("over,msg", [
    (dict(x=None), "x is NULL"),
    (dict(x=FAKE + 2), "16-byte aligned"),
    (dict(D=100), "multiple of 8"),
    (dict(D=264), "not supported"),
    (dict(S=0), "positive"),
    (dict(xs=_strides(8 * 64 * 128, 64, 8 * 64, 2)), "unit stride"),
    (dict(os=_strides(8 * 64 * 128, 64, 7)), "multiple of 8"),
    (dict(f=None), "freqs is NULL"),
    (dict(fss=130), "multiples of 4"),
    (dict(eps=-1.0), "eps"),
    (dict(w=FAKE, wdt=7), "dtype"),
    (dict(w=FAKE + 4, wdt=1), "weight must be 16-byte aligned"),
])
def test_forward_rejects_bad_arguments_on_the_host(over, msg):
    rc = _fwd(**over)
    assert rc != _lib.HARP_QK_OK
    assert msg in harp_amd.load_abi().harp_qk_last_error().decode()


def test_backward_validation_and_workspace_size():
    lib = harp_amd.load_abi()
    st = _strides(8 * 64 * 128, 64, 8 * 64)
    rc = lib.harp_qk_rmsnorm_backward(FAKE, st, FAKE, st, None, 1, None, FAKE, st, None, 1, 1, 8, 64, 128,
                                      None, 0, None)
    assert rc == 1 and "rms is NULL" in lib.harp_qk_last_error().decode()
    # 1*8*64 rows -> 32 blocks of 16 rows (+ 1 group row), 128 floats each
    assert lib.harp_qk_backward_workspace_bytes(1, 8, 64, 128) == (32 + 1) * 128 * 4
    # capped at 2048 blocks (+ 32 groups of 64)
    assert lib.harp_qk_backward_workspace_bytes(1, 24, 8192, 128) == (2048 + 32) * 128 * 4
    assert lib.harp_qk_backward_workspace_bytes(1, 8, 64, 100) == 2 ** 64 - 1


def _qkv(over_outs=None, **over):
    """harp_qkv_project with valid-looking arguments (fake, aligned pointers)
    except for the given overrides; validation must fail before any launch."""
    lib = harp_amd.load_abi()
    outs = (_lib.QkvOut * 3)()
    for o in outs:
        o.weight, o.ld_weight, o.y, o.ld_y = FAKE, 256, FAKE, 256
        o.y_lin, o.norm_weight, o.norm_weight_dtype, o.eps, o.rms = None, FAKE, _lib.HARP_QK_BF16, 1e-6, None
    for i, kv in (over_outs or {}).items():
        for k, v in kv.items():
            setattr(outs[i], k, v)
    a = dict(x=FAKE, ldx=256, B=1, S=64, K=256, n_out=256, f=FAKE, fsb=0, fss=128, n_outs=3)
    a.update(over)
    rc = lib.harp_qkv_project(a["x"], a["ldx"], a["B"], a["S"], a["K"], a["n_out"], a["f"], a["fsb"], a["fss"],
                              outs, a["n_outs"], None)
    return rc, lib.harp_qk_last_error().decode()


@pytest.mark.parametrize(
    "over,outs_over,code,msg",
    [
        (dict(K=100), None, 2, "k_dim"),
        (dict(K=0), None, 2, "k_dim"),
        (dict(n_out=200), None, 2, "n_out"),
        (dict(x=FAKE + 2), None, 1, "x must"),
        (dict(ldx=128), None, 1, "ld_x"),
        (dict(ldx=260), None, 1, "ld_x"),
        (dict(B=0), None, 1, "batch"),
        (dict(n_outs=0), None, 1, "outs"),
        (dict(n_outs=4), None, 1, "outs"),
        (dict(fss=3), None, 1, "freqs"),
        ({}, {1: dict(weight=None)}, 1, "outs[1].weight"),
        ({}, {0: dict(ld_weight=100)}, 1, "ld_weight"),
        ({}, {2: dict(ld_y=128)}, 1, "ld_y"),
        ({}, {0: dict(y=FAKE + 8)}, 1, "outs[0].y"),
        ({}, {2: dict(norm_weight=None, y_lin=FAKE)}, 1, "y_lin and rms"),
        ({}, {1: dict(norm_weight_dtype=7)}, 1, "dtype"),
    ],
)
def test_qkv_project_rejects_bad_arguments_on_the_host(over, outs_over, code, msg):
    rc, err = _qkv(outs_over, **over)
    assert rc == code and msg in err, (rc, err)


def test_async_op_schemas_are_the_references():
    harp_amd.load_async_ops()
    for name, schema in REF_SCHEMAS.items():
        got = str(getattr(torch.ops.async_op, name).default._schema)
        assert got == "async_op::" + schema, got


def test_cpu_tensors_are_refused():
    harp_amd.load_async_ops()
    x = torch.zeros(1, 2, 3, 64, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="HIP device only"):
        torch.ops.async_op.rope_forward_impl(x, torch.zeros(3, 32, dtype=torch.complex64), x)


def test_namespace_is_shared_with_another_library():
    """The operators are a fragment of async_op: a library that defines the
    namespace's other operators (as the reference's own async_op library
    does for silu, tanh, add, ...) loads next to this one."""
    harp_amd.load_async_ops()
    other = torch.library.Library("async_op", "DEF")
    try:
        other.define("silu_out(Tensor input, Tensor(a!) output) -> ()")
        assert str(torch.ops.async_op.silu_out.default._schema).startswith("async_op::silu_out")
        assert str(torch.ops.async_op.rope_forward_impl.default._schema) == "async_op::" + REF_SCHEMAS["rope_forward_impl"]
    finally:
        other._destroy()


def test_attention_block_on_cpu_tensors_raises():
    """The block module has no CPU path either: its first GPU operator
    (the fused QK norm + RoPE) refuses CPU tensors."""
    from torch import nn

    attn = nn.Module()
    attn.heads = 2
    attn.to_q, attn.to_k, attn.to_v = (nn.Linear(128, 128, bias=False).to(torch.bfloat16) for _ in range(3))
    attn.to_out = nn.ModuleList([nn.Linear(128, 128, bias=False).to(torch.bfloat16)])
    norm = nn.Module()
    norm.weight = nn.Parameter(torch.ones(64, dtype=torch.bfloat16))
    norm.eps = 1e-5
    attn.norm_q = attn.norm_k = norm
    block = harp_amd.RingZAttention(attn, 2)
    x = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    freqs = torch.polar(torch.ones(32, 32), torch.zeros(32, 32))
    with pytest.raises(RuntimeError, match="HIP device only"):
        block(x, freqs)
    with pytest.raises(ValueError, match="multiple of sp_size"):
        harp_amd.RingZAttention(attn, 3)(x, freqs)


def test_qkv_project_validates_shapes_before_the_kernel():
    """harp_amd.qkv.qkv_project refuses CPU tensors and mismatched weights on
    the host: the kernel itself cannot see a weight's row count."""
    from harp_amd import qkv

    x = torch.zeros((1, 8, 128), dtype=torch.bfloat16)
    w = torch.zeros((256, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="HIP device"):
        qkv.qkv_project(x, [w, w, w], [(None, 0.0)] * 3, None)


class _DevView:
    """A CPU tensor that answers as a device tensor at a chosen address, so
    fused_supported's pointer and stride checks run without a GPU."""

    is_cuda = True
    device = "cuda:0"

    def __init__(self, t, addr=1 << 20):
        self.t, self.addr = t, addr

    dtype = property(lambda self: self.t.dtype)
    shape = property(lambda self: self.t.shape)

    def dim(self):
        return self.t.dim()

    def size(self, *a):
        return self.t.size(*a)

    def stride(self, *a):
        return self.t.stride(*a)

    def numel(self):
        return self.t.numel()

    def is_contiguous(self):
        return self.t.is_contiguous()

    def data_ptr(self):
        return self.addr


def _module(K=128, H=2, wq=None, nw=None):
    from types import SimpleNamespace

    n = H * 128
    lin = [SimpleNamespace(weight=_DevView(torch.zeros(n, K, dtype=torch.bfloat16)), bias=None) for _ in range(3)]
    if wq is not None:
        lin[0].weight = wq
    norm = SimpleNamespace(weight=nw if nw is not None else _DevView(torch.ones(128, dtype=torch.bfloat16)), eps=1e-6)
    return SimpleNamespace(heads=H, to_q=lin[0], to_k=lin[1], to_v=lin[2], norm_q=norm, norm_k=norm)


def test_fused_supported_mirrors_the_kernel_checks():
    """Everything harp_qkv_project refuses (weight leading dimension not a
    multiple of 8 or above 2^22, misaligned x / weight / norm weight, a
    strided norm weight) takes the unfused path instead of raising."""
    from harp_amd import qkv

    x = _DevView(torch.zeros(1, 16, 128, dtype=torch.bfloat16))
    assert qkv.fused_supported(_module(), x, None)
    # a misaligned hidden-state slice (contiguous: passed as is)
    assert not qkv.fused_supported(_module(), _DevView(x.t, (1 << 20) + 2), None)
    # a weight at an address that is not 16-byte aligned
    assert not qkv.fused_supported(_module(wq=_DevView(torch.zeros(256, 128, dtype=torch.bfloat16), (1 << 20) + 4)),
                                   x, None)
    # weight rows padded to a stride that is not a multiple of 8
    odd = torch.zeros(256, 131, dtype=torch.bfloat16)[:, :128]
    assert odd.stride(0) == 131
    assert not qkv.fused_supported(_module(wq=_DevView(odd)), x, None)
    ok8 = torch.zeros(256, 136, dtype=torch.bfloat16)[:, :128]
    assert qkv.fused_supported(_module(wq=_DevView(ok8)), x, None)
    # leading dimension above 2^22 elements
    huge = _DevView(torch.zeros(256, 128, dtype=torch.bfloat16))
    huge.stride = lambda *a: ((1 << 22) + 8, 1)[a[0]] if a else ((1 << 22) + 8, 1)
    assert not qkv.fused_supported(_module(wq=huge), x, None)
    # norm weight: misaligned, or a strided view
    assert not qkv.fused_supported(_module(nw=_DevView(torch.ones(128, dtype=torch.bfloat16), (1 << 20) + 2)), x,
                                   None)
    assert not qkv.fused_supported(_module(nw=_DevView(torch.ones(256, dtype=torch.bfloat16)[::2])), x, None)
