"""CPU tests of the boundary: the C-ABI library loads and exports every
function include/harp_ring_attn.h declares, validates arguments on the host
before touching a device, sizes its workspace, and the operator library
registers the reference's schemas (no GPU needed)."""

import ctypes
import math
import os
import re
import subprocess

import pytest
import torch

import harp_amd
from harp_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "harp_ring_attn.h")

REF_FWD_SCHEMA = ("ring_attention_forward(Tensor q, Tensor k, Tensor v, Tensor(a!) out, Tensor(b!) m_i, "
                  "Tensor(c!) l_i, int sp_size, float scale")
REF_BWD_SCHEMA = ("ring_attention_backward(Tensor q, Tensor(a!) grad_q, Tensor k, Tensor(b!) dK, Tensor v, "
                  "Tensor(c!) dV, Tensor grad_out, Tensor m_i, Tensor l_i, Tensor D, int sp_size, float scale")


def header_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"HARP_RA_API\s+[\w\s\*]+?\b(harp_ra_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    fns = header_functions()
    for name in ("harp_ra_forward", "harp_ra_backward", "harp_ra_delta"):
        assert name in fns
    assert set(fns) == set(_lib.ABI_PROTOTYPES), "ctypes prototypes must cover exactly the header"


def test_library_exports_every_declared_symbol():
    lib = harp_amd.load_abi()
    for name in header_functions():
        assert hasattr(lib, name), name
    nm = subprocess.run(["nm", "-D", "--defined-only", str(_lib.ABI_LIB)], capture_output=True, text=True)
    exported = {ln.split()[-1] for ln in nm.stdout.splitlines() if " T " in ln}
    ours = {s for s in exported if s.startswith("harp_ra_")}
    assert ours == set(header_functions()), ours ^ set(header_functions())
    assert lib.harp_ra_version().decode().startswith("harp_ra")


def _fwd_call(**over):
    lib = harp_amd.load_abi()
    st = _lib.i64_array([8 * 64 * 128, 64, 8 * 64, 1])
    fake = 1 << 20  # never dereferenced: validation fails first
    a = dict(q=fake, qs=st, kc=_lib.ptr_array([fake]), vc=_lib.ptr_array([fake]), ks=st, tc=128, lens=None,
             out=fake, os=st, m=fake, mdt=_lib.HARP_RA_BF16, l=fake, B=1, H=8, T=128, D=64, sp=1, rank=0,
             scale=0.125, ws=fake, wsb=1 << 30, stream=None)
    a.update(over)
    return lib.harp_ra_forward(a["q"], a["qs"], a["kc"], a["vc"], a["ks"], a["tc"], a["lens"], a["out"], a["os"],
                               a["m"], a["mdt"], a["l"], a["B"], a["H"], a["T"], a["D"], a["sp"], a["rank"],
                               a["scale"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize(
    "over,code,msg",
    [
        (dict(T=0), _lib.HARP_RA_EINVAL, "sizes must be positive"),
        (dict(D=60), _lib.HARP_RA_EUNSUPPORTED, "multiple of 8"),
        (dict(D=136), _lib.HARP_RA_EUNSUPPORTED, "> 128"),
        (dict(sp=0), _lib.HARP_RA_EINVAL, "sp_size"),
        (dict(sp=17), _lib.HARP_RA_EINVAL, "sp_size"),
        (dict(rank=1), _lib.HARP_RA_EINVAL, "ring_rank"),
        (dict(q=None), _lib.HARP_RA_EINVAL, "q is NULL"),
        (dict(q=(1 << 20) + 2), _lib.HARP_RA_EINVAL, "16-byte aligned"),
        (dict(qs=_lib.i64_array([8 * 64 * 128, 64, 8 * 64, 2])), _lib.HARP_RA_EINVAL, "unit stride"),
        (dict(qs=_lib.i64_array([8 * 64 * 128, 60, 8 * 64, 1])), _lib.HARP_RA_EINVAL, "multiple of 8"),
        (dict(lens=_lib.i32_array([129])), _lib.HARP_RA_EINVAL, "kv_valid_lens"),
        (dict(mdt=7), _lib.HARP_RA_EINVAL, "m_i_dtype"),
        (dict(scale=float("nan")), _lib.HARP_RA_EINVAL, "scale"),
        (dict(scale=-0.125), _lib.HARP_RA_EINVAL, "positive"),
        # a row stride of 0 (an expanded view) or below D would cut every row short
        (dict(ks=_lib.i64_array([8 * 64 * 128, 64, 0, 1])), _lib.HARP_RA_EINVAL, "row stride"),
        (dict(qs=_lib.i64_array([8 * 64 * 128, 64, 56, 1])), _lib.HARP_RA_EINVAL, "row stride"),
        # a short chunk whose rows lie 32 MiB apart: a 128-row tile's copy
        # offsets would pass 2^32 (the extent counts at least 128 rows)
        (dict(ks=_lib.i64_array([8 * 64 * 128, 64, 1 << 24, 1]), tc=16), _lib.HARP_RA_EUNSUPPORTED, "buffer range"),
        # outputs whose strides alias elements are refused (stores would race)
        (dict(os=_lib.i64_array([8 * 64 * 128, 64, 0, 1])), _lib.HARP_RA_EINVAL, "overlap"),
        (dict(os=_lib.i64_array([8 * 64 * 128, 0, 8 * 64, 1])), _lib.HARP_RA_EINVAL, "overlap"),
        (dict(os=_lib.i64_array([8 * 64 * 128, 32, 8 * 64, 1])), _lib.HARP_RA_EINVAL, "overlap"),
    ],
)
def test_forward_rejects_bad_arguments_before_any_device_call(over, code, msg):
    rc = _fwd_call(**over)
    assert rc == code
    assert msg in _lib.last_error()


def test_workspace_sizes():
    # the forward stages everything in LDS; the backward keeps two fp32
    # statistics planes of B*H*T rows, rounded up to 256 bytes
    # (no device here: KV splits, which depend on the device's CU count, are off)
    assert harp_amd.forward_workspace_bytes(1, 24, 8192, 128, 8, 8192) == 0
    assert harp_amd.backward_workspace_bytes(1, 24, 8192, 128, 8, 8192) == 2 * 4 * 24 * 8192
    assert harp_amd.backward_workspace_bytes(1, 1, 33, 64, 1, 64) == 512
    assert harp_amd.forward_workspace_bytes(2, 16, 4429, 72, 4, 4480, [4429] * 4) == 0
    with pytest.raises(ValueError, match="sp_size"):
        harp_amd.forward_workspace_bytes(1, 1, 64, 64, 0, 64)
    with pytest.raises(ValueError, match="multiple of 8"):
        harp_amd.forward_workspace_bytes(1, 1, 64, 66, 1, 64)


def test_timing_read_validates_arguments():
    lib = harp_amd.load_abi()
    assert lib.harp_ra_timing_read(None, None, 5) == _lib.HARP_RA_EINVAL
    assert lib.harp_ra_timing_enable(0) == _lib.HARP_RA_OK
    t = _lib.timing_read()
    assert set(t) == set(_lib.KERNEL_KINDS) and all(v == (0.0, 0) for v in t.values())


def test_operator_library_registers_reference_schemas():
    harp_amd.load_ops()
    f = str(torch.ops.ring_attention_ops.ring_attention_forward.default._schema)
    b = str(torch.ops.ring_attention_ops.ring_attention_backward.default._schema)
    assert f.startswith("ring_attention_ops::" + REF_FWD_SCHEMA)
    assert b.startswith("ring_attention_ops::" + REF_BWD_SCHEMA)
    # reference positional calls stay valid: only defaulted trailing args were added
    tail = "int ring_rank=0, int[]? kv_lens=None, int kv_chunk_len=0) -> (Tensor(a!), Tensor(b!), Tensor(c!))"
    assert f.endswith(tail)
    assert b.endswith(tail)


def test_cpu_tensors_raise_instead_of_falling_back():
    harp_amd.load_ops()
    q = torch.zeros(1, 2, 16, 64, dtype=torch.bfloat16)
    out = torch.zeros(1, 2, 16, 64)
    m = torch.zeros(1, 2, 16, 1, dtype=torch.bfloat16)
    l = torch.zeros(1, 2, 16, 1)
    with pytest.raises(RuntimeError, match="no CPU path"):
        torch.ops.ring_attention_ops.ring_attention_forward(q, q, q, out, m, l, 1, 0.125)
    with pytest.raises(RuntimeError, match="no CPU path"):
        torch.ops.ring_attention_ops.ring_attention_delta(q, out)
    with pytest.raises(RuntimeError, match="no CPU path"):
        torch.ops.ring_attention_ops.ring_attention_backward(q, q, q, q, q, q, q, l, l, l, 1, 0.125)


def test_product_package_never_imports_the_oracle():
    pkg = os.path.join(ROOT, "harp_amd")
    for dirpath, _, files in os.walk(pkg):
        for fn in files:
            if fn.endswith((".py", ".cpp", ".hip", ".h")):
                text = open(os.path.join(dirpath, fn)).read()
                assert "oracle" not in text.replace("oracle/", "").lower() or fn == "build.py", fn


_ST128 = _lib.i64_array([8 * 128 * 128, 128, 8 * 128, 1])


def _bwd_call(**over):
    lib = harp_amd.load_abi()
    st = _lib.i64_array([8 * 64 * 128, 64, 8 * 64, 1])
    fake = 1 << 20  # never dereferenced: validation fails first
    a = dict(q=fake, qs=st, dq=fake, dqs=st, dqt=_lib.HARP_RA_BF16, kc=_lib.ptr_array([fake]),
             vc=_lib.ptr_array([fake]), ks=st, dkc=_lib.ptr_array([fake]), dvc=_lib.ptr_array([fake]), dks=st,
             dkt=_lib.HARP_RA_BF16, tc=128, lens=None, do=fake, dos=st, m=fake, mdt=_lib.HARP_RA_BF16, l=fake,
             d=fake, B=1, H=8, T=128, D=64, sp=1, rank=0, scale=0.125, ws=None, wsb=0, stream=None)
    a.update(over)
    return lib.harp_ra_backward(a["q"], a["qs"], a["dq"], a["dqs"], a["dqt"], a["kc"], a["vc"], a["ks"], a["dkc"],
                                a["dvc"], a["dks"], a["dkt"], a["tc"], a["lens"], a["do"], a["dos"], a["m"],
                                a["mdt"], a["l"], a["d"], a["B"], a["H"], a["T"], a["D"], a["sp"], a["rank"],
                                a["scale"], a["ws"], a["wsb"], a["stream"])


@pytest.mark.parametrize(
    "over,msg",
    [
        (dict(dos=_lib.i64_array([8 * 64 * 128, 64, 0, 1])), "grad_out row stride"),
        (dict(ks=_lib.i64_array([0, 0, 0, 1])), "k chunk row stride"),
        (dict(dqs=_lib.i64_array([8 * 64 * 128, 64, 0, 1])), "grad_q strides make elements overlap"),
        (dict(dks=_lib.i64_array([8 * 64 * 128, 0, 8 * 64, 1])), "dK chunk strides make elements overlap"),
        # bf16 dK / dV rows at head dim 128 are stored 8 bytes per lane
        (dict(D=128, qs=_ST128, dqs=_ST128, ks=_ST128, dos=_ST128,
              dks=_lib.i64_array([8 * 130 * 128, 130, 8 * 130, 1])), "must be a multiple of 4 elements"),
        (dict(D=128, qs=_ST128, dqs=_ST128, ks=_ST128, dos=_ST128, dks=_ST128,
              dkc=_lib.ptr_array([(1 << 20) + 2])), "must be 8-byte aligned"),
        # and so are bf16 dQ rows
        (dict(D=128, qs=_ST128, ks=_ST128, dos=_ST128, dks=_ST128,
              dqs=_lib.i64_array([8 * 130 * 128, 130, 8 * 130, 1])), "grad_q stride[1]=130 must be a multiple"),
        (dict(D=128, qs=_ST128, dqs=_ST128, ks=_ST128, dos=_ST128, dks=_ST128, dq=(1 << 20) + 2),
         "bf16 grad_q must be 8-byte aligned"),
    ],
)
def test_backward_rejects_degenerate_strides(over, msg):
    assert _bwd_call(**over) == _lib.HARP_RA_EINVAL
    assert msg in _lib.last_error()


@pytest.mark.parametrize("dkt", [_lib.HARP_RA_BF16, _lib.HARP_RA_F32])
def test_backward_unaligned_dkdv_views_pass_validation_below_head_dim_128(dkt):
    """The dK / dV kernel for head dims other than 128 stores element by
    element, so bf16 (and fp32) dK / dV views at an odd element offset with
    an odd row stride are accepted there: validation gets past them to the
    statistics check (m_i NULL here, so nothing is launched)."""
    odd = _lib.i64_array([8 * 65 * 128, 65, 8 * 65, 1])
    rc = _bwd_call(dkc=_lib.ptr_array([(1 << 20) + 2]), dvc=_lib.ptr_array([(1 << 21) + 2]), dks=odd, dkt=dkt,
                   m=None)
    assert rc == _lib.HARP_RA_EINVAL
    assert "m_i / l_i / delta are NULL" in _lib.last_error()


def _cpu_qkv(T=16, Tk=16, H=2, D=64):
    q = torch.zeros(1, H, T, D, dtype=torch.bfloat16)
    k = torch.zeros(1, H, Tk, D, dtype=torch.bfloat16)
    out = torch.zeros(1, H, T, D)
    m = torch.zeros(1, H, T, 1, dtype=torch.bfloat16)
    l = torch.zeros(1, H, T, 1)
    return q, k, out, m, l


def test_reference_local_only_call_is_rejected():
    """HARP's own call (attn.py:29): k / v hold only the local chunk while
    sp_size > 1.  One GPU has no peers to take the other chunks from, so the
    operator refuses it rather than attending over the local keys only."""
    harp_amd.load_ops()
    ops = torch.ops.ring_attention_ops
    q, k, out, m, l = _cpu_qkv(T=16, Tk=16)
    with pytest.raises(RuntimeError, match="hold only the local chunk"):
        ops.ring_attention_forward(q, k, k, out, m, l, 4, 0.125)
    with pytest.raises(RuntimeError, match="hold only the local chunk"):
        ops.ring_attention_backward(q, q, k, k, k, k, q, l, l, l, 4, 0.125)


@pytest.mark.parametrize(
    "Tk,sp,lens,chunk,expect",
    [
        (64, 4, None, 0, "no CPU path"),        # all sp_size chunks of q's length: accepted
        (40, 1, None, 0, "no CPU path"),        # sp_size 1: k is the one chunk, any length
        (48, 4, None, 0, "does not match"),     # neither pattern: refused without kv_chunk_len
        (48, 4, None, 12, "no CPU path"),       # explicit chunk length: accepted
        (48, 4, None, 16, "must equal sp_size"),
        (48, 4, [12, 12, 10, 0], 0, "no CPU path"),  # kv_lens opts in to k.size(2) / sp_size
        (50, 4, [12, 12, 10, 0], 0, "not a multiple"),
    ],
)
def test_chunk_layout_contract(Tk, sp, lens, chunk, expect):
    """Which k / v shapes the operator accepts; the CPU key checks the layout
    before it refuses CPU tensors, so these run without a GPU."""
    harp_amd.load_ops()
    q, k, out, m, l = _cpu_qkv(T=16, Tk=Tk)
    with pytest.raises(RuntimeError, match=expect):
        torch.ops.ring_attention_ops.ring_attention_forward(q, k, k, out, m, l, sp, 0.125, 0, lens, chunk)
    with pytest.raises(RuntimeError, match=expect):
        torch.ops.ring_attention_ops.ring_attention_backward(q, q, k, k, k, k, q, l, l, l, sp, 0.125, 0, lens, chunk)


def test_autograd_function_rejects_ragged_concatenation():
    with pytest.raises(ValueError, match="not a multiple of sp_size"):
        harp_amd.RingAttention.apply(torch.zeros(1, 1, 8, 64), torch.zeros(1, 1, 10, 64), torch.zeros(1, 1, 10, 64), 4)
