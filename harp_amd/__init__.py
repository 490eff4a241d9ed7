"""harp_amd — MI355X (gfx950) ring-attention block for HARP's sequence-parallel attention.

Drop-in for HARP's ``libring_attention_ops.so`` (namespace ``ring_attention_ops``):
hand-written HIP kernels behind the C ABI of ``include/harp_ring_attn.h``
(``kernels/libharp_ra.so``) and a PyTorch-ROCm operator library
(``kernels/libring_attention_ops.so``).  The step before it, QK RMSNorm and the
rotary embedding, runs on the GPU too (``include/harp_qk_norm_rope.h``,
``kernels/libharp_async_op.so``, namespace ``async_op``), and
:class:`RingZAttention` wires projections, QK norm, RoPE, ring attention and
the output projection as the model's attention block does.  Build with
``python -m harp_amd.build``.
"""

from ._lib import ABI_LIB, ASYNC_OPS_LIB, OPS_LIB, load_abi, load_async_ops, load_ops  # noqa: F401
from .ops import (  # noqa: F401
    RingAttention,
    abi_backward,
    abi_delta,
    abi_forward,
    backward_workspace_bytes,
    concat_chunks,
    forward_workspace_bytes,
    ring_attention,
)
from .qk import ApplyRotaryComplexFn, QKNormRopeFn, RMSNormFn  # noqa: F401
from .attention import RingZAttention, project_qkv  # noqa: F401
from .wait_engine import CommWork, WaitEngine  # noqa: F401
from .gemm import xhblas_gemm  # noqa: F401

__version__ = "0.1.0"
