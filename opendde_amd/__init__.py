"""opendde_amd — MI355X (gfx950) backend for OpenDDE's Pairformer pair stack.

Drop-in modules with the reference's signatures, parameter names and
kernel-selection hook (``triangle_attention`` / ``triangle_multiplicative``
in {"torch", "hip", "cuequivariance" (alias of "hip")}); the accelerated path
runs hand-written HIP kernels through the C ABI in ``include/opendde_amd.h``.
"""

from .hook import (ACCELERATED, TRIANGLE_KERNELS, apply_runtime_compatibility,
                   get_hip_runtime_status, resolve_auto_triangle_kernels,
                   validate_triangle_kernels)
from .pairformer import (AttentionPairBias, PairformerBlock, PairformerStack,
                         Transition)
from .triangular import (Attention, TriangleAttention, TriangleMultiplicationIncoming,
                         TriangleMultiplicationOutgoing, TriangleMultiplicativeUpdate,
                         hip_triangular_attn, kernel_triangular_mult)

__version__ = "0.1.0"
