"""The fast LayerNorm extension's eight entry points, on the HIP library.

Same names, arguments, return values and checks as the reference's pybind
module ``fast_layer_norm_cuda_v2`` (opendde/model/layer_norm/kernel/
layer_norm_cuda.cpp:142-179, argument checks :22-71, output allocation
:73-121):

* ``forward_{none,with_bias,with_weight,with_both}_affine(input,
  normalized_shape, [gamma], [beta], epsilon)`` -> ``[output, mean, invvar]``
  with ``output`` like ``input`` and ``mean`` / ``invvar`` float32 ``[n1]``;
* ``backward_*_affine(dout, mean, invvar, input, normalized_shape, [gamma],
  [beta], epsilon)`` -> ``[grad_input, grad_gamma, grad_beta]``, each
  gradient of a parameter that was not passed being ``None``.

``n1`` is the product of the leading dims of ``input``, ``n2`` that of
``normalized_shape``.  Tensors must be on a GPU and contiguous; gamma, beta
and dout must match ``input``'s dtype (float32, bfloat16 or float16).  The
arithmetic runs in ``libopendde_amd.so`` (``odde_layer_norm_fwd`` /
``odde_layer_norm_bwd``) on the current stream; nothing here computes.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence, Tuple

import torch

from . import _lib

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16, torch.float16: _lib.F16}


def _check_input(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a CUDA tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def _n1_n2(input: torch.Tensor, normalized_shape: Sequence[int]) -> Tuple[int, int]:
    shape = tuple(int(s) for s in normalized_shape)
    if len(shape) < 1:
        raise RuntimeError("Expected normalized_shape to be at least 1-dimensional, i.e., "
                           f"containing at least one element, but got normalized_shape={list(shape)}")
    if input.dim() < len(shape) or tuple(input.shape[input.dim() - len(shape):]) != shape:
        raise RuntimeError(f"Given normalized_shape={list(shape)}, expected input with shape "
                           f"[*, {', '.join(str(s) for s in shape)}], but got input of size"
                           f"{list(input.shape)}")
    n2 = 1
    for s in shape:
        n2 *= s
    n1 = 1
    for s in input.shape[:input.dim() - len(shape)]:
        n1 *= int(s)
    if n2 <= 0:
        raise RuntimeError("LayerNorm over an empty normalized shape")
    return n1, n2


def _dtype_code(input: torch.Tensor) -> int:
    try:
        return _DTYPES[input.dtype]
    except KeyError:
        raise RuntimeError(f"fast LayerNorm supports float32, bfloat16 and float16, "
                           f"got {input.dtype}") from None


def _param(p: Optional[torch.Tensor], input: torch.Tensor, n2: int, name: str):
    if p is None:
        return None
    if p.device != input.device:
        raise RuntimeError(f"{name} must be on the input's device")
    if p.dtype != input.dtype:
        raise RuntimeError(f"{name} dtype {p.dtype} differs from the input's {input.dtype}")
    if p.numel() != n2:
        raise RuntimeError(f"{name} has {p.numel()} elements, expected {n2}")
    return p.contiguous()


def _ptr(t: Optional[torch.Tensor]) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr() if t is not None else 0)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def layer_norm_affine(input: torch.Tensor, normalized_shape, gamma: Optional[torch.Tensor],
                      beta: Optional[torch.Tensor], epsilon: float) -> List[torch.Tensor]:
    """Forward: ``[output, mean, invvar]`` (layer_norm_cuda.cpp:73-90)."""
    _check_input(input, "input")
    n1, n2 = _n1_n2(input, normalized_shape)
    dt = _dtype_code(input)
    gamma = _param(gamma, input, n2, "gamma")
    beta = _param(beta, input, n2, "beta")
    output = torch.empty_like(input)
    mean = torch.empty((n1,), dtype=torch.float32, device=input.device)
    invvar = torch.empty_like(mean)
    a = _lib.LayerNormArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype, a.n1, a.n2, a.eps = dt, n1, n2, float(epsilon)
    a.x, a.gamma, a.beta = _ptr(input), _ptr(gamma), _ptr(beta)
    a.out, a.mean, a.invvar = _ptr(output), _ptr(mean), _ptr(invvar)
    lib = _lib.load()
    with torch.cuda.device(input.device):
        _lib.check(lib.odde_layer_norm_fwd(ctypes.byref(a), _stream(input.device)),
                   "odde_layer_norm_fwd")
    return [output, mean, invvar]


def layer_norm_gradient_affine(dout: torch.Tensor, mean: torch.Tensor, invvar: torch.Tensor,
                               input: torch.Tensor, normalized_shape,
                               gamma: Optional[torch.Tensor], beta: Optional[torch.Tensor],
                               epsilon: float) -> List[Optional[torch.Tensor]]:
    """Backward: ``[grad_input, grad_gamma, grad_beta]`` (layer_norm_cuda.cpp:
    99-139); ``grad_gamma`` exists when gamma was passed, ``grad_beta`` when
    beta was."""
    for t, name in ((dout, "dout"), (mean, "mean"), (invvar, "invvar"), (input, "input")):
        _check_input(t, name)
    n1, n2 = _n1_n2(input, normalized_shape)
    dt = _dtype_code(input)
    if dout.shape != input.shape or dout.dtype != input.dtype:
        raise RuntimeError("dout must have the input's shape and dtype")
    for t, name in ((mean, "mean"), (invvar, "invvar")):
        if t.dtype != torch.float32 or t.numel() != n1:
            raise RuntimeError(f"{name} must be float32 with {n1} elements")
    gamma = _param(gamma, input, n2, "gamma")
    beta = _param(beta, input, n2, "beta")
    grad_input = torch.empty_like(input)
    grad_gamma = torch.empty_like(gamma) if gamma is not None else None
    grad_beta = torch.empty_like(beta) if beta is not None else None
    a = _lib.LayerNormBwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype, a.n1, a.n2 = dt, n1, n2
    a.dout, a.mean, a.invvar, a.x = _ptr(dout), _ptr(mean), _ptr(invvar), _ptr(input)
    a.gamma = _ptr(gamma)
    a.grad_input, a.grad_gamma, a.grad_beta = _ptr(grad_input), _ptr(grad_gamma), _ptr(grad_beta)
    lib = _lib.load()
    ws = None
    if grad_gamma is not None or grad_beta is not None:
        nb = ctypes.c_uint64(0)
        _lib.check(lib.odde_layer_norm_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)),
                   "odde_layer_norm_bwd_workspace_bytes")
        # torch's caching allocator returns 256-byte aligned blocks
        ws = torch.empty(max(int(nb.value), 256), dtype=torch.uint8, device=input.device)
        a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
    with torch.cuda.device(input.device):
        _lib.check(lib.odde_layer_norm_bwd(ctypes.byref(a), _stream(input.device)),
                   "odde_layer_norm_bwd")
    return [grad_input, grad_gamma, grad_beta]


# ------------------------------------------------ the eight named entry points


def forward_none_affine(input, normalized_shape, epsilon):
    return layer_norm_affine(input, normalized_shape, None, None, epsilon)


def forward_with_bias_affine(input, normalized_shape, beta, epsilon):
    return layer_norm_affine(input, normalized_shape, None, beta, epsilon)


def forward_with_weight_affine(input, normalized_shape, gamma, epsilon):
    return layer_norm_affine(input, normalized_shape, gamma, None, epsilon)


def forward_with_both_affine(input, normalized_shape, gamma, beta, epsilon):
    return layer_norm_affine(input, normalized_shape, gamma, beta, epsilon)


def backward_none_affine(dout, mean, invvar, input, normalized_shape, epsilon):
    return layer_norm_gradient_affine(dout, mean, invvar, input, normalized_shape, None, None,
                                      epsilon)


def backward_with_bias_affine(dout, mean, invvar, input, normalized_shape, beta, epsilon):
    return layer_norm_gradient_affine(dout, mean, invvar, input, normalized_shape, None, beta,
                                      epsilon)


def backward_with_weight_affine(dout, mean, invvar, input, normalized_shape, gamma, epsilon):
    return layer_norm_gradient_affine(dout, mean, invvar, input, normalized_shape, gamma, None,
                                      epsilon)


def backward_with_both_affine(dout, mean, invvar, input, normalized_shape, gamma, beta, epsilon):
    return layer_norm_gradient_affine(dout, mean, invvar, input, normalized_shape, gamma, beta,
                                      epsilon)
