"""FusedLayerNorm: the reference's optional fast LayerNorm module, on HIP.

Mirrors opendde/model/layer_norm/layer_norm.py:
* ``_FAST_LAYER_NORM_REQUIRED_SYMBOLS`` and the validation of a loaded
  extension (:31-58);
* ``_load_fast_layer_norm_cuda_v2()`` and the module global
  ``fast_layer_norm_cuda_v2``: lazy, lock-protected, cached load, including a
  cached failure logged once (:61-108); the reference's own names, which its
  tests patch and reset.  Without a GPU it returns ``None`` and
  does not mark the load as attempted.  The extension here is
  ``opendde_amd.fast_layer_norm`` over ``libopendde_amd.so``; nothing is
  compiled at run time;
* ``FusedLayerNormAffineFunction`` (:111-230): the eight-entry-point dispatch
  on which of weight / bias exist, parameters cast to the input's (forward)
  or gradient's (backward) dtype, one gradient returned per input;
* ``FusedLayerNorm`` (:233-288): ``weight`` / ``bias`` parameters (ones /
  zeros), ``F.layer_norm`` for CPU tensors.

One deliberate difference: when the library is unusable and a GPU tensor
arrives, the reference warns and falls back to ``F.layer_norm``; here the
call raises with the cached load error, so a run that selected the fast
LayerNorm never silently computes with torch instead.
"""

from __future__ import annotations

import importlib
import logging
import numbers
import threading
from typing import Any, Optional, Union

import torch
import torch.nn.functional as F
from torch.nn.parameter import Parameter

logger = logging.getLogger(__name__)

_FAST_LAYER_NORM_REQUIRED_SYMBOLS = (
    "forward_none_affine",
    "forward_with_bias_affine",
    "forward_with_weight_affine",
    "forward_with_both_affine",
    "backward_none_affine",
    "backward_with_bias_affine",
    "backward_with_weight_affine",
    "backward_with_both_affine",
)

fast_layer_norm_cuda_v2: Any = None  # the loaded extension (the reference's name)
_fast_layer_norm_load_attempted = False
_fast_layer_norm_load_error: Optional[BaseException] = None
_fast_layer_norm_load_lock = threading.Lock()


def _validate_fast_layer_norm_extension(extension: Any) -> Any:
    missing = [s for s in _FAST_LAYER_NORM_REQUIRED_SYMBOLS
               if not callable(getattr(extension, s, None))]
    if missing:
        raise ImportError("Fast LayerNorm extension is missing required symbols: "
                          + ", ".join(missing))
    return extension


def _load_fast_layer_norm_cuda_v2() -> Any:
    """The validated extension module, or ``None`` (no GPU, or load failed)."""
    global fast_layer_norm_cuda_v2, _fast_layer_norm_load_attempted, _fast_layer_norm_load_error
    if not torch.cuda.is_available():
        return None
    if _fast_layer_norm_load_attempted:
        return fast_layer_norm_cuda_v2
    with _fast_layer_norm_load_lock:
        if _fast_layer_norm_load_attempted:
            return fast_layer_norm_cuda_v2
        try:
            extension = importlib.import_module(".fast_layer_norm", package=__package__)
            extension = _validate_fast_layer_norm_extension(extension)
            from . import _lib
            _lib.load()  # the entry points are only usable with the library
        except Exception as error:  # noqa: BLE001 - cached, logged once, re-raised on use
            logger.warning("Fast LayerNorm HIP library is unavailable: %s", error)
            _fast_layer_norm_load_error = error
            extension = None
        fast_layer_norm_cuda_v2 = extension
        _fast_layer_norm_load_attempted = True
        return extension


def _reset_loader_for_tests() -> None:
    global fast_layer_norm_cuda_v2, _fast_layer_norm_load_attempted, _fast_layer_norm_load_error
    with _fast_layer_norm_load_lock:
        fast_layer_norm_cuda_v2 = None
        _fast_layer_norm_load_attempted = False
        _fast_layer_norm_load_error = None


class FusedLayerNormAffineFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, input: torch.Tensor, weight: Optional[torch.Tensor],
                bias: Optional[torch.Tensor], normalized_shape: torch.Size,
                eps: float) -> torch.Tensor:
        d = input.dtype
        ext = fast_layer_norm_cuda_v2
        ctx.normalized_shape = normalized_shape
        ctx.eps = eps
        input_ = input.contiguous()
        if weight is None:
            if bias is None:
                output, mean, invvar = ext.forward_none_affine(input_, normalized_shape, eps)
            else:
                output, mean, invvar = ext.forward_with_bias_affine(
                    input_, normalized_shape, bias.to(d), eps)
        elif bias is None:
            output, mean, invvar = ext.forward_with_weight_affine(
                input_, normalized_shape, weight.to(d), eps)
        else:
            output, mean, invvar = ext.forward_with_both_affine(
                input_, normalized_shape, weight.to(d), bias.to(d), eps)
        ctx.save_for_backward(input_, weight, bias, mean, invvar)
        return output

    @staticmethod
    def backward(ctx: Any, *grad_outputs: Any):
        (grad_output,) = grad_outputs
        d = grad_output.dtype
        ext = fast_layer_norm_cuda_v2
        input_, weight_, bias_, mean, invvar = ctx.saved_tensors
        g = grad_output.contiguous()
        shape, eps = ctx.normalized_shape, ctx.eps
        if weight_ is None:
            if bias_ is None:
                grad_input, grad_weight, grad_bias = ext.backward_none_affine(
                    g, mean, invvar, input_, shape, eps)
            else:
                grad_input, grad_weight, grad_bias = ext.backward_with_bias_affine(
                    g, mean, invvar, input_, shape, bias_.to(dtype=d), eps)
        elif bias_ is None:
            grad_input, grad_weight, grad_bias = ext.backward_with_weight_affine(
                g, mean, invvar, input_, shape, weight_.to(dtype=d), eps)
        else:
            grad_input, grad_weight, grad_bias = ext.backward_with_both_affine(
                g, mean, invvar, input_, shape, weight_.to(dtype=d), bias_.to(dtype=d), eps)
        return (grad_input,
                None if weight_ is None else grad_weight,
                None if bias_ is None else grad_bias,
                None, None)


class FusedLayerNorm(torch.nn.Module):
    """LayerNorm over ``normalized_shape`` with optional scale (``weight``) and
    offset (``bias``); eps 1e-5 by default."""

    def __init__(self, normalized_shape: Union[int, list, torch.Size], create_scale: bool = True,
                 create_offset: bool = True, eps: float = 1e-5) -> None:
        super().__init__()
        if isinstance(normalized_shape, numbers.Integral):
            shape = (int(normalized_shape),)
        else:
            shape = tuple(normalized_shape)
        self.normalized_shape = torch.Size(shape)
        self.eps = eps
        self.weight = Parameter(torch.ones(*self.normalized_shape)) if create_scale else None
        self.bias = Parameter(torch.zeros(*self.normalized_shape)) if create_offset else None
        self.reset_parameters()

    def reset_parameters(self) -> None:
        if self.weight is not None:
            torch.nn.init.ones_(self.weight)
        if self.bias is not None:
            torch.nn.init.zeros_(self.bias)

    def forward(self, input: torch.Tensor) -> torch.Tensor:
        if not input.is_cuda:
            return F.layer_norm(input, self.normalized_shape, self.weight, self.bias, self.eps)
        if _load_fast_layer_norm_cuda_v2() is None:
            raise RuntimeError("fast LayerNorm was selected but the HIP library is unusable: "
                               f"{_fast_layer_norm_load_error}")
        return FusedLayerNormAffineFunction.apply(input, self.weight, self.bias,
                                                  self.normalized_shape, self.eps)
