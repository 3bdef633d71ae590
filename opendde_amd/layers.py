"""Linear / LayerNorm layers with the reference's parameter names and dtype
rules (opendde/model/triangular/layers.py:128-282, modules/primitives.py:24-93).

These carry the checkpoint contract (``weight`` / ``bias`` names and shapes)
and the "torch" kernel value's arithmetic; the HIP backend reads their
parameters directly.
"""

from __future__ import annotations

import math
import os
from functools import partial
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .kernels import prepared

# LayerNorm selection, read once at import as the reference does
# (layers.py:24-29).
_use_fast_layer_norm = os.getenv("LAYERNORM_TYPE", "torch") == "fast_layernorm"
if _use_fast_layer_norm:
    try:
        from .layer_norm import FusedLayerNorm
    except (ImportError, OSError, RuntimeError):
        _use_fast_layer_norm = False

# std of a standard normal truncated to [-2, 2]:
# var = 1 - 2*2*phi(2) / (Phi(2) - Phi(-2))
_PHI2 = math.exp(-2.0) / math.sqrt(2.0 * math.pi)
_Z = math.erf(2.0 / math.sqrt(2.0))
TRUNC_STD = math.sqrt(1.0 - 4.0 * _PHI2 / _Z)


def trunc_normal_init_(weight: torch.Tensor, scale: float = 1.0) -> None:
    """Fan-in truncated normal on [-2 std, 2 std] (LeCun for scale 1, He for 2)."""
    fan_in = max(1, weight.shape[1])
    std = math.sqrt(scale / fan_in) / TRUNC_STD
    with torch.no_grad():
        nn.init.trunc_normal_(weight, mean=0.0, std=std, a=-2 * std, b=2 * std)


class OpenfoldLinear(nn.Linear):
    """nn.Linear with the reference's init strings ("default", "relu",
    "glorot", "gating", "normal", "final") and bf16 rule: a bf16 input runs a
    bf16 linear with the weight cast to bf16 (layers.py:128-223)."""

    def __init__(self, in_dim: int, out_dim: int, bias: bool = True, init: str = "default",
                 init_fn=None, precision: Optional[torch.dtype] = None):
        super().__init__(in_dim, out_dim, bias=bias)
        with torch.no_grad():
            if bias:
                self.bias.fill_(0)
            if init_fn is not None:
                init_fn(self.weight, self.bias)
            elif init == "default":
                trunc_normal_init_(self.weight, 1.0)
            elif init == "relu":
                trunc_normal_init_(self.weight, 2.0)
            elif init == "glorot":
                nn.init.xavier_uniform_(self.weight, gain=1)
            elif init == "gating":
                self.weight.fill_(0.0)
                if bias:
                    self.bias.fill_(1.0)
            elif init == "normal":
                nn.init.kaiming_normal_(self.weight, nonlinearity="linear")
            elif init == "final":
                self.weight.fill_(0.0)
            else:
                raise ValueError("Invalid init string.")
        self.precision = precision

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        d = x.dtype
        if self.precision is not None:
            with torch.amp.autocast("cuda", enabled=False):
                b = self.bias.to(self.precision) if self.bias is not None else None
                return F.linear(x.to(self.precision), self.weight.to(self.precision), b).to(d)
        if d is torch.bfloat16:
            with torch.amp.autocast("cuda", enabled=False):
                b = self.bias.to(d) if self.bias is not None else None
                return F.linear(x, self.weight.to(d), b)
        return F.linear(x, self.weight, self.bias)


class OpenFoldLayerNorm(nn.Module):
    """LayerNorm over the last dim, eps 1e-5; a bf16 input runs in bf16 with
    the affine parameters cast (layers.py:226-269)."""

    def __init__(self, c_in: int, create_scale: bool = True, create_offset: bool = True,
                 eps: float = 1e-5):
        super().__init__()
        self.c_in = (c_in,)
        self.eps = eps
        if create_scale:
            self.weight = nn.Parameter(torch.ones(c_in))
        else:
            self.register_parameter("weight", None)
        if create_offset:
            self.bias = nn.Parameter(torch.zeros(c_in))
        else:
            self.register_parameter("bias", None)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        d = x.dtype
        if d is torch.bfloat16:
            with torch.amp.autocast("cuda", enabled=False):
                w = self.weight.to(d) if self.weight is not None else None
                b = self.bias.to(d) if self.bias is not None else None
                return F.layer_norm(x, self.c_in, w, b, self.eps)
        return F.layer_norm(x, self.c_in, self.weight, self.bias, self.eps)


def LayerNorm(c_in: int, create_scale: bool = True, create_offset: bool = True,
              eps: float = 1e-5) -> nn.Module:
    """Factory of the reference (layers.py:272-282): the HIP ``FusedLayerNorm``
    when ``LAYERNORM_TYPE=fast_layernorm`` was set at import, else
    ``OpenFoldLayerNorm``.  Both carry ``weight`` / ``bias`` / ``eps``."""
    if _use_fast_layer_norm:
        return FusedLayerNorm(c_in, create_scale=create_scale, create_offset=create_offset,
                              eps=eps)
    return OpenFoldLayerNorm(c_in, create_scale, create_offset, eps)


class Linear(nn.Linear):
    """primitives.Linear: zero bias, truncated-normal / zero weight init
    (modules/primitives.py:24-90)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True,
                 precision: Optional[torch.dtype] = None, initializer: str = "default", **kw):
        self.use_bias = bias
        self.precision = precision
        self.initializer = initializer
        super().__init__(in_features, out_features, bias=bias, **kw)
        with torch.no_grad():
            if bias:
                nn.init.zeros_(self.bias)
            if initializer == "default":
                trunc_normal_init_(self.weight, 1.0)
            elif initializer == "relu":
                trunc_normal_init_(self.weight, 2.0)
            elif initializer == "zeros":
                nn.init.zeros_(self.weight)
            else:
                raise ValueError(f"Invalid initializer: {initializer}.")

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.precision is not None:
            d = x.dtype
            with torch.amp.autocast("cuda", enabled=False):
                b = self.bias.to(self.precision) if self.bias is not None else None
                return F.linear(x.to(self.precision), self.weight.to(self.precision), b).to(d)
        if x.is_cuda and _bf16_autocast(x) and not self._needs_grad():
            # what bf16 autocast does for F.linear (input, weight and bias in
            # bf16, bf16 result), with the weight and bias cast once per
            # version instead of on every call; the cached copies are
            # detached, so a call that trains the parameters takes F.linear
            # under autocast below
            bf = torch.bfloat16
            with torch.amp.autocast("cuda", enabled=False):
                b = prepared(self.bias, bf) if self.bias is not None else None
                return F.linear(x.to(bf), prepared(self.weight, bf), b)
        return F.linear(x, self.weight, self.bias)

    def _needs_grad(self) -> bool:
        if not torch.is_grad_enabled():
            return False
        return self.weight.requires_grad or (self.bias is not None and self.bias.requires_grad)


LinearNoBias = partial(Linear, bias=False)


def _bf16_autocast(x: torch.Tensor) -> bool:
    """CUDA autocast to bf16 is on and would cast this floating input."""
    return (x.dtype in (torch.float32, torch.bfloat16) and torch.is_autocast_enabled("cuda")
            and torch.get_autocast_dtype("cuda") == torch.bfloat16)
