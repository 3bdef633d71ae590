"""OuterProductMean: the MSA -> pair update of the MSA module.

Drop-in for ``opendde.model.triangular.layers.OuterProductMean``
(triangular/layers.py:497-627, Alg. 10): same constructor, parameter names
(``layer_norm``, ``linear_1``, ``linear_2``, ``linear_out``) and
``forward(m, mask=None, chunk_size=None, inplace_safe=False)``.  The
reference has no kernel hook for this module; ``kernel="hip"`` (or the
accelerated alias ``"cuequivariance"``) selects the gfx950 kernels, which
compute in bf16 (the reference's bf16 mode).  ``hip_apply`` also offers the
MSA module's fused ``z += update`` (pairformer.py:1289-1293).
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import hook
from . import kernels as K
from .layers import LayerNorm, OpenfoldLinear


class OuterProductMean(nn.Module):
    """Alg. 10: a = mask * W_1 LN(m), b = mask * W_2 LN(m);
    out[i, j] = W_out vec(sum_s a[s, i] (x) b[s, j]) / (sum_s mask[s, i] mask[s, j] + eps)."""

    def __init__(self, c_m: int, c_z: int, c_hidden: int, eps: float = 1e-3) -> None:
        super().__init__()
        self.c_m = c_m
        self.c_z = c_z
        self.c_hidden = c_hidden
        self.eps = eps
        self.layer_norm = LayerNorm(c_m)
        self.linear_1 = OpenfoldLinear(c_m, c_hidden, bias=False)
        self.linear_2 = OpenfoldLinear(c_m, c_hidden, bias=False)
        self.linear_out = OpenfoldLinear(c_hidden ** 2, c_z, init="final")

    def hip_supported(self, m: torch.Tensor) -> bool:
        """The HIP kernels compute in bf16: bf16 inputs, or float32 inputs
        under bf16 autocast."""
        return (m.is_cuda and m.dim() == 3 and self.c_hidden == 32 and self.c_m in K.OPM_C_M
                and self.c_z in K.OPM_C_Z and K.autocast_compute_dtype(m) == torch.bfloat16)

    def hip_apply(self, m: torch.Tensor, mask: Optional[torch.Tensor] = None,
                  out: Optional[torch.Tensor] = None, add_residual: bool = False) -> torch.Tensor:
        """The update on the HIP kernels, m: [S, N, c_m].  With
        ``add_residual`` the update is added into ``out`` (the pair tensor
        [N, N, c_z]) in place."""
        if K.autocast_compute_dtype(m) != torch.bfloat16:
            raise NotImplementedError(
                "the HIP outer product mean computes in bf16 (bf16 input or bf16 autocast)")
        return K.outer_product_mean(
            m.contiguous(), mask, ln_w=self.layer_norm.weight, ln_b=self.layer_norm.bias,
            w_1=self.linear_1.weight, w_2=self.linear_2.weight, w_out=self.linear_out.weight,
            b_out=self.linear_out.bias, out=out, add_residual=add_residual,
            ln_eps=self.layer_norm.eps, eps=self.eps)

    def _opm(self, a: torch.Tensor, b: torch.Tensor) -> torch.Tensor:
        outer = torch.einsum("...bac,...dae->...bdce", a, b)
        outer = outer.reshape(outer.shape[:-2] + (-1,))
        return self.linear_out(outer)

    def _forward_torch(self, m: torch.Tensor, mask: Optional[torch.Tensor],
                       chunk_size: Optional[int]) -> torch.Tensor:
        if mask is None:
            mask = m.new_ones(m.shape[:-1])
        ln = self.layer_norm(m)
        mask = mask.unsqueeze(-1)
        a = self.linear_1(ln) * mask
        b = self.linear_2(ln) * mask
        del ln
        a = a.transpose(-2, -3)
        b = b.transpose(-2, -3)
        if chunk_size is not None and a.shape[-3] > chunk_size:
            # row chunks over i: numerically neutral (layers.py:539-566)
            outer = torch.cat([self._opm(a[..., i:i + chunk_size, :, :], b)
                               for i in range(0, a.shape[-3], chunk_size)], dim=-3)
        else:
            outer = self._opm(a, b)
        norm = torch.einsum("...abc,...adc->...bdc", mask, mask) + self.eps
        return outer / norm

    def forward(self, m: torch.Tensor, mask: Optional[torch.Tensor] = None,
                chunk_size: Optional[int] = None, inplace_safe: bool = False,
                kernel: str = "torch") -> torch.Tensor:
        """m: [*, N_seq, N_res, C_m], mask: [*, N_seq, N_res] ->
        [*, N_res, N_res, C_z].  An accelerated ``kernel`` on a GPU tensor
        runs the HIP kernels (one MSA, no leading batch dims) or raises."""
        if kernel not in hook.MODULE_KERNELS:
            raise ValueError(f"kernel must be 'hip', 'cuequivariance' or 'torch', but got {kernel}")
        if hook.is_accelerated(kernel) and m.is_cuda:
            if m.dim() != 3:
                raise NotImplementedError("the HIP outer product mean takes one [S, N, c_m] MSA")
            return self.hip_apply(m, mask)
        return self._forward_torch(m, mask, chunk_size)
