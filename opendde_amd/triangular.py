"""Triangle attention and triangle multiplicative update, drop-in for the
reference's modules (opendde/model/triangular/triangular.py,
opendde/model/triangular/layers.py:325-494).

Same constructor and ``forward`` signatures, parameter names and
kernel-selection kwarg.  ``"torch"`` runs plain PyTorch ops; ``"hip"`` (alias
``"cuequivariance"``) on a GPU tensor runs the fused gfx950 kernels of
``libopendde_amd.so`` when they cover the call's shape and dtype, and the
torch ops otherwise (logged once), as the reference's accelerated slot does;
on a CPU tensor it runs the torch ops.  A missing library raises.
"""

from __future__ import annotations

import math
from functools import partialmethod
from typing import List, Optional

import torch
import torch.nn as nn

from . import hook
from . import kernels as K
from .layers import LayerNorm, OpenfoldLinear


def _use_hip(name: str, t: torch.Tensor) -> bool:
    return hook.is_accelerated(name) and t.is_cuda


# ---------------------------------------------------------------------------
# accelerated slots (same call shapes as the reference's cuEq slots)
# ---------------------------------------------------------------------------


def hip_triangular_attn(q, k, v, bias, mask, scale):
    """HIP replacement of ``cuequivariance_triangular_attn`` (layers.py:484-494):
    q, k, v [*, H, J, D] strided views (not pre-scaled), bias [*, 1, H, J, J]
    float, mask bool [*, I, 1, 1, J] (True = keep).  Returns a 1-tuple like
    the reference's slot (callers take ``[0]``)."""
    return (K.triangle_attention_core(q, k, v, bias, mask, scale),)


cuequivariance_triangular_attn = hip_triangular_attn


def kernel_triangular_mult(x, direction, mask, norm_in_weight, norm_in_bias, p_in_weight,
                           g_in_weight, norm_out_weight, norm_out_bias, p_out_weight,
                           g_out_weight, eps):
    """HIP replacement of ``kernel_triangular_mult`` (triangular.py:17-79): x
    [..., N, N, C], mask [..., N, N]; returns the update (no residual)."""
    if direction not in ("outgoing", "incoming"):
        raise ValueError(f"direction must be 'outgoing' or 'incoming', got {direction}")
    # all leading views in one library call (batch strides), as the module
    # path runs them
    return K.triangle_multiplication(
        hip_layout(x), mask, outgoing=direction == "outgoing",
        norm_in_weight=norm_in_weight, norm_in_bias=norm_in_bias,
        p_in_weight=p_in_weight, g_in_weight=g_in_weight,
        norm_out_weight=norm_out_weight, norm_out_bias=norm_out_bias,
        p_out_weight=p_out_weight, g_out_weight=g_out_weight, eps=eps)


def hip_layout(z: torch.Tensor) -> torch.Tensor:
    """``z`` itself when the kernels read it through its strides, else a
    contiguous copy (leading dims that no view collapses, a non-unit channel
    stride or unaligned rows)."""
    return z if K.pair_layout_ok(z) else z.contiguous()


# ---------------------------------------------------------------------------
# triangle MHA
# ---------------------------------------------------------------------------


def softmax_no_cast(t: torch.Tensor, dim: int = -1) -> torch.Tensor:
    """Softmax that stays in bf16 for bf16 input (layers.py:285-298)."""
    if t.dtype is torch.bfloat16:
        with torch.amp.autocast("cuda", enabled=False):
            return torch.softmax(t, dim=dim)
    return torch.softmax(t, dim=dim)


def _attention(query, key, value, biases: List[torch.Tensor]) -> torch.Tensor:
    """softmax(q k^T + sum biases) v (layers.py:302-322)."""
    a = torch.matmul(query, key.transpose(-1, -2))
    for b in biases:
        a += b
    a = softmax_no_cast(a, -1)
    return torch.matmul(a, value)


class Attention(nn.Module):
    """Triangle multi-head attention with a list of additive biases
    (layers.py:325-481).  ``c_hidden`` is the per-head dim."""

    def __init__(self, c_q: int, c_k: int, c_v: int, c_hidden: int, no_heads: int,
                 gating: bool = True) -> None:
        super().__init__()
        self.c_q, self.c_k, self.c_v = c_q, c_k, c_v
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.gating = gating
        hd = c_hidden * no_heads
        self.linear_q = OpenfoldLinear(c_q, hd, bias=False)
        self.linear_k = OpenfoldLinear(c_k, hd, bias=False)
        self.linear_v = OpenfoldLinear(c_v, hd, bias=False)
        self.linear_o = OpenfoldLinear(hd, c_q, bias=False, init="final")
        self.linear_g = OpenfoldLinear(c_q, hd, bias=False, init="gating") if gating else None
        self.sigmoid = nn.Sigmoid()

    def _prep_qkv(self, q_x, kv_x, apply_scale: bool = True):
        q, k, v = self.linear_q(q_x), self.linear_k(kv_x), self.linear_v(kv_x)
        q = q.view(q.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        k = k.view(k.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        v = v.view(v.shape[:-1] + (self.no_heads, -1)).transpose(-2, -3)
        if apply_scale:
            q = q / math.sqrt(self.c_hidden)
        return q, k, v

    def _wrap_up(self, o, q_x):
        if self.linear_g is not None:
            g = self.sigmoid(self.linear_g(q_x))
            o = o * g.view(g.shape[:-1] + (self.no_heads, -1))
        o = o.reshape(o.shape[:-2] + (-1,))
        return self.linear_o(o)

    def forward(self, q_x: torch.Tensor, kv_x: torch.Tensor,
                biases: Optional[List[torch.Tensor]] = None,
                triangle_attention: str = "torch") -> torch.Tensor:
        hook.check_attention_kernel(triangle_attention)
        if biases is None:
            biases = []
        use_hip = _use_hip(triangle_attention, q_x)
        q, k, v = self._prep_qkv(q_x, kv_x, apply_scale=not use_hip)
        if use_hip:
            why = K.attention_core_unsupported(q)
            if why is not None:
                hook.note_fallback("Attention", why)
                use_hip = False
                q = q / math.sqrt(self.c_hidden)
        if use_hip:
            if len(biases) != 2:
                raise ValueError("the accelerated slot takes [mask_bias, triangle_bias]")
            scale = 1.0 / math.sqrt(self.c_hidden)
            o = hip_triangular_attn(q, k, v, biases[1].float(), (biases[0] == 0).bool(), scale)[0]
        else:
            o = _attention(q, k, v, biases)
        o = o.transpose(-2, -3)
        return self._wrap_up(o, q_x)


# ---------------------------------------------------------------------------
# TriangleAttention
# ---------------------------------------------------------------------------


class TriangleAttention(nn.Module):
    """Triangle attention (triangular.py:586-706); returns the update."""

    def __init__(self, c_in: int, c_hidden: int, no_heads: int, starting: bool = True,
                 inf: float = 1e9) -> None:
        super().__init__()
        self.c_in = c_in
        self.c_hidden = c_hidden
        self.no_heads = no_heads
        self.starting = starting
        self.inf = inf
        self.layer_norm = LayerNorm(c_in)
        self.linear = OpenfoldLinear(c_in, no_heads, bias=False)
        self.mha = Attention(c_in, c_in, c_in, c_hidden, no_heads)

    # -- HIP path ------------------------------------------------------------
    def hip_apply(self, z: torch.Tensor, mask: Optional[torch.Tensor], *, transpose: bool = False,
                  out: Optional[torch.Tensor] = None, add_residual: bool = False,
                  compute_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Fused HIP forward on z [*, N, N, C] (the leading dims in one library
        call).  With ``transpose`` the module acts on the transposed pair view
        (the ending-node form the Pairformer builds around a starting-node
        module) without copying z.  ``add_residual`` writes z + update into
        ``out``."""
        mha = self.mha
        return K.triangle_attention(
            z, mask, ln_w=self.layer_norm.weight, ln_b=self.layer_norm.bias,
            w_bias=self.linear.weight, w_q=mha.linear_q.weight, w_k=mha.linear_k.weight,
            w_v=mha.linear_v.weight, w_g=mha.linear_g.weight, w_o=mha.linear_o.weight,
            heads=self.no_heads, starting=self.starting != transpose, out=out,
            add_residual=add_residual, compute_dtype=compute_dtype, inf=self.inf,
            eps=self.layer_norm.eps)

    def hip_unsupported(self, z: torch.Tensor) -> Optional[str]:
        """Reason the fused kernels do not take this module on z, or None."""
        return K.triangle_attention_unsupported(z, self.no_heads, self.c_hidden)

    # -- torch path ----------------------------------------------------------
    def _chunk(self, x, biases, chunk_size, triangle_attention="torch"):
        lead = x.shape[:-2]
        n_rows = 1
        for d in lead:
            n_rows *= d
        xf = x.reshape((n_rows,) + tuple(x.shape[-2:]))
        mb = biases[0].expand(lead + tuple(biases[0].shape[-3:])).reshape(
            (n_rows,) + tuple(biases[0].shape[-3:]))
        tb = biases[1].reshape((-1,) + tuple(biases[1].shape[-3:]))
        out = None
        for s in range(0, n_rows, chunk_size):
            o = self.mha(q_x=xf[s:s + chunk_size], kv_x=xf[s:s + chunk_size],
                         biases=[mb[s:s + chunk_size], tb], triangle_attention=triangle_attention)
            if out is None:
                out = o.new_zeros((n_rows,) + tuple(o.shape[1:]))
            out[s:s + chunk_size] = o
        return out.reshape(lead + tuple(out.shape[1:]))

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None,
                chunk_size: Optional[int] = None, triangle_attention: str = "torch",
                inplace_safe: bool = False) -> torch.Tensor:
        hook.check_attention_kernel(triangle_attention)
        if _use_hip(triangle_attention, x):
            why = self.hip_unsupported(x)
            if why is None:
                # chunk_size only bounds memory in the torch path; the fused
                # HIP path never materialises the logits.
                return self.hip_apply(hip_layout(x), mask)
            hook.note_fallback("TriangleAttention", why)
        if mask is None:
            mask = x.new_ones(x.shape[:-1])
        if not self.starting:
            x = x.transpose(-2, -3)
            mask = mask.transpose(-1, -2)
        x = self.layer_norm(x)
        mask_bias = (self.inf * (mask - 1))[..., :, None, None, :]
        triangle_bias = self.linear(x).movedim(-1, -3).unsqueeze(-4)
        biases = [mask_bias, triangle_bias]
        if chunk_size is not None:
            x = self._chunk(x, biases, chunk_size, triangle_attention="torch")
        else:
            x = self.mha(q_x=x, kv_x=x, biases=biases, triangle_attention="torch")
        if not self.starting:
            x = x.transpose(-2, -3)
        return x


# ---------------------------------------------------------------------------
# Triangle multiplicative update
# ---------------------------------------------------------------------------


class TriangleMultiplicativeUpdate(nn.Module):
    """Algorithms 11/12 (triangular.py:82-567)."""

    def __init__(self, c_z: int, c_hidden: int, _outgoing: bool = True) -> None:
        super().__init__()
        self.c_z = c_z
        self.c_hidden = c_hidden
        self._outgoing = _outgoing
        self.linear_g = OpenfoldLinear(c_z, c_z, bias=False, init="gating")
        self.linear_z = OpenfoldLinear(c_hidden, c_z, bias=False, init="final")
        self.layer_norm_in = LayerNorm(c_z)
        self.layer_norm_out = LayerNorm(c_hidden)
        self.sigmoid = nn.Sigmoid()
        self.linear_a_p = OpenfoldLinear(c_z, c_hidden, bias=False)
        self.linear_a_g = OpenfoldLinear(c_z, c_hidden, bias=False, init="gating")
        self.linear_b_p = OpenfoldLinear(c_z, c_hidden, bias=False)
        self.linear_b_g = OpenfoldLinear(c_z, c_hidden, bias=False, init="gating")

    def _combine_projections(self, a, b):
        if self._outgoing:
            a = a.movedim(-1, -3)
            b = b.movedim(-1, -3).transpose(-1, -2)
        else:
            a = a.movedim(-1, -3).transpose(-1, -2)
            b = b.movedim(-1, -3)
        return torch.matmul(a, b).movedim(-3, -1)

    def hip_apply(self, z: torch.Tensor, mask: Optional[torch.Tensor], *,
                  out: Optional[torch.Tensor] = None, add_residual: bool = False,
                  compute_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
        """Fused HIP forward on z [*, N, N, C] (the leading dims in one library
        call); ``add_residual`` writes z + update into ``out`` (which may be
        z: the in-place inference form)."""
        ct = compute_dtype or K.autocast_compute_dtype(z)
        p_in = K.prepared_cat([self.linear_a_p.weight, self.linear_b_p.weight], ct)
        g_in = K.prepared_cat([self.linear_a_g.weight, self.linear_b_g.weight], ct)
        return K.triangle_multiplication(
            z, mask, outgoing=self._outgoing,
            norm_in_weight=self.layer_norm_in.weight, norm_in_bias=self.layer_norm_in.bias,
            p_in_weight=p_in, g_in_weight=g_in,
            norm_out_weight=self.layer_norm_out.weight, norm_out_bias=self.layer_norm_out.bias,
            p_out_weight=self.linear_z.weight, g_out_weight=self.linear_g.weight,
            out=out, add_residual=add_residual, compute_dtype=compute_dtype,
            eps=self.layer_norm_in.eps)

    def hip_unsupported(self, z: torch.Tensor) -> Optional[str]:
        """Reason the fused kernels do not take this module on z, or None."""
        return K.triangle_multiplication_unsupported(z, self.c_hidden)

    def forward(self, z: torch.Tensor, mask: Optional[torch.Tensor] = None,
                inplace_safe: bool = False, _add_with_inplace: bool = False,
                _inplace_chunk_size: Optional[int] = 256,
                triangle_multiplicative: str = "torch") -> torch.Tensor:
        hook.check_multiplicative_kernel(triangle_multiplicative)
        add = inplace_safe is True and _add_with_inplace
        if _use_hip(triangle_multiplicative, z):
            why = self.hip_unsupported(z)
            if why is None:
                zl = hip_layout(z)
                if add:
                    # in-place inference form: z <- z + update, one fused pass
                    if zl is z:
                        return self.hip_apply(z, mask, out=z, add_residual=True)
                    z.copy_(self.hip_apply(zl, mask, out=zl, add_residual=True))
                    return z
                return self.hip_apply(zl, mask)
            hook.note_fallback("TriangleMultiplicativeUpdate", why)
        if mask is None:
            mask = z.new_ones(z.shape[:-1])
        m = mask.unsqueeze(-1)
        z_in = z
        zn = self.layer_norm_in(z)
        a = m * self.sigmoid(self.linear_a_g(zn)) * self.linear_a_p(zn)
        b = m * self.sigmoid(self.linear_b_g(zn)) * self.linear_b_p(zn)
        x = self._combine_projections(a, b)
        del a, b
        x = self.layer_norm_out(x)
        x = self.linear_z(x)
        x = x * self.sigmoid(self.linear_g(zn))
        if add:
            z_in += x
            return z_in
        return x


class TriangleMultiplicationOutgoing(TriangleMultiplicativeUpdate):
    """Algorithm 11."""

    __init__ = partialmethod(TriangleMultiplicativeUpdate.__init__, _outgoing=True)


class TriangleMultiplicationIncoming(TriangleMultiplicativeUpdate):
    """Algorithm 12."""

    __init__ = partialmethod(TriangleMultiplicativeUpdate.__init__, _outgoing=False)
