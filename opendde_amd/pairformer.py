"""PairformerBlock / PairformerStack and their non-triangle members, drop-in
for opendde/model/modules/pairformer.py:59-451 (blocks part),
modules/primitives.py:158-279,645-857 and modules/transformer.py:39-671.

With an accelerated triangle kernel value on GPU tensors the block runs the
fused HIP kernels with the residual add folded in, in place when
``inplace_safe``; the ending-node attention reads and writes z through
transposed strides instead of the reference's two full transposed copies of z
(pairformer.py:218-226).  The pair and single transitions run as fused HIP
kernels (bf16 or fp32 arithmetic); the pair transition's epilogue also forms
the single track's 16-head pair bias from the rows it writes, and the single
track's attention core runs on the HIP fp32 bias-attention kernel.  The
single track's small s-side projections (LayerNorm and linears over N x 384)
stay PyTorch ops.
"""

from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import hook
from . import kernels as K
from .layers import LayerNorm, Linear, LinearNoBias, _bf16_autocast
from .triangular import (TriangleAttention, TriangleMultiplicationIncoming,
                         TriangleMultiplicationOutgoing)

_TRANSITION_FLAT_CHUNK_ROWS = 262_144


class Transition(nn.Module):
    """SwiGLU transition (primitives.py:158-217), flat-chunked by rows."""

    def __init__(self, c_in: int, n: int) -> None:
        super().__init__()
        self.n = n
        self.c_in = c_in
        self.layernorm1 = LayerNorm(c_in)
        self.linear_no_bias_a = LinearNoBias(in_features=c_in, out_features=n * c_in,
                                             initializer="relu")
        self.linear_no_bias_b = LinearNoBias(in_features=c_in, out_features=n * c_in,
                                             initializer="relu")
        self.linear_no_bias = LinearNoBias(in_features=n * c_in, out_features=c_in,
                                           initializer="zeros")

    def hip_supported(self, x: torch.Tensor) -> bool:
        """The fused HIP kernels take n = 4 and c in ``K.TRANSITION_CHANNELS``,
        in bf16 arithmetic (bf16 inputs, or float32 inputs under bf16
        autocast, the reference's bf16 mode) or fp32 arithmetic (float32
        inputs without autocast).  A GPU call outside that is noted once and
        runs the torch path."""
        if not x.is_cuda:
            return False
        why = K.transition_unsupported(x, self.c_in, self.n)
        if why is not None:
            hook.note_fallback("Transition", why)
        return why is None

    def hip_apply(self, x: torch.Tensor, out: Optional[torch.Tensor] = None,
                  add_residual: bool = False, pair_bias: Optional[tuple] = None) -> torch.Tensor:
        return K.transition(x, ln_w=self.layernorm1.weight, ln_b=self.layernorm1.bias,
                            w_a=self.linear_no_bias_a.weight, w_b=self.linear_no_bias_b.weight,
                            w_o=self.linear_no_bias.weight, out=out, add_residual=add_residual,
                            eps=self.layernorm1.eps, pair_bias=pair_bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        other = x.shape[:-1]
        xf = x.reshape(-1, x.shape[-1])
        if xf.shape[0] > _TRANSITION_FLAT_CHUNK_ROWS:
            chunks = xf.split(_TRANSITION_FLAT_CHUNK_ROWS, dim=0)
        elif x.dim() >= 2 and x.shape[-2] >= 3200:
            chunks = torch.chunk(xf, 8, dim=0)
        else:
            chunks = (xf,)
        outputs = None
        start = 0
        for ch in chunks:
            y = self.layernorm1(ch)
            a = F.silu(self.linear_no_bias_a(y))
            b = self.linear_no_bias_b(y)
            del y
            b = b * a
            del a
            b = self.linear_no_bias(b)
            if outputs is None:
                outputs = torch.empty((xf.shape[0], self.c_in), dtype=x.dtype, device=x.device)
            outputs[start:start + b.shape[0]] = b
            start += b.shape[0]
        return outputs.reshape(*other, self.c_in)


def _sdpa_fp32(q, k, v, bias):
    """Attention in fp32 (primitives.py:220-258): SDPA with scale 1 and an
    additive bias; returns the input dtype."""
    d = q.dtype
    o = F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                       attn_mask=None if bias is None else bias.float(), scale=1.0)
    return o.to(d)


class SingleAttention(nn.Module):
    """primitives.Attention restricted to what AttentionPairBias uses
    (primitives.py:645-857): q with bias, k/v/o/g without, gating, q /= sqrt(dh)."""

    def __init__(self, c_q: int, c_k: int, c_v: int, c_hidden: int, num_heads: int,
                 gating: bool = True, q_linear_bias: bool = True, zero_init: bool = True):
        super().__init__()
        self.c_hidden = c_hidden
        self.num_heads = num_heads
        hd = c_hidden * num_heads
        self.linear_q = Linear(c_q, hd) if q_linear_bias else LinearNoBias(c_q, hd)
        self.linear_k = LinearNoBias(c_k, hd)
        self.linear_v = LinearNoBias(c_v, hd)
        self.linear_o = LinearNoBias(hd, c_q)
        self.linear_g = LinearNoBias(c_q, hd, initializer="zeros") if gating else None
        self.sigmoid = nn.Sigmoid()
        if zero_init:
            nn.init.zeros_(self.linear_o.weight)

    def _hip_fused(self, x: torch.Tensor, attn_bias: Optional[torch.Tensor]) -> torch.Tensor:
        """Self-attention of one sequence x [N, c] under bf16 autocast on the
        HIP core: q, k, v and g from one GEMM (the four weights row-
        concatenated, the q bias padded with zeros; cached per version), the
        1 / sqrt(c_hidden) scale and the sigmoid gate applied inside the core,
        whose output is written token-major, so linear_o reads it in place."""
        bf = torch.bfloat16
        hd = self.c_hidden * self.num_heads
        w = K.prepared_cat((self.linear_q.weight, self.linear_k.weight, self.linear_v.weight,
                            self.linear_g.weight), bf)
        if self.linear_q.bias is not None:
            if getattr(self, "_zero_bias", None) is None or self._zero_bias.device != x.device:
                self._zero_bias = torch.zeros(3 * hd, device=x.device)
            b = K.prepared_cat((self.linear_q.bias, self._zero_bias), bf)
        else:
            b = None
        n = x.shape[0]
        with torch.autocast(device_type="cuda", enabled=False):
            y = F.linear(x.to(bf), w, b)  # [N, 4 hd]: q | k | v | g
            parts = [y[:, i * hd:(i + 1) * hd].view(n, self.num_heads, self.c_hidden)
                     .transpose(0, 1) for i in range(4)]
            o = torch.empty((n, self.num_heads, self.c_hidden), dtype=bf, device=x.device)
            K.bias_attention(parts[0], parts[1], parts[2], attn_bias,
                             scale=1.0 / math.sqrt(self.c_hidden), gate=parts[3],
                             out=o.transpose(0, 1))
        return self.linear_o(o.view(n, hd))

    def forward(self, q_x, kv_x, attn_bias=None, hip: bool = False):
        """``hip``: run the fp32 attention core on the HIP kernel (one
        sequence [N, c], GPU tensors, supported head dim)."""
        def heads(t):
            return t.view(t.shape[:-1] + (self.num_heads, -1)).transpose(-2, -3)
        if (hip and q_x.is_cuda and kv_x is q_x and q_x.dim() == 2 and _bf16_autocast(q_x)
                and self.linear_g is not None and self.c_hidden in K.BIAS_ATTN_HEAD_DIMS
                and (attn_bias is None or attn_bias.dim() == 3)):
            return self._hip_fused(q_x, attn_bias)
        if q_x.is_cuda and _bf16_autocast(q_x):
            # the bf16 cast autocast gives each of the four projections, once
            same = kv_x is q_x
            q_x = q_x.to(torch.bfloat16)
            kv_x = q_x if same else kv_x
        q = heads(self.linear_q(q_x)) / math.sqrt(self.c_hidden)
        k = heads(self.linear_k(kv_x))
        v = heads(self.linear_v(kv_x))
        if (hip and q.is_cuda and q.dim() == 3 and self.c_hidden in K.BIAS_ATTN_HEAD_DIMS
                and (attn_bias is None or attn_bias.dim() == 3)):
            o = K.bias_attention(q, k, v, attn_bias).transpose(-2, -3)
        else:
            if attn_bias is not None and attn_bias.dim() != q.dim():
                attn_bias = attn_bias.unsqueeze(-3)
            o = _sdpa_fp32(q, k, v, attn_bias).transpose(-2, -3)
        if self.linear_g is not None:
            g = self.sigmoid(self.linear_g(q_x))
            o = o * g.view(g.shape[:-1] + (self.num_heads, -1))
        o = o.reshape(o.shape[:-2] + (-1,))
        return self.linear_o(o)


class AttentionPairBias(nn.Module):
    """Algorithm 24 with has_s=False (transformer.py:39-671): single-track
    attention biased by a per-head projection of LN(z)."""

    def __init__(self, has_s: bool = False, create_offset_ln_z: bool = True, n_heads: int = 16,
                 c_a: int = 384, c_s: int = 384, c_z: int = 128) -> None:
        super().__init__()
        if has_s:
            raise NotImplementedError("only the Pairformer form (has_s=False) is provided")
        assert c_a % n_heads == 0
        self.n_heads = n_heads
        self.layernorm_a = LayerNorm(c_a)
        self.attention = SingleAttention(c_a, c_a, c_a, c_a // n_heads, n_heads, gating=True,
                                         q_linear_bias=True, zero_init=True)
        self.layernorm_z = LayerNorm(c_z, create_offset=create_offset_ln_z)
        self.linear_nobias_z = LinearNoBias(in_features=c_z, out_features=n_heads)

    def hip_pair_bias_ok(self) -> bool:
        """The pair-bias projection can be produced by the fused transition
        kernel (16 heads, LN with a scale)."""
        return self.n_heads == 16 and self.layernorm_z.weight is not None

    def pair_bias_spec(self, dest: torch.Tensor) -> tuple:
        return (self.layernorm_z.weight, self.layernorm_z.bias, self.linear_nobias_z.weight,
                self.layernorm_z.eps, dest)

    def forward(self, a: torch.Tensor, s: Optional[torch.Tensor], z: torch.Tensor,
                extra_attn_bias: Optional[torch.Tensor] = None,
                z_bias: Optional[torch.Tensor] = None, hip: bool = False,
                **_unused) -> torch.Tensor:
        """``z_bias`` ([heads, N, N]) is ``linear_nobias_z(layernorm_z(z))``
        already computed from this z (the fused transition kernel makes it
        while writing z); ``z`` is then not read."""
        a = self.layernorm_a(a)
        if z_bias is None:
            bias = self.linear_nobias_z(self.layernorm_z(z)).movedim(-1, -3)
        else:
            bias = z_bias
        if extra_attn_bias is not None:
            eb = extra_attn_bias
            while eb.dim() < bias.dim() - 1:
                eb = eb.unsqueeze(0)
            if eb.dim() == bias.dim() - 1:
                eb = eb.unsqueeze(-3)
            bias = bias + eb.to(dtype=bias.dtype, device=bias.device)
        return self.attention(q_x=a, kv_x=a, attn_bias=bias, hip=hip)


def _hip_covers(mod: nn.Module, z: torch.Tensor, name: str) -> bool:
    why = mod.hip_unsupported(z)
    if why is not None:
        hook.note_fallback(name, why)
    return why is None


_SIDE_STREAMS = {}


def _side_stream(device: torch.device) -> "torch.cuda.Stream":
    """One extra stream per device (default priority) for the single track."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(idx)
    if st is None:
        st = _SIDE_STREAMS[idx] = torch.cuda.Stream(device=idx)
    return st


class PairformerBlock(nn.Module):
    """Algorithm 17 block (pairformer.py:59-273)."""

    def __init__(self, n_heads: int = 16, c_z: int = 128, c_s: int = 384, c_hidden_mul: int = 128,
                 c_hidden_pair_att: int = 32, no_heads_pair: int = 4,
                 num_intermediate_factor: int = 4, hidden_scale_up: bool = False) -> None:
        super().__init__()
        self.n_heads = n_heads
        if hidden_scale_up:
            no_heads_pair = c_z // c_hidden_pair_att
            c_hidden_mul = c_z
        self.tri_mul_out = TriangleMultiplicationOutgoing(c_z=c_z, c_hidden=c_hidden_mul)
        self.tri_mul_in = TriangleMultiplicationIncoming(c_z=c_z, c_hidden=c_hidden_mul)
        self.tri_att_start = TriangleAttention(c_in=c_z, c_hidden=c_hidden_pair_att,
                                               no_heads=no_heads_pair)
        self.tri_att_end = TriangleAttention(c_in=c_z, c_hidden=c_hidden_pair_att,
                                             no_heads=no_heads_pair)
        self.pair_transition = Transition(c_in=c_z, n=num_intermediate_factor)
        self.c_s = c_s
        if c_s > 0:
            self.attention_pair_bias = AttentionPairBias(has_s=False, create_offset_ln_z=True,
                                                         n_heads=n_heads, c_a=c_s, c_z=c_z)
            self.single_transition = Transition(c_in=c_s, n=4)

    def forward(self, s: Optional[torch.Tensor], z: torch.Tensor, pair_mask: torch.Tensor,
                triangle_multiplicative: str = "torch", triangle_attention: str = "torch",
                inplace_safe: bool = False, chunk_size: Optional[int] = None,
                extra_attn_bias: Optional[torch.Tensor] = None):
        z, z_bias, accel = self.pair_update(z, pair_mask, triangle_multiplicative,
                                            triangle_attention, inplace_safe, chunk_size)
        s = self.single_update(s, z, z_bias, accel, extra_attn_bias)
        return s, z

    def pair_update(self, z: torch.Tensor, pair_mask: torch.Tensor,
                    triangle_multiplicative: str = "torch", triangle_attention: str = "torch",
                    inplace_safe: bool = False, chunk_size: Optional[int] = None):
        """The pair track of the block (pairformer.py:196-227): returns the
        updated z, the single track's pair bias when the fused transition
        formed it (else None), and whether the accelerated path runs."""
        hook.check_multiplicative_kernel(triangle_multiplicative)
        hook.check_attention_kernel(triangle_attention)
        hip_mul = hook.is_accelerated(triangle_multiplicative) and z.is_cuda
        hip_att = hook.is_accelerated(triangle_attention) and z.is_cuda
        accel = hip_mul or hip_att  # the transitions and the single track follow
        # shapes or dtypes the kernels do not cover run the torch path
        hip_mul = hip_mul and _hip_covers(self.tri_mul_out, z, "TriangleMultiplicativeUpdate")
        hip_att = hip_att and _hip_covers(self.tri_att_start, z, "TriangleAttention")
        if (hip_mul or hip_att) and not K.pair_layout_ok(z):
            # the kernels read z through its strides; a layout they cannot
            # (uncollapsible leading dims, unaligned rows) runs on a copy
            z = z.contiguous()

        # triangle multiplications: z + update, in place when allowed
        for mod in (self.tri_mul_out, self.tri_mul_in):
            if hip_mul:
                z = mod.hip_apply(z, pair_mask, out=z if inplace_safe else None,
                                  add_residual=True)
            elif inplace_safe:
                z = mod(z, mask=pair_mask, inplace_safe=True, _add_with_inplace=True,
                        triangle_multiplicative="torch")
            else:
                z = z + mod(z, mask=pair_mask, triangle_multiplicative="torch")

        if hip_att:
            z = self.tri_att_start.hip_apply(z, pair_mask, out=z if inplace_safe else None,
                                             add_residual=True)
            z = self.tri_att_end.hip_apply(z, pair_mask, transpose=True,
                                           out=z if inplace_safe else None, add_residual=True)
        else:
            upd = self.tri_att_start(z, mask=pair_mask, triangle_attention="torch",
                                     chunk_size=chunk_size)
            z = z.add_(upd) if inplace_safe else z + upd
            zt = z.transpose(-2, -3).contiguous()
            upd = self.tri_att_end(zt, mask=pair_mask.transpose(-1, -2) if pair_mask is not None
                                   else None, triangle_attention="torch", chunk_size=chunk_size)
            zt = zt.add_(upd) if inplace_safe else zt + upd
            z = zt.transpose(-2, -3).contiguous()

        z_bias = None
        if accel and self.pair_transition.hip_supported(z):
            pb = None
            if self.c_s > 0 and z.dim() == 3 and self.attention_pair_bias.hip_pair_bias_ok():
                z_bias = torch.empty((16, z.shape[0], z.shape[1]), dtype=torch.float32,
                                     device=z.device)
                pb = self.attention_pair_bias.pair_bias_spec(z_bias.view(16, -1))
            z = self.pair_transition.hip_apply(z, out=z if inplace_safe else None,
                                               add_residual=True, pair_bias=pb)
        else:
            upd = self.pair_transition(z)
            z = z.add_(upd) if inplace_safe else z + upd
        return z, z_bias, accel

    def single_update(self, s: Optional[torch.Tensor], z: torch.Tensor,
                      z_bias: Optional[torch.Tensor], accel: bool,
                      extra_attn_bias: Optional[torch.Tensor] = None):
        """The single track of the block (pairformer.py:228-273).  With
        ``z_bias`` given, z is not read."""
        if self.c_s > 0:
            s = s + self.attention_pair_bias(a=s, s=None, z=z, extra_attn_bias=extra_attn_bias,
                                             z_bias=z_bias, hip=accel)
            if accel and self.single_transition.hip_supported(s):
                s = self.single_transition.hip_apply(s.contiguous(), add_residual=True)
            else:
                s = s + self.single_transition(s)
        return s


class PairformerStack(nn.Module):
    """Algorithm 17 stack (pairformer.py:276-451); no activation checkpointing
    (inference)."""

    def __init__(self, n_blocks: int = 48, n_heads: int = 16, c_z: int = 128, c_s: int = 384,
                 num_intermediate_factor: int = 4, blocks_per_ckpt: Optional[int] = None,
                 hidden_scale_up: bool = False) -> None:
        super().__init__()
        self.n_blocks = n_blocks
        self.n_heads = n_heads
        self.blocks_per_ckpt = blocks_per_ckpt
        self.blocks = nn.ModuleList(
            PairformerBlock(n_heads=n_heads, c_z=c_z, c_s=c_s,
                            num_intermediate_factor=num_intermediate_factor,
                            hidden_scale_up=hidden_scale_up) for _ in range(n_blocks))

    # Run each block's single track on a second stream, beside the next
    # block's pair track (see forward).
    overlap_single_track = True

    def forward(self, s, z, pair_mask, triangle_multiplicative: str = "torch",
                triangle_attention: str = "torch", inplace_safe: bool = False,
                chunk_size: Optional[int] = None, extra_attn_bias=None):
        if (self.overlap_single_track and s is not None and z.is_cuda and len(self.blocks) > 1
                and (hook.is_accelerated(triangle_multiplicative)
                     or hook.is_accelerated(triangle_attention))):
            return self._forward_overlapped(s, z, pair_mask, triangle_multiplicative,
                                            triangle_attention, inplace_safe, chunk_size,
                                            extra_attn_bias)
        for b in self.blocks:
            s, z = b(s, z, pair_mask, triangle_multiplicative=triangle_multiplicative,
                     triangle_attention=triangle_attention, inplace_safe=inplace_safe,
                     chunk_size=chunk_size, extra_attn_bias=extra_attn_bias)
        return s, z

    def _forward_overlapped(self, s, z, pair_mask, triangle_multiplicative, triangle_attention,
                            inplace_safe, chunk_size, extra_attn_bias):
        """The z track of the stack never reads s (pairformer.py:196-227), and
        a block's single track reads z only through the pair bias that the
        fused pair transition writes into its own buffer.  So block b's
        single track runs on a second stream while block b + 1's pair track
        runs on the caller's: the second stream waits for an event recorded
        after block b's pair transition, and the caller's stream waits for
        the second stream before returning.  The kernels and their inputs
        are those of the sequential order, so the results are bit-identical;
        the single track's small kernels fill the pair kernels' tails.  A
        block whose pair bias the transition could not form (its single
        track would read z, which the next block overwrites in place) runs
        its single track in order on the caller's stream."""
        main = torch.cuda.current_stream(z.device)
        side = _side_stream(z.device)
        for b in self.blocks:
            z, z_bias, accel = b.pair_update(z, pair_mask, triangle_multiplicative,
                                             triangle_attention, inplace_safe, chunk_size)
            if b.c_s <= 0:
                continue
            if z_bias is None:
                main.wait_stream(side)
                s = b.single_update(s, z, None, accel, extra_attn_bias)
                continue
            side.wait_stream(main)
            with torch.cuda.stream(side):
                s = b.single_update(s, z, z_bias, accel, extra_attn_bias)
            # z_bias was allocated on the caller's stream: keep its memory from
            # being reused there before the second stream has read it
            z_bias.record_stream(side)
        main.wait_stream(side)
        # s was allocated on the second stream and is used on the caller's
        s.record_stream(main)
        return s, z
