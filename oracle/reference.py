"""Plain-PyTorch CPU restatement of the reference "torch" path (test oracle).

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the ``opendde_amd`` package.

All functions take parameters as a flat ``dict`` keyed by the reference's
``named_parameters()`` names (``layer_norm.weight``, ``mha.linear_q.weight``,
``linear_a_p.weight`` ...), optionally under a prefix such as
``"tri_att_start."``.  Every op runs in the dtype of its inputs, so the same
code is the float64 pinning oracle and the float32 parity oracle.

Reference files followed (paths relative to the reference root):
  opendde/model/triangular/layers.py      LayerNorm, OpenfoldLinear, _attention, Attention
  opendde/model/triangular/triangular.py  TriangleAttention, TriangleMultiplicativeUpdate
  opendde/model/modules/primitives.py     Transition, primitives Attention, _attention
  opendde/model/modules/transformer.py    AttentionPairBias
  opendde/model/modules/pairformer.py     PairformerBlock, PairformerStack
  opendde/model/triangular/layers.py      OuterProductMean (MSA -> pair update)
  opendde/model/utils.py                  chunk_layer (numerically neutral row chunking)
"""

from __future__ import annotations

import math
from typing import Dict, Optional

import torch
import torch.nn.functional as F

Params = Dict[str, torch.Tensor]

# Additive mask magnitude (triangular.py:609 ``inf=1e9``) and LN eps
# (layers.py:232, triangular.py:514).
MASK_INF = 1e9
LN_EPS = 1e-5

# Which independent check pins each oracle function (tests/test_oracle_*.py).
PINNED_BY = {
    "layer_norm": "torch.nn.functional.layer_norm (library) + float64 brute force",
    "linear": "float64 brute force",
    "layer_norm_fwd": "torch.nn.functional.layer_norm (library) + float64 brute force; "
    "statistics == torch.var_mean",
    "layer_norm_bwd": "torch autograd of F.layer_norm (library) + float64 brute force "
    "(loops over the derivative definition); sum_c grad_input == 0",
    "attention_core": "float64 brute force; SDPA library routine with zero bias; "
    "key-permutation invariance; fully-masked row == mean(V)",
    "triangle_attention": "float64 brute force (start and end); "
    "end == T(start(T z)); chunked == unchunked",
    "combine_projections": "float64 triple loop; contract_in(a,b) == contract_out(aT,bT)",
    "triangle_multiplication": "float64 brute force (out, in); zero linear_z -> 0; "
    "zero gating weights -> gates 0.5; masked rows/cols -> a,b zero",
    "triangle_multiplication_inplace": "== standard forward + z (the reference's design "
    "claim) for odd/even N and chunk sizes straddling N/2",
    "transition": "float64 brute force",
    "attention_pair_bias": "float64 brute force; SDPA library routine",
    "pairformer_block": "float64 brute force composition; in-place == out-of-place",
    "pairformer_stack": "== sequential pairformer_block",
    "outer_product_mean": "float64 brute force (loops over s, c1, c2); mask=None -> "
    "norm S + eps; a fully masked MSA row == that row removed",
}


def _sub(params: Params, prefix: str) -> Params:
    """Parameters under ``prefix`` with the prefix stripped."""
    n = len(prefix)
    return {k[n:]: v for k, v in params.items() if k.startswith(prefix)}


# ---------------------------------------------------------------------------
# Primitives
# ---------------------------------------------------------------------------


def layer_norm(x: torch.Tensor, weight: Optional[torch.Tensor],
               bias: Optional[torch.Tensor], eps: float = LN_EPS) -> torch.Tensor:
    """LayerNorm over the last dim, biased variance.

    Follows OpenFoldLayerNorm.forward (triangular/layers.py:250-269), which is
    ``F.layer_norm`` with eps 1e-5; written out explicitly here.
    """
    mu = x.mean(dim=-1, keepdim=True)
    xc = x - mu
    var = (xc * xc).mean(dim=-1, keepdim=True)
    y = xc * torch.rsqrt(var + eps)
    if weight is not None:
        y = y * weight.to(x.dtype)
    if bias is not None:
        y = y + bias.to(x.dtype)
    return y


def layer_norm_fwd(x: torch.Tensor, n2: int, gamma: Optional[torch.Tensor],
                   beta: Optional[torch.Tensor], eps: float = LN_EPS):
    """Fast LayerNorm forward contract: ``(out, mean, invvar)`` over the last
    ``n2`` elements of each row, ``mean`` / ``invvar`` of shape ``[n1]``
    (layer_norm/kernel/layer_norm_cuda.cpp:73-90; row statistics in
    layer_norm_cuda_kernel.cu:145-229: biased variance,
    invvar = 1/sqrt(var + eps), out = (x - mean) * invvar * gamma + beta).
    Statistics are computed in float64 when ``x`` is float64, else float32."""
    sd = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf = x.reshape(-1, n2).to(sd)
    mu = xf.mean(dim=1)
    xc = xf - mu[:, None]
    invvar = torch.rsqrt((xc * xc).mean(dim=1) + eps)
    y = xc * invvar[:, None]
    if gamma is not None:
        y = y * gamma.reshape(n2).to(sd)
    if beta is not None:
        y = y + beta.reshape(n2).to(sd)
    return y.to(x.dtype).reshape(x.shape), mu, invvar


def layer_norm_bwd(dout: torch.Tensor, mean: torch.Tensor, invvar: torch.Tensor,
                   x: torch.Tensor, n2: int, gamma: Optional[torch.Tensor]):
    """Fast LayerNorm backward contract: ``(grad_input, grad_gamma,
    grad_beta)`` (layer_norm_cuda.cpp:99-139; layer_norm_cuda_kernel.cu:
    412-836).  With xhat = (x - mean) * invvar and g = dout * gamma (dout when
    gamma is absent):
        grad_input = invvar * (g - mean_c(g) - xhat * mean_c(g * xhat))
        grad_gamma = sum_rows dout * xhat,  grad_beta = sum_rows dout.
    Computed in float64 when ``x`` is float64, else float32; the parameter
    gradients are returned in that precision."""
    sd = torch.float64 if x.dtype == torch.float64 else torch.float32
    xf = x.reshape(-1, n2).to(sd)
    df = dout.reshape(-1, n2).to(sd)
    mu = mean.reshape(-1, 1).to(sd)
    iv = invvar.reshape(-1, 1).to(sd)
    xhat = (xf - mu) * iv
    g = df * gamma.reshape(n2).to(sd) if gamma is not None else df
    dx = iv * (g - g.mean(dim=1, keepdim=True) - xhat * (g * xhat).mean(dim=1, keepdim=True))
    return dx.to(x.dtype).reshape(x.shape), (df * xhat).sum(dim=0), df.sum(dim=0)


def linear(x: torch.Tensor, weight: torch.Tensor,
           bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x W^T (+ b).  OpenfoldLinear.forward (triangular/layers.py:201-223),
    primitives.Linear.forward (primitives.py:74-90)."""
    y = torch.matmul(x, weight.to(x.dtype).t())
    if bias is not None:
        y = y + bias.to(x.dtype)
    return y


def _ln(x: torch.Tensor, p: Params, name: str) -> torch.Tensor:
    return layer_norm(x, p.get(name + ".weight"), p.get(name + ".bias"))


# ---------------------------------------------------------------------------
# Triangle attention
# ---------------------------------------------------------------------------


def attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   biases) -> torch.Tensor:
    """softmax(q k^T + sum(biases)) v over the last axis.

    Follows ``_attention`` (triangular/layers.py:302-322): logits = q @ k^T,
    biases added in list order, softmax over keys, then @ v.  ``q`` already
    carries the 1/sqrt(D) scale (layers.py:405-406).
    """
    a = torch.matmul(q, k.transpose(-1, -2))
    for b in biases:
        a = a + b
    a = torch.softmax(a, dim=-1)
    return torch.matmul(a, v)


def triangle_attention(x: torch.Tensor, mask: Optional[torch.Tensor], p: Params,
                       no_heads: int, starting: bool = True, inf: float = MASK_INF,
                       chunk_size: Optional[int] = None) -> torch.Tensor:
    """Triangle attention update (the caller adds the residual).

    Follows TriangleAttention.forward (triangular/triangular.py:648-706) with
    Attention._prep_qkv/_wrap_up/forward (triangular/layers.py:387-481):

    * x [*, I, J, C]; ending node (starting=False) transposes x and mask first
      and the output back (triangular.py:669-671, 703-704);
    * x = LN(x); mask_bias = inf*(mask-1) broadcast over [*, I, 1, 1, J];
      tri_bias = linear(x) permuted to [*, 1, H, I, J] (triangular.py:674-683);
    * q,k,v,g = x W^T per head, q /= sqrt(D); softmax(q k^T + mask_bias +
      tri_bias) v; o *= sigmoid(g); out = linear_o(o).

    ``chunk_size`` slices the flattened leading (B*I) rows as chunk_layer does
    (model/utils.py:503-611); the math is identical.
    """
    if mask is None:
        mask = x.new_ones(x.shape[:-1])
    if not starting:
        x = x.transpose(-2, -3)
        mask = mask.transpose(-1, -2)
    x = _ln(x, p, "layer_norm")
    mask_bias = (inf * (mask.to(x.dtype) - 1))[..., :, None, None, :]
    tri_bias = linear(x, p["linear.weight"])              # [*, I, J, H]
    tri_bias = tri_bias.movedim(-1, -3).unsqueeze(-4)     # [*, 1, H, I, J]

    hd = p["mha.linear_q.weight"].shape[0]
    d = hd // no_heads

    def mha(xr: torch.Tensor, mbias: torch.Tensor) -> torch.Tensor:
        def heads(w):
            t = linear(xr, w)
            t = t.view(t.shape[:-1] + (no_heads, d))
            return t.transpose(-2, -3)                    # [*, H, J, D]
        q = heads(p["mha.linear_q.weight"]) / math.sqrt(d)
        k = heads(p["mha.linear_k.weight"])
        v = heads(p["mha.linear_v.weight"])
        o = attention_core(q, k, v, [mbias, tri_bias_b])
        o = o.transpose(-2, -3)                           # [*, J, H, D]
        g = torch.sigmoid(linear(xr, p["mha.linear_g.weight"]))
        o = o * g.view(g.shape[:-1] + (no_heads, d))
        o = o.reshape(o.shape[:-2] + (hd,))
        return linear(o, p["mha.linear_o.weight"])

    if chunk_size is None:
        tri_bias_b = tri_bias
        out = mha(x, mask_bias)
    else:
        lead = x.shape[:-2]
        n_rows = int(torch.tensor(lead).prod()) if len(lead) else 1
        xf = x.reshape((n_rows,) + x.shape[-2:])
        mf = mask_bias.expand(lead + mask_bias.shape[-3:]).reshape(
            (n_rows,) + mask_bias.shape[-3:])
        # tri_bias [*,1,H,I,J] is broadcast, not sliced (utils.py:544-547,565):
        # with a single batch entry it broadcasts over every row chunk.
        tb = tri_bias.reshape((-1,) + tri_bias.shape[-3:])
        assert tb.shape[0] == 1, "row chunking restated for one batch entry"
        tri_bias_b = tb
        out = x.new_zeros(xf.shape[:-1] + (p["mha.linear_o.weight"].shape[0],))
        for s in range(0, n_rows, chunk_size):
            out[s:s + chunk_size] = mha(xf[s:s + chunk_size], mf[s:s + chunk_size])
        out = out.reshape(lead + out.shape[-2:])
    if not starting:
        out = out.transpose(-2, -3)
    return out


# ---------------------------------------------------------------------------
# Triangle multiplicative update
# ---------------------------------------------------------------------------


def combine_projections(a: torch.Tensor, b: torch.Tensor, outgoing: bool) -> torch.Tensor:
    """Outgoing p[i,j,c] = sum_k a[i,k,c] b[j,k,c]; incoming
    p[i,j,c] = sum_k a[k,i,c] b[k,j,c].  Follows
    BaseTriangleMultiplicativeUpdate._combine_projections
    (triangular/triangular.py:112-139): channel-first permutes + one matmul."""
    if outgoing:
        ap = a.movedim(-1, -3)                     # [*, C, I, K]
        bp = b.movedim(-1, -3).transpose(-1, -2)   # [*, C, K, J]
    else:
        ap = a.movedim(-1, -3).transpose(-1, -2)   # [*, C, I, K]  (a[k,i])
        bp = b.movedim(-1, -3)                     # [*, C, K, J]
    return torch.matmul(ap, bp).movedim(-3, -1)


def _trimul_projections(zn: torch.Tensor, mask: torch.Tensor, p: Params, which: str):
    g = torch.sigmoid(linear(zn, p[f"linear_{which}_g.weight"]))
    return mask * g * linear(zn, p[f"linear_{which}_p.weight"])


def triangle_multiplication(z: torch.Tensor, mask: Optional[torch.Tensor], p: Params,
                            outgoing: bool = True) -> torch.Tensor:
    """Triangle multiplicative update, standard (out-of-place) path; returns the
    update.  Follows TriangleMultiplicativeUpdate.forward
    (triangular/triangular.py:530-567): zn = LN_in(z);
    a = mask*sigmoid(W_ag zn)*(W_ap zn); b likewise; p = combine(a, b);
    x = W_z LN_out(p) * sigmoid(W_g zn).  (The fp16-only a/b std rescale at
    :548-552 does not apply to fp32/bf16.)"""
    if mask is None:
        mask = z.new_ones(z.shape[:-1])
    m = mask.to(z.dtype).unsqueeze(-1)
    zn = _ln(z, p, "layer_norm_in")
    a = _trimul_projections(zn, m, p, "a")
    b = _trimul_projections(zn, m, p, "b")
    x = combine_projections(a, b, outgoing)
    x = _ln(x, p, "layer_norm_out")
    x = linear(x, p["linear_z.weight"])
    g = torch.sigmoid(linear(zn, p["linear_g.weight"]))
    return x * g


def triangle_multiplication_inplace(z: torch.Tensor, mask: Optional[torch.Tensor],
                                    p: Params, outgoing: bool = True,
                                    chunk: int = 256, with_add: bool = True) -> torch.Tensor:
    """In-place inference form (z-cache algorithm), returns the overwritten z.

    Follows TriangleMultiplicativeUpdate._inference_forward
    (triangular/triangular.py:188-456): manifest ``a`` channel-first in row
    chunks; walk column chunks j (one chunk shortened so none straddles
    ceil(N/2)); recompute the b chunk from z, restoring rows already
    overwritten from a half-size cache of z that is re-oriented at the
    half-way point; x_chunk = a @ b_chunk -> LN_out -> W_z -> * sigmoid(W_g
    LN_in(z[:, j-chunk])); write z[:, j-chunk] (+)= x_chunk.
    """
    z = z.clone()
    if mask is None:
        mask = z.new_ones(z.shape[:-1])
    m = mask.to(z.dtype).unsqueeze(-1)
    n = z.shape[-2]
    half = n // 2 + n % 2
    row, col = -3, -2

    def proj(pair, msk, which):
        t = _trimul_projections(_ln(pair, p, "layer_norm_in"), msk, p, which)
        return t.movedim(-1, -3)                  # [*, C, X, Y]

    # a manifested as [*, C, I, K] (a[i,k] outgoing, a[k,i] incoming).
    a = proj(z, m, "a")
    if not outgoing:
        a = a.transpose(-1, -2)

    def sl(t, s, e, dim):
        idx = [slice(None)] * t.dim()
        idx[dim] = slice(s, e)
        return t[tuple(idx)]

    b_dim = row if outgoing else col
    cache = sl(z, 0, half, col).clone()           # left half of z
    rotated = False
    starts = list(range(0, half, chunk))
    widths = [e - s for s, e in zip(starts, starts[1:] + [half])]
    starts2 = list(range(half, n, chunk))
    widths += [chunk] * len(starts2)
    starts += starts2
    for s, w in zip(starts, widths):
        if not rotated and s >= half:
            # Re-orient the cache to hold quadrants 3 (from the cache) and 4
            # (from z) of the original z, transposed (triangular.py:283-306).
            q3 = sl(cache, half, None, row)
            cache = cache.transpose(row, col)[..., : n // 2, :, :].clone()
            idx = [slice(None)] * cache.dim()
            idx[col] = slice(0, half)
            cache[tuple(idx)] = q3
            idx[col] = slice(half, None)
            cache[tuple(idx)] = sl(sl(z, half, None, row), half, None, col)
            rotated = True
        mk = sl(m, s, s + w, b_dim)
        if b_dim == col:
            zb = sl(z, s, s + w, col)
        elif not rotated:
            zb = sl(z, s, s + w, row).clone()
            idx = [slice(None)] * zb.dim()
            idx[col] = slice(0, half)
            zb[tuple(idx)] = sl(cache, s, s + w, row)
        else:
            zb = sl(cache, s - half, s - half + w, row)
        bc = proj(zb, mk, "b")                     # [*, C, w, N] or [*, C, N, w]
        if outgoing:
            bc = bc.transpose(-1, -2)              # [*, C, K, w]
        x = torch.matmul(a, bc).movedim(-3, -1)    # [*, I, w, C]
        x = _ln(x, p, "layer_norm_out")
        x = linear(x, p["linear_z.weight"])
        zg = sl(z, s, s + w, col)
        g = torch.sigmoid(linear(_ln(zg, p, "layer_norm_in"), p["linear_g.weight"]))
        x = x * g
        idx = [slice(None)] * z.dim()
        idx[col] = slice(s, s + w)
        if with_add:
            z[tuple(idx)] += x
        else:
            z[tuple(idx)] = x
    return z


# ---------------------------------------------------------------------------
# Block members
# ---------------------------------------------------------------------------


def transition(x: torch.Tensor, p: Params) -> torch.Tensor:
    """SwiGLU transition: W_o( silu(W_a y) * (W_b y) ), y = LN(x).
    Follows Transition.forward (modules/primitives.py:182-217); its flat row
    chunking (:21,196-201) is numerically neutral and not restated."""
    y = _ln(x, p, "layernorm1")
    a = F.silu(linear(y, p["linear_no_bias_a.weight"]))
    b = linear(y, p["linear_no_bias_b.weight"]) * a
    return linear(b, p["linear_no_bias.weight"])


def attention_pair_bias(s: torch.Tensor, z: torch.Tensor, p: Params,
                        n_heads: int) -> torch.Tensor:
    """AttentionPairBias with has_s=False, create_offset_ln_z=True, no local
    attention, no extra bias: returns the single update.

    Follows AttentionPairBias.forward / standard_multihead_attention
    (modules/transformer.py:550-671) and primitives Attention
    (modules/primitives.py:645-857, _attention :220-258): a = LN(s);
    bias[h,i,j] = W_z LN_z(z)[i,j,h]; q = W_q a + b_q, k = W_k a, v = W_v a,
    per head dim c_a/H, q /= sqrt(dh); o = softmax(q k^T + bias) v computed in
    fp32 (SDPA with scale 1); o *= sigmoid(W_g a); out = W_o o.
    """
    a = _ln(s, p, "layernorm_a")
    bias = linear(_ln(z, p, "layernorm_z"), p["linear_nobias_z.weight"])
    bias = bias.movedim(-1, -3)                                  # [*, H, N, N]
    c_a = a.shape[-1]
    dh = c_a // n_heads

    def heads(t):
        t = t.view(t.shape[:-1] + (n_heads, dh))
        return t.transpose(-2, -3)
    q = heads(linear(a, p["attention.linear_q.weight"], p["attention.linear_q.bias"]))
    k = heads(linear(a, p["attention.linear_k.weight"]))
    v = heads(linear(a, p["attention.linear_v.weight"]))
    q = q / math.sqrt(dh)
    in_dtype = q.dtype
    wd = torch.float64 if in_dtype == torch.float64 else torch.float32
    o = attention_core(q.to(wd), k.to(wd), v.to(wd), [bias.to(wd)]).to(in_dtype)
    o = o.transpose(-2, -3)
    g = torch.sigmoid(linear(a, p["attention.linear_g.weight"]))
    o = o * g.view(g.shape[:-1] + (n_heads, dh))
    o = o.reshape(o.shape[:-2] + (c_a,))
    return linear(o, p["attention.linear_o.weight"])


def pairformer_block(s: Optional[torch.Tensor], z: torch.Tensor, mask: torch.Tensor,
                     p: Params, no_heads_pair: int = 4, n_heads: int = 16,
                     chunk_size: Optional[int] = None, inplace: bool = False):
    """One PairformerBlock forward; returns (s, z).

    Follows PairformerBlock.forward (modules/pairformer.py:157-273): z +=
    tri_mul_out; z += tri_mul_in; z += tri_att_start; z += T(tri_att_end(T z))
    (the block transposes z and the mask around a starting-node module,
    :218-226); z += pair_transition(z); then, if s is given, s +=
    attention_pair_bias(s, z); s += single_transition(s).  ``inplace``
    selects the reference's in-place branch (:196-227), which routes the
    triangle multiplications through the z-cache form.
    """
    if inplace:
        z = triangle_multiplication_inplace(z, mask, _sub(p, "tri_mul_out."), True)
        z = triangle_multiplication_inplace(z, mask, _sub(p, "tri_mul_in."), False)
    else:
        z = z + triangle_multiplication(z, mask, _sub(p, "tri_mul_out."), True)
        z = z + triangle_multiplication(z, mask, _sub(p, "tri_mul_in."), False)
    z = z + triangle_attention(z, mask, _sub(p, "tri_att_start."), no_heads_pair,
                               chunk_size=chunk_size)
    zt = z.transpose(-2, -3)
    zt = zt + triangle_attention(zt, mask.transpose(-1, -2), _sub(p, "tri_att_end."),
                                 no_heads_pair, chunk_size=chunk_size)
    z = zt.transpose(-2, -3)
    z = z + transition(z, _sub(p, "pair_transition."))
    if s is not None:
        s = s + attention_pair_bias(s, z, _sub(p, "attention_pair_bias."), n_heads)
        s = s + transition(s, _sub(p, "single_transition."))
    return s, z


def pairformer_stack(s, z, mask, p: Params, n_blocks: int, **kw):
    """PairformerStack.forward without checkpointing (inference;
    modules/pairformer.py:390-451, model/utils.py:618-673)."""
    for b in range(n_blocks):
        s, z = pairformer_block(s, z, mask, _sub(p, f"blocks.{b}."), **kw)
    return s, z


# ---------------------------------------------------------------------------
# MSA -> pair: OuterProductMean
# ---------------------------------------------------------------------------

OPM_EPS = 1e-3  # OuterProductMean(eps=1e-3), triangular/layers.py:512


def outer_product_mean(m: torch.Tensor, mask: Optional[torch.Tensor], p: Params,
                       eps: float = OPM_EPS) -> torch.Tensor:
    """OuterProductMean update for an MSA ``m`` [S, N, c_m] (mask [S, N] or
    None = all ones): returns [N, N, c_z].

    Follows OuterProductMean._forward / _opm (triangular/layers.py:525-616):
    y = LN(m); a = (W_1 y) * mask; b = (W_2 y) * mask;
    outer[i, j, c1, c2] = sum_s a[s, i, c1] b[s, j, c2], flattened c1-major;
    out = W_out outer + b_out; out /= (sum_s mask[s, i] mask[s, j] + eps).
    Its chunking over i (_chunk, :539-566) is numerically neutral and not
    restated.
    """
    if mask is None:
        mask = m.new_ones(m.shape[:-1])
    y = _ln(m, p, "layer_norm")
    mk = mask.to(m.dtype).unsqueeze(-1)
    a = linear(y, p["linear_1.weight"], p.get("linear_1.bias")) * mk
    b = linear(y, p["linear_2.weight"], p.get("linear_2.bias")) * mk
    outer = torch.einsum("sic,sjd->ijcd", a, b)
    outer = outer.reshape(outer.shape[:-2] + (-1,))
    out = linear(outer, p["linear_out.weight"], p.get("linear_out.bias"))
    norm = torch.einsum("si,sj->ij", mask.to(m.dtype), mask.to(m.dtype)) + eps
    return out / norm.unsqueeze(-1)


def flops_outer_product_mean(s: int, n: int, c_m: int, c: int, c_z: int) -> float:
    """Projections 2*S*N*c_m*2c, outer product 2*S*N^2*c^2, W_out 2*N^2*c^2*c_z."""
    return 2.0 * s * n * c_m * 2 * c + 2.0 * s * n * n * c * c + 2.0 * n * n * c * c * c_z


# ---------------------------------------------------------------------------
# FLOP accounting (algorithmic, multiply-add = 2)
# ---------------------------------------------------------------------------


def flops_triatt_core(n: int, h: int, d: int, batch: int = 1) -> float:
    return 4.0 * batch * n ** 3 * h * d


def flops_triatt_linears(n: int, c: int, h: int, d: int, batch: int = 1) -> float:
    return 2.0 * batch * n * n * c * (5 * h * d + h)


def flops_trimul_contract(n: int, ch: int, batch: int = 1) -> float:
    return 2.0 * batch * n ** 3 * ch


def flops_trimul_linears(n: int, c: int, ch: int, batch: int = 1) -> float:
    return 2.0 * batch * n * n * (4 * c * ch + c * c + ch * c)


def flops_transition(rows: int, c: int, nf: int = 4) -> float:
    return 2.0 * rows * (2 * c * nf * c + nf * c * c)


def flops_single(n: int, c_z: int, c_s: int, n_heads: int) -> float:
    return (2.0 * n * n * c_z * n_heads + 8.0 * n * c_s * c_s + 4.0 * n * n * c_s
            + 2.0 * n * c_s * c_s + flops_transition(n, c_s))


def flops_block(n: int, c_z: int = 128, c_s: int = 384, h: int = 4, d: int = 32,
                ch: int = 128, n_heads: int = 16) -> float:
    f = 2 * (flops_triatt_core(n, h, d) + flops_triatt_linears(n, c_z, h, d))
    f += 2 * (flops_trimul_contract(n, ch) + flops_trimul_linears(n, c_z, ch))
    f += flops_transition(n * n, c_z)
    if c_s > 0:
        f += flops_single(n, c_z, c_s, n_heads)
    return f
