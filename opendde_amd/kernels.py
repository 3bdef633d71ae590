"""Tensor-level entry points of the HIP backend (thin layer over the C ABI).

PyTorch is used here only as plumbing: it owns device memory (outputs and the
per-call workspace, via the caching allocator) and names the current stream.
All arithmetic happens in the gfx950 kernels of ``libopendde_amd.so``.
There is no fallback in this module: unsupported shapes, non-GPU tensors or a
missing library raise.  The ``*_unsupported`` predicates name the shapes the
kernels do not cover, so that the modules can route those calls to their
torch path before reaching an entry point.
"""

from __future__ import annotations

import ctypes
import weakref
from typing import Dict, Optional, Tuple

import torch

from . import _lib

SUPPORTED_CHANNELS = (64, 128, 256, 384)
HEAD_DIM = 32


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return _lib.F32
    if dt == torch.bfloat16:
        return _lib.BF16
    raise TypeError(f"HIP backend supports float32 and bfloat16 tensors, got {dt}")


def autocast_compute_dtype(t: torch.Tensor) -> torch.dtype:
    """Compute precision for a call: the tensor's own dtype, or bf16 when a
    float32 tensor arrives under CUDA autocast with bf16 (the reference's bf16
    inference mode keeps the residual stream in float32 and runs the module
    arithmetic in bf16)."""
    if t.dtype == torch.bfloat16:
        return torch.bfloat16
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        return torch.bfloat16
    return torch.float32


def _ptr(t: Optional[torch.Tensor]):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _require_gpu(*ts: torch.Tensor) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("HIP backend tensors must be on a GPU device")


def _pair_view_ok(t: torch.Tensor, name: str) -> None:
    if t.dim() < 3:
        raise ValueError(f"{name} must be [*, N, N, C], got {tuple(t.shape)}")
    if t.stride(-1) != 1:
        raise ValueError(f"{name} must have a unit channel stride")
    if t.shape[-3] != t.shape[-2]:
        raise ValueError(f"{name} must be square in its pair dims")


def pair_layout_ok(t: torch.Tensor) -> bool:
    """The kernels can read (and write) ``t`` [*, N, N, C] in place through
    its strides: unit channel stride, leading dims that collapse to one batch
    stride by a view, and 16-byte aligned rows (base address and the row,
    column and batch strides)."""
    if t.dim() < 3 or t.stride(-1) != 1:
        return False
    if t.numel() == 0:
        return True
    try:
        v = t.view((-1,) + tuple(t.shape[-3:]))
    except RuntimeError:
        return False
    es = t.element_size()
    strides = (v.stride(0) if v.shape[0] > 1 else 0, v.stride(1), v.stride(2))
    return t.data_ptr() % 16 == 0 and all((st * es) % 16 == 0 for st in strides)


def _batch_view(t: torch.Tensor, name: str) -> Tuple[torch.Tensor, int, int]:
    """``t`` [*, N, N, C] as a [B, N, N, C] view (never a copy: ``out`` is
    written through it) with B and the batch stride in elements."""
    _pair_view_ok(t, name)
    if t.numel() == 0:
        return t, 0, 0
    if t.dim() == 3:
        return t.unsqueeze(0), 1, 0
    try:
        v = t.view((-1,) + tuple(t.shape[-3:]))
    except RuntimeError:
        raise ValueError(f"{name}'s leading dims must collapse to one batch stride") from None
    return v, v.shape[0], v.stride(0) if v.shape[0] > 1 else 0


# Converted weights are cached per source tensor *object* (held by weak
# reference, so a freed parameter whose device address is reused by a new one
# can never hit) and its version counter (in-place updates invalidate).  An
# entry is dropped as soon as one of its source tensors is freed, so the
# converted copies of a discarded model release their device memory with it.
_wcache: Dict[Tuple, Tuple] = {}


def _evictor(cache: Dict, key):
    """Weakref callback dropping ``cache[key]`` when one of the entry's own
    source references dies (closure state only: it may run at interpreter
    shutdown, after module globals are cleared)."""
    def cb(ref) -> None:
        ent = cache.get(key)
        if ent is not None and any(r is ref for r in ent[0]):
            del cache[key]
    return cb


def _cached(key, srcs, make):
    ent = _wcache.get(key)
    if ent is not None:
        refs, versions, val = ent
        if all(r() is s for r, s in zip(refs, srcs)) and versions == tuple(s._version for s in srcs):
            return val
    val = make()
    cb = _evictor(_wcache, key)
    refs = tuple(weakref.ref(s, cb) for s in srcs)
    _wcache[key] = (refs, tuple(s._version for s in srcs), val)
    return val


def cache_size() -> int:
    """Number of converted-weight entries held (for tests)."""
    return len(_wcache)


def prepared(t: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
    """``t`` as a contiguous ``dtype`` tensor, converted once per version."""
    return _cached((id(t), dtype), (t,), lambda: t.detach().to(dtype).contiguous())


def prepared_cat(ts, dtype: torch.dtype) -> torch.Tensor:
    """Row-concatenation of ``ts`` as a contiguous ``dtype`` tensor (cached)."""
    ts = tuple(ts)
    return _cached(("cat",) + tuple(id(t) for t in ts) + (dtype,), ts,
                   lambda: torch.cat([t.detach() for t in ts], 0).to(dtype).contiguous())


def _mask_view(mask: Optional[torch.Tensor], lead: Tuple[int, ...], n: int,
               device) -> Tuple[Optional[torch.Tensor], int, int, int]:
    """The mask as float32 [B, N, N] for z's leading dims ``lead`` (a mask
    without them broadcasts: batch stride 0); returns (mask, s0, s1, sb)."""
    if mask is None:
        return None, 0, 0, 0
    if mask.dim() < 2 or tuple(mask.shape[-2:]) != (n, n) or mask.dim() > len(lead) + 2:
        raise ValueError(f"mask must be [*, N, N] = [..., {n}, {n}] over z's leading dims, "
                         f"got {tuple(mask.shape)}")
    if mask.device != device:
        raise ValueError("mask must be on the same device as z")
    if mask.dtype != torch.float32:
        mask = mask.float()
    try:
        m = mask.expand(tuple(lead) + (n, n)).reshape(-1, n, n)
    except RuntimeError:
        raise ValueError(f"mask {tuple(mask.shape)} does not broadcast to z's leading dims "
                         f"{tuple(lead)}") from None
    return m, m.stride(1), m.stride(2), m.stride(0) if m.shape[0] > 1 else 0


# ---------------------------------------------------------------------------
# coverage: why a call is outside what the kernels take (None = covered).
# The modules run their torch path for such calls, as the reference's
# accelerated slot does for configurations its kernel lacks
# (opendde/model/triangular/layers.py:455-468, triangular.py:482-486); the
# entry points below raise for them.
# ---------------------------------------------------------------------------


def _dtype_reason(t: torch.Tensor, compute_dtype: Optional[torch.dtype]) -> Optional[str]:
    if t.dtype not in (torch.float32, torch.bfloat16):
        return f"{t.dtype} tensors (the kernels take float32 and bfloat16)"
    ct = compute_dtype or autocast_compute_dtype(t)
    if t.dtype == torch.bfloat16 and ct == torch.float32:
        return "bf16 storage with fp32 arithmetic"
    return None


def triangle_attention_unsupported(z: torch.Tensor, heads: int, head_dim: int,
                                   compute_dtype: Optional[torch.dtype] = None) -> Optional[str]:
    """Reason the fused triangle attention does not take z [*, N, N, C] with
    ``heads`` x ``head_dim``, or None."""
    if head_dim != HEAD_DIM:
        return f"per-head dim {head_dim} (the kernels take {HEAD_DIM})"
    c = z.shape[-1]
    if c not in SUPPORTED_CHANNELS or heads * HEAD_DIM not in SUPPORTED_CHANNELS:
        return f"c={c}, heads={heads} (c and heads*32 must be in {SUPPORTED_CHANNELS})"
    return _dtype_reason(z, compute_dtype)


def triangle_multiplication_unsupported(z: torch.Tensor, c_hidden: int,
                                        compute_dtype: Optional[torch.dtype] = None
                                        ) -> Optional[str]:
    """Reason the fused triangle multiplication does not take z [*, N, N, C]
    with ``c_hidden``, or None."""
    c = z.shape[-1]
    if c not in SUPPORTED_CHANNELS or c_hidden not in SUPPORTED_CHANNELS:
        return f"c={c}, c_hidden={c_hidden} (both must be in {SUPPORTED_CHANNELS})"
    return _dtype_reason(z, compute_dtype)


def attention_core_unsupported(q: torch.Tensor) -> Optional[str]:
    """Reason the triangle attention core does not take q [*, H, J, D], or
    None."""
    if q.shape[-1] != HEAD_DIM:
        return f"per-head dim {q.shape[-1]} (the core takes {HEAD_DIM})"
    if q.dtype not in (torch.float32, torch.bfloat16):
        return f"{q.dtype} tensors (the core takes float32 and bfloat16)"
    return None


def transition_unsupported(x: torch.Tensor, c: int, n: int,
                           compute_dtype: Optional[torch.dtype] = None) -> Optional[str]:
    """Reason the fused transition does not take rows x [*, c] with
    intermediate factor ``n``, or None."""
    if n != 4 or c not in TRANSITION_CHANNELS:
        return f"c={c}, n={n} (the kernels take n=4, c in {TRANSITION_CHANNELS})"
    if not x.is_contiguous():
        return "non-contiguous rows"
    return _dtype_reason(x, compute_dtype)


def _workspace(nbytes: int, device) -> torch.Tensor:
    # torch's caching allocator returns 256-byte aligned blocks.
    return torch.empty(max(int(nbytes), 256), dtype=torch.uint8, device=device)


def triangle_attention(z: torch.Tensor, mask: Optional[torch.Tensor], *, ln_w, ln_b,
                       w_bias, w_q, w_k, w_v, w_g, w_o, heads: int, starting: bool = True,
                       out: Optional[torch.Tensor] = None, add_residual: bool = False,
                       compute_dtype: Optional[torch.dtype] = None, inf: float = 1e9,
                       eps: float = 1e-5) -> torch.Tensor:
    """Fused triangle attention on pair tensors z [*, N, N, C] (leading dims
    run as one batch of views in one library call).

    starting=False runs the ending-node form by reading z, the mask and the
    output through transposed strides (no transposed copies).  With
    ``add_residual`` the result is z + update, written to ``out`` (which may
    be z itself for an in-place update); otherwise ``out`` receives the
    update.  Returns ``out``.

    fp32 arithmetic with ``torch.backends.cuda.matmul.allow_tf32`` set (the
    reference's inference default, ``enable_tf32``) runs every product of
    the module (projections, attention core, output) on the bf16 MFMA in
    three parts (each operand as a bf16 pair; about 2^-16 of relative error
    per product, against TF32's 2^-11), the way the reference's kernel slot
    and its linear layers take their TF32 mode from that flag
    (opendde/model/triangular/triangular.py:55-56).  Otherwise the products
    are true fp32.
    """
    _require_gpu(z, mask)
    zb, nbatch, z_sb = _batch_view(z, "z")
    n, c = z.shape[-3], z.shape[-1]
    if c not in SUPPORTED_CHANNELS or heads * HEAD_DIM not in SUPPORTED_CHANNELS:
        raise NotImplementedError(
            f"HIP triangle attention supports c, heads*32 in {SUPPORTED_CHANNELS}; got c={c}, "
            f"heads={heads}")
    if w_q.shape[0] != heads * HEAD_DIM:
        raise NotImplementedError("HIP triangle attention requires a per-head dim of 32")
    ct = compute_dtype or autocast_compute_dtype(z)
    if z.dtype == torch.bfloat16 and ct == torch.float32:
        raise NotImplementedError("bf16 storage with fp32 compute is not provided")
    if out is None:
        out = torch.empty_like(z, memory_format=torch.contiguous_format)
    if out.dtype != z.dtype or out.shape != z.shape:
        raise ValueError("out must match z in shape and dtype")
    ob, _, o_sb = _batch_view(out, "out")
    m, ms0, ms1, m_sb = _mask_view(mask, z.shape[:-3], n, z.device)
    if z.numel() == 0:
        return out
    zs0, zs1 = zb.stride(1), zb.stride(2)
    os0, os1 = ob.stride(1), ob.stride(2)
    if not starting:
        zs0, zs1, ms0, ms1, os0, os1 = zs1, zs0, ms1, ms0, os1, os0
    lnw = prepared(ln_w, torch.float32)
    lnb = prepared(ln_b, torch.float32)
    ws = [prepared(w, ct) for w in (w_bias, w_q, w_k, w_v, w_g, w_o)]
    a = _lib.TriattArgs()
    a.struct_size = ctypes.sizeof(_lib.TriattArgs)
    a.n, a.c, a.heads, a.head_dim = n, c, heads, HEAD_DIM
    a.z_dtype, a.compute_dtype = dtype_code(z.dtype), dtype_code(ct)
    if a.compute_dtype == _lib.F32 and torch.backends.cuda.matmul.allow_tf32:
        a.compute_dtype = _lib.F32X3
    a.add_residual = 1 if add_residual else 0
    a.z, a.z_s0, a.z_s1 = _ptr(z), zs0, zs1
    a.mask, a.mask_s0, a.mask_s1 = _ptr(m), ms0, ms1
    a.out, a.out_s0, a.out_s1 = _ptr(out), os0, os1
    a.ln_w, a.ln_b = _ptr(lnw), _ptr(lnb)
    a.w_bias, a.w_q, a.w_k, a.w_v, a.w_g, a.w_o = (_ptr(w) for w in ws)
    a.inf, a.eps = float(inf), float(eps)
    a.batch, a.z_sb, a.mask_sb, a.out_sb = nbatch, z_sb, m_sb, o_sb
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    _lib.check(lib.odde_triatt_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)), "triatt workspace")
    work = _workspace(nb.value, z.device)
    a.workspace, a.workspace_bytes = _ptr(work), work.numel()
    _lib.check(lib.odde_triatt_fwd(ctypes.byref(a), _stream(z.device)), "odde_triatt_fwd")
    return out


def triangle_multiplication(z: torch.Tensor, mask: Optional[torch.Tensor], *, outgoing: bool,
                            norm_in_weight, norm_in_bias, p_in_weight, g_in_weight,
                            norm_out_weight, norm_out_bias, p_out_weight, g_out_weight,
                            out: Optional[torch.Tensor] = None, add_residual: bool = False,
                            compute_dtype: Optional[torch.dtype] = None,
                            eps: float = 1e-5, f32_out_weight: bool = True) -> torch.Tensor:
    """Fused triangle multiplicative update on z [*, N, N, C] (one library
    call for the leading dims);
    same ``out`` / ``add_residual`` contract as :func:`triangle_attention`.
    ``p_in_weight``/``g_in_weight`` are [2*Ch, C] (a rows then b rows).
    ``f32_out_weight``: with bf16 compute, also hand the library linear_z in
    f32 (it folds LN_out into that weight with a single bf16 rounding).
    fp32 arithmetic with ``torch.backends.cuda.matmul.allow_tf32`` set runs
    the products in three bf16 parts, as :func:`triangle_attention` does:
    the projections and the output always, the contraction where Np is a
    multiple of 256 (true fp32 products otherwise)."""
    _require_gpu(z, mask)
    zb, nbatch, z_sb = _batch_view(z, "z")
    n, c = z.shape[-3], z.shape[-1]
    ch = p_in_weight.shape[0] // 2
    if c not in SUPPORTED_CHANNELS or ch not in SUPPORTED_CHANNELS:
        raise NotImplementedError(
            f"HIP triangle multiplication supports c, c_hidden in {SUPPORTED_CHANNELS}; "
            f"got c={c}, c_hidden={ch}")
    ct = compute_dtype or autocast_compute_dtype(z)
    if z.dtype == torch.bfloat16 and ct == torch.float32:
        raise NotImplementedError("bf16 storage with fp32 compute is not provided")
    if out is None:
        out = torch.empty_like(z, memory_format=torch.contiguous_format)
    if out.dtype != z.dtype or out.shape != z.shape:
        raise ValueError("out must match z in shape and dtype")
    ob, _, o_sb = _batch_view(out, "out")
    m, ms0, ms1, m_sb = _mask_view(mask, z.shape[:-3], n, z.device)
    if z.numel() == 0:
        return out
    f32 = torch.float32
    a = _lib.TrimulArgs()
    a.struct_size = ctypes.sizeof(_lib.TrimulArgs)
    a.n, a.c, a.c_hidden = n, c, ch
    a.z_dtype, a.compute_dtype = dtype_code(z.dtype), dtype_code(ct)
    if a.compute_dtype == _lib.F32 and torch.backends.cuda.matmul.allow_tf32:
        a.compute_dtype = _lib.F32X3
    a.outgoing = 1 if outgoing else 0
    a.add_residual = 1 if add_residual else 0
    a.z, a.z_s0, a.z_s1 = _ptr(z), zb.stride(1), zb.stride(2)
    a.mask, a.mask_s0, a.mask_s1 = _ptr(m), ms0, ms1
    a.out, a.out_s0, a.out_s1 = _ptr(out), ob.stride(1), ob.stride(2)
    a.batch, a.z_sb, a.mask_sb, a.out_sb = nbatch, z_sb, m_sb, o_sb
    keep = [prepared(norm_in_weight, f32), prepared(norm_in_bias, f32),
            prepared(norm_out_weight, f32), prepared(norm_out_bias, f32),
            prepared(p_in_weight, ct), prepared(g_in_weight, ct),
            prepared(p_out_weight, ct), prepared(g_out_weight, ct)]
    (a.norm_in_weight, a.norm_in_bias, a.norm_out_weight, a.norm_out_bias,
     a.p_in_weight, a.g_in_weight, a.p_out_weight, a.g_out_weight) = (_ptr(t) for t in keep)
    if ct == torch.bfloat16 and f32_out_weight:
        keep.append(prepared(p_out_weight, f32))
        a.p_out_weight_f32 = _ptr(keep[-1])
    a.eps = float(eps)
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    _lib.check(lib.odde_trimul_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)), "trimul workspace")
    work = _workspace(nb.value, z.device)
    a.workspace, a.workspace_bytes = _ptr(work), work.numel()
    _lib.check(lib.odde_trimul_fwd(ctypes.byref(a), _stream(z.device)), "odde_trimul_fwd")
    return out


def triangle_attention_core(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                            bias: torch.Tensor, mask: Optional[torch.Tensor],
                            scale: float, inf: float = 1e9) -> torch.Tensor:
    """The accelerated slot of the reference's Attention.forward
    (``cuequivariance_triangular_attn(q, k, v, bias, mask, scale)``,
    opendde/model/triangular/layers.py:484-494):

      q, k, v: [B, I, H, J, D] (or [B*I, H, J, D]; any strides, D contiguous);
      bias: broadcastable to [B, 1, H, J, J] (float);
      mask: bool, broadcastable to [B, I, 1, 1, J], True = keep (or None).
    Returns softmax(scale*q k^T + bias + mask_term) v as [B, I, H, J, D] in q's
    dtype, where dropped keys get -inf (= -1e9, the torch path's value).
    """
    _require_gpu(q, k, v, bias, mask)
    squeeze = False
    if q.dim() == 4:
        q, k, v = q.unsqueeze(0), k.unsqueeze(0), v.unsqueeze(0)
        squeeze = True
    if q.dim() != 5 or q.shape != k.shape or q.shape != v.shape:
        raise ValueError("q, k, v must share a [B, I, H, J, D] shape")
    bsz, rows, heads, n, d = q.shape
    if d != HEAD_DIM:
        raise NotImplementedError("HIP triangle attention core requires head_dim == 32")
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise ValueError("q, k, v need a unit stride on the head dim")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise TypeError("q, k, v dtypes differ")
    b = bias
    while b.dim() < 5:
        b = b.unsqueeze(0)
    b = b.float().expand(bsz, 1, heads, n, n)[:, 0]
    if mask is not None:
        mk = mask
        while mk.dim() < 5:
            mk = mk.unsqueeze(0)
        mk = mk.expand(bsz, rows, 1, 1, n)[:, :, 0, 0, :].to(torch.uint8)
    else:
        mk = None
    out = torch.empty((bsz, rows, heads, n, d), dtype=q.dtype, device=q.device)
    a = _lib.TriattCoreArgs()
    a.struct_size = ctypes.sizeof(_lib.TriattCoreArgs)
    a.batch, a.rows, a.heads, a.n, a.head_dim = bsz, rows, heads, n, d
    a.dtype = dtype_code(q.dtype)
    a.q, a.q_sb, a.q_si, a.q_sh, a.q_sj = _ptr(q), *q.stride()[:4]
    a.k, a.k_sb, a.k_si, a.k_sh, a.k_sj = _ptr(k), *k.stride()[:4]
    a.v, a.v_sb, a.v_si, a.v_sh, a.v_sj = _ptr(v), *v.stride()[:4]
    a.bias, a.b_sb, a.b_sh, a.b_sq, a.b_sk = _ptr(b), *b.stride()
    if mk is not None:
        a.mask, a.m_sb, a.m_si, a.m_sk = _ptr(mk), *mk.stride()
    a.out, a.o_sb, a.o_si, a.o_sh, a.o_sj = _ptr(out), *out.stride()[:4]
    a.scale, a.inf_value = float(scale), float(inf)
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    _lib.check(lib.odde_triatt_core_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)),
               "triatt core workspace")
    work = _workspace(nb.value, q.device)
    a.workspace, a.workspace_bytes = _ptr(work), work.numel()
    _lib.check(lib.odde_triatt_core_fwd(ctypes.byref(a), _stream(q.device)), "odde_triatt_core_fwd")
    return out[0] if squeeze else out


TRANSITION_CHANNELS = (64, 128, 256, 384)


def transition(x: torch.Tensor, *, ln_w, ln_b, w_a, w_b, w_o, out: Optional[torch.Tensor] = None,
               add_residual: bool = False, eps: float = 1e-5,
               pair_bias: Optional[tuple] = None,
               compute_dtype: Optional[torch.dtype] = None) -> torch.Tensor:
    """Fused SwiGLU transition over the last dim of ``x``:
    out = (x if add_residual else 0) + W_o(silu(W_a LN(x)) * W_b LN(x)).
    ``out`` may be ``x`` (in-place residual update).  Arithmetic is bf16 for
    bf16 ``x`` or under bf16 autocast, fp32 otherwise (float32 ``x``).

    ``pair_bias = (ln_w, ln_b, w, eps, dest)`` also writes
    ``dest[h, r] = (LN(out[r]) @ w.T)[h]`` (w: [16, c], dest: float32
    [16, rows]) from the rows as written, i.e. AttentionPairBias's
    ``linear_nobias_z(layernorm_z(z))`` over the updated pair tensor.

    fp32 arithmetic with ``torch.backends.cuda.matmul.allow_tf32`` set runs
    the products in three bf16 parts, as :func:`triangle_attention` does
    (the pair-bias projection stays true fp32)."""
    _require_gpu(x)
    c = x.shape[-1]
    nf = w_a.shape[0] // c
    if c not in TRANSITION_CHANNELS or nf != 4 or w_a.shape[0] != nf * c:
        raise NotImplementedError(f"HIP transition supports c in {TRANSITION_CHANNELS}, n=4")
    if not x.is_contiguous():
        raise ValueError("transition input must be contiguous")
    if out is None:
        out = torch.empty_like(x)
    if not out.is_contiguous() or out.shape != x.shape or out.dtype != x.dtype:
        raise ValueError("out must be a contiguous tensor like x")
    ct = compute_dtype or autocast_compute_dtype(x)
    if x.dtype == torch.bfloat16 and ct == torch.float32:
        raise NotImplementedError("bf16 storage with fp32 compute is not provided")
    bf = ct
    keep = [prepared(ln_w, torch.float32), prepared(ln_b, torch.float32),
            prepared(w_a, bf), prepared(w_b, bf), prepared(w_o, bf)]
    a = _lib.TransitionArgs()
    a.struct_size = ctypes.sizeof(_lib.TransitionArgs)
    a.c, a.n_factor = c, nf
    a.x_dtype, a.compute_dtype = dtype_code(x.dtype), dtype_code(ct)
    if a.compute_dtype == _lib.F32 and torch.backends.cuda.matmul.allow_tf32:
        a.compute_dtype = _lib.F32X3
    a.add_residual = 1 if add_residual else 0
    a.rows = x.numel() // c
    a.x, a.out = _ptr(x), _ptr(out)
    a.ln_w, a.ln_b, a.w_a, a.w_b, a.w_o = (_ptr(t) for t in keep)
    a.eps = float(eps)
    if pair_bias is not None:
        pln_w, pln_b, pw, peps, dest = pair_bias
        rows = a.rows
        if pw.shape != (16, c):
            raise NotImplementedError("pair-bias projection needs a [16, c] weight")
        if dest.dtype != torch.float32 or dest.shape != (16, rows) or not dest.is_contiguous() \
                or dest.device != x.device:
            raise ValueError("pair-bias destination must be a contiguous float32 [16, rows] "
                             "tensor on x's device")
        pkeep = [prepared(pln_w, torch.float32), prepared(pw, bf)]
        if pln_b is not None:
            pkeep.append(prepared(pln_b, torch.float32))
        keep += pkeep
        a.pb_heads = 16
        a.pb_ln_w, a.pb_w = _ptr(pkeep[0]), _ptr(pkeep[1])
        a.pb_ln_b = _ptr(pkeep[2]) if pln_b is not None else None
        a.pb_out = _ptr(dest)
        a.pb_eps = float(peps)
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    _lib.check(lib.odde_transition_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)),
               "odde_transition_workspace_bytes")
    ws = None
    if nb.value:
        ws = _workspace(nb.value, x.device)
        a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
    _lib.check(lib.odde_transition_fwd(ctypes.byref(a), _stream(x.device)),
               "odde_transition_fwd")
    return out


OPM_C_M = (32, 64, 128)
OPM_C_Z = (64, 128, 256, 384)


def outer_product_mean(m: torch.Tensor, mask: Optional[torch.Tensor], *, ln_w, ln_b, w_1, w_2,
                       w_out, b_out=None, out: Optional[torch.Tensor] = None,
                       add_residual: bool = False, out_dtype: Optional[torch.dtype] = None,
                       ln_eps: float = 1e-5, eps: float = 1e-3) -> torch.Tensor:
    """OuterProductMean update of an MSA ``m`` [S, N, c_m] (bf16 arithmetic):
    ``(W_out outer(LN(m)) + b_out) / (mask^T mask + eps)`` as [N, N, c_z],
    rounded to bf16; written to ``out`` (``out += update`` with
    ``add_residual``, the MSA module's ``z = z + opm_update``).  ``mask``:
    [S, N] or None (all ones)."""
    _require_gpu(m, mask)
    if m.dim() != 3 or not m.is_contiguous():
        raise ValueError("m must be a contiguous [S, N, c_m] tensor")
    S, N, c_m = m.shape
    c, c_z = w_1.shape[0], w_out.shape[0]
    if c != 32 or c_m not in OPM_C_M or c_z not in OPM_C_Z or w_out.shape[1] != c * c:
        raise NotImplementedError(
            f"HIP outer product mean supports c_hidden = 32, c_m in {OPM_C_M}, c_z in {OPM_C_Z}")
    if out is None:
        if add_residual:
            raise ValueError("add_residual needs out (the pair tensor)")
        out = torch.empty((N, N, c_z), dtype=out_dtype or torch.bfloat16, device=m.device)
    if not out.is_contiguous() or tuple(out.shape) != (N, N, c_z):
        raise ValueError(f"out must be a contiguous [{N}, {N}, {c_z}] tensor")
    mk = None
    if mask is not None:
        if tuple(mask.shape) != (S, N):
            raise ValueError(f"mask must be [S, N] = [{S}, {N}], got {tuple(mask.shape)}")
        mk = mask.to(torch.float32).contiguous()
    f32, bf = torch.float32, torch.bfloat16
    keep = [prepared(ln_w, f32), prepared(ln_b, f32), prepared_cat((w_1, w_2), bf),
            prepared(w_out, bf)]
    if b_out is not None:
        keep.append(prepared(b_out, f32))
    a = _lib.OpmArgs()
    a.struct_size = ctypes.sizeof(_lib.OpmArgs)
    a.n_seq, a.n_res, a.c_m, a.c_hidden, a.c_z = S, N, c_m, c, c_z
    a.m_dtype, a.out_dtype, a.compute_dtype = dtype_code(m.dtype), dtype_code(out.dtype), _lib.BF16
    a.add_residual = 1 if add_residual else 0
    a.m, a.mask, a.out = _ptr(m), _ptr(mk), _ptr(out)
    a.ln_w, a.ln_b, a.w_12, a.w_out = (_ptr(t) for t in keep[:4])
    a.b_out = _ptr(keep[4]) if b_out is not None else None
    a.ln_eps, a.eps = float(ln_eps), float(eps)
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    _lib.check(lib.odde_opm_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)),
               "odde_opm_workspace_bytes")
    ws = _workspace(nb.value, m.device)
    a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
    _lib.check(lib.odde_opm_fwd(ctypes.byref(a), _stream(m.device)), "odde_opm_fwd")
    return out


BIAS_ATTN_HEAD_DIMS = (8, 16, 24, 32, 48, 64)


def bias_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                   bias: Optional[torch.Tensor], scale: float = 1.0,
                   gate: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 attention with an additive bias, the single track's attention
    core (primitives._attention with scale 1): q, k, v [H, N, D] (any head
    and row strides, D contiguous; f32 or bf16), bias [H, Nq, Nk] or None.
    ``scale`` multiplies q . k (the caller's q / sqrt(c_hidden)); ``gate``
    [H, Nq, D] (q's dtype, D contiguous) multiplies the output by
    sigmoid(gate) (Attention._wrap_up's gating). ``out`` [H, Nq, D] (any
    head and row strides, D contiguous) receives the result; by default a
    new contiguous tensor. Returns the output in q's dtype."""
    _require_gpu(q, k, v, bias)
    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3 or k.shape != v.shape:
        raise ValueError("q, k, v must be [H, N, D] with matching k and v")
    h, nq, d = q.shape
    nk = k.shape[1]
    if k.shape[0] != h or k.shape[2] != d:
        raise ValueError("q and k disagree in heads or head dim")
    if d not in BIAS_ATTN_HEAD_DIMS:
        raise NotImplementedError(f"HIP bias attention supports head_dim in {BIAS_ATTN_HEAD_DIMS}")
    if q.dtype != k.dtype or q.dtype != v.dtype:
        raise ValueError("q, k, v must share a dtype")
    for t in (q, k, v):
        if t.stride(-1) != 1:
            raise ValueError("q, k, v need a contiguous head dim")
    es = q.element_size()
    if any((t.data_ptr() | t.stride(0) * es | t.stride(1) * es) & 15 for t in (k, v)):
        # rows must start on 16-byte boundaries: a fresh allocation is 256-byte
        # aligned (.contiguous() would return a contiguous but misaligned view
        # unchanged)
        k = k.clone(memory_format=torch.contiguous_format)
        v = v.clone(memory_format=torch.contiguous_format)
    b = None
    if bias is not None:
        b = bias.to(torch.float32).expand(h, nq, nk).contiguous()
    if gate is not None and (tuple(gate.shape) != (h, nq, d) or gate.dtype != q.dtype
                             or gate.stride(-1) != 1 or gate.device != q.device):
        raise ValueError("gate must be [H, Nq, D] in q's dtype with D contiguous")
    if out is None:
        out = torch.empty((h, nq, d), dtype=q.dtype, device=q.device)
    elif (tuple(out.shape) != (h, nq, d) or out.dtype != q.dtype or out.stride(-1) != 1
          or out.device != q.device):
        raise ValueError("out must be [H, Nq, D] in q's dtype with D contiguous")
    a = _lib.BiasAttnArgs()
    a.struct_size = ctypes.sizeof(_lib.BiasAttnArgs)
    a.n_q, a.n_k, a.heads, a.head_dim, a.dtype = nq, nk, h, d, dtype_code(q.dtype)
    a.q, a.q_sh, a.q_sn = _ptr(q), q.stride(0), q.stride(1)
    a.k, a.k_sh, a.k_sn = _ptr(k), k.stride(0), k.stride(1)
    a.v, a.v_sh, a.v_sn = _ptr(v), v.stride(0), v.stride(1)
    a.bias = _ptr(b)
    a.out, a.o_sh, a.o_sn = _ptr(out), out.stride(0), out.stride(1)
    if gate is not None:
        a.gate, a.g_sh, a.g_sn = _ptr(gate), gate.stride(0), gate.stride(1)
    a.q_scale = float(scale)
    _lib.check(_lib.load().odde_bias_attn_fwd(ctypes.byref(a), _stream(q.device)),
               "odde_bias_attn_fwd")
    return out
