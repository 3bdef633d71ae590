"""GPU parity of the HIP fast LayerNorm (the eight-symbol contract).

Every case runs the C-ABI entry points through ``opendde_amd.fast_layer_norm``
and compares with the oracle (``layer_norm_fwd`` / ``layer_norm_bwd``, f32
statistics) on the same input, and with torch (``F.layer_norm`` and its
autograd):
* float32: output, mean, invvar and grad_input to 1e-5 abs / rel; parameter
  gradients (sums over up to 1000 rows) to 1e-4 rel;
* bfloat16 / float16: outputs rounded once from f32, so within one unit in
  the last place of the type (rtol 2^-7 for bf16, 2^-10 for f16, plus a small
  atol for values near 0), parameter gradients the same after their f32 sum.
Shapes cover each kernel path: the row kernels (n2 a multiple of the 16-byte
vector: lane groups of 16/32/64 lanes with 1 or 3 vectors per lane, and a
one-lane-per-row case), the generic kernels (odd n2, a misaligned view,
n2 > 2048), n1 = 0, and the pair LayerNorm of the N=1024 workload
(1,048,576 rows x 128, bf16) through size-independent properties.
"""

import pytest
import torch
import torch.nn.functional as F

from helpers import say
from oracle import reference as ref
from opendde_amd import _lib
from opendde_amd import fast_layer_norm as fln
from opendde_amd import layer_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
AFFINE = ["none", "bias", "weight", "both"]
TOL = {torch.float32: dict(rtol=1e-5, atol=1e-5),
       torch.bfloat16: dict(rtol=2 ** -7, atol=2e-2),
       torch.float16: dict(rtol=2 ** -10, atol=2e-3)}
PTOL = {torch.float32: dict(rtol=1e-4, atol=1e-4),
        torch.bfloat16: dict(rtol=2 ** -7, atol=5e-2),
        torch.float16: dict(rtol=2 ** -10, atol=1e-2)}


def _params(affine, shape, dtype, gen):
    w = (torch.randn(shape, generator=gen) * 0.5 + 1).to(DEV, dtype) \
        if affine in ("weight", "both") else None
    b = (torch.randn(shape, generator=gen) * 0.5).to(DEV, dtype) \
        if affine in ("bias", "both") else None
    return w, b


def _fwd(x, shape, w, b, eps=1e-5):
    if w is None and b is None:
        return fln.forward_none_affine(x, shape, eps)
    if w is None:
        return fln.forward_with_bias_affine(x, shape, b, eps)
    if b is None:
        return fln.forward_with_weight_affine(x, shape, w, eps)
    return fln.forward_with_both_affine(x, shape, w, b, eps)


def _bwd(dout, mean, invvar, x, shape, w, b, eps=1e-5):
    if w is None and b is None:
        return fln.backward_none_affine(dout, mean, invvar, x, shape, eps)
    if w is None:
        return fln.backward_with_bias_affine(dout, mean, invvar, x, shape, b, eps)
    if b is None:
        return fln.backward_with_weight_affine(dout, mean, invvar, x, shape, w, eps)
    return fln.backward_with_both_affine(dout, mean, invvar, x, shape, w, b, eps)


def _close(got, exp, tol, what):
    torch.testing.assert_close(got.float().cpu(), exp.float().cpu(), **tol, msg=lambda m: f"{what}: {m}")


# (leading shape, normalized shape): row kernels with G=16 NV=1 (bf16 128),
# G=32 NV=1 (f32 128), G=16 NV=3 (bf16 384), G=1 NV=3 (bf16 24); generic
# kernels for n2 = 37 and n2 = 4096; a 2-d normalized shape.
SHAPES = [((1000,), (128,)), ((37,), (384,)), ((5, 3), (24,)), ((19,), (37,)),
          ((6,), (4096,)), ((7,), (4, 32))]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("affine", AFFINE)
@pytest.mark.parametrize("lead,norm", SHAPES)
def test_forward_backward_match_oracle_and_torch(lead, norm, affine, dtype):
    say(f"[gpu] layer_norm {lead}x{norm} {affine} {dtype}")
    gen = torch.Generator().manual_seed(sum(lead) * 31 + sum(norm) * 7 + AFFINE.index(affine))
    x = (torch.randn(*lead, *norm, generator=gen) * 2 + 0.3).to(DEV, dtype)
    dout = torch.randn(*lead, *norm, generator=gen).to(DEV, dtype)
    w, b = _params(affine, norm, dtype, gen)
    n2 = 1
    for s in norm:
        n2 *= s
    before = (_lib.launch_count(_lib.K_LAYER_NORM), _lib.launch_count(_lib.K_LAYER_NORM_BWD))
    out, mean, invvar = _fwd(x, norm, w, b)
    gi, gw, gb = _bwd(dout, mean, invvar, x, norm, w, b)
    torch.cuda.synchronize()
    assert _lib.launch_count(_lib.K_LAYER_NORM) == before[0] + 1
    assert _lib.launch_count(_lib.K_LAYER_NORM_BWD) == before[1] + 1
    assert out.dtype == dtype and out.shape == x.shape
    assert mean.dtype == invvar.dtype == torch.float32 and mean.shape == (x.numel() // n2,)
    assert (gw is None) == (w is None) and (gb is None) == (b is None)

    # oracle on the same (already rounded) input, f32 arithmetic
    xo, wo, bo = x.float().cpu(), None if w is None else w.float().cpu(), \
        None if b is None else b.float().cpu()
    oe, me, ie = ref.layer_norm_fwd(xo, n2, wo, bo)
    _close(out, oe, TOL[dtype], "output")
    _close(mean, me, dict(rtol=1e-5, atol=1e-5), "mean")
    _close(invvar, ie, dict(rtol=1e-5, atol=1e-5), "invvar")
    # torch's own LayerNorm on the device
    _close(out, F.layer_norm(x, norm, w, b, 1e-5), TOL[dtype], "output vs F.layer_norm")

    dxe, dwe, dbe = ref.layer_norm_bwd(dout.float().cpu(), me, ie, xo, n2, wo)
    _close(gi, dxe, TOL[dtype], "grad_input")
    if gw is not None:
        assert gw.dtype == dtype and gw.shape == w.shape
        _close(gw, dwe.reshape(norm), PTOL[dtype], "grad_gamma")
    if gb is not None:
        _close(gb, dbe.reshape(norm), PTOL[dtype], "grad_beta")
    if dtype == torch.float32:
        # absent parameters enter torch's autograd as constant ones / zeros
        # (its device backward rejects a missing weight beside a bias)
        xa = x.clone().requires_grad_(True)
        wa = (w.clone() if w is not None else torch.ones(norm, device=DEV)).requires_grad_(True)
        ba = (b.clone() if b is not None else torch.zeros(norm, device=DEV)).requires_grad_(True)
        F.layer_norm(xa, norm, wa, ba, 1e-5).backward(dout)
        _close(gi, xa.grad, TOL[dtype], "grad_input vs autograd")
        if gw is not None:
            _close(gw, wa.grad, PTOL[dtype], "grad_gamma vs autograd")
        if gb is not None:
            _close(gb, ba.grad, PTOL[dtype], "grad_beta vs autograd")


def test_generic_and_row_kernels_agree_on_a_misaligned_view():
    say("[gpu] layer_norm misaligned view -> generic kernels")
    gen = torch.Generator().manual_seed(7)
    base = torch.randn(300 * 128 + 1, generator=gen).to(DEV)
    x_mis = base[1:].view(300, 128)          # 4-byte offset: not 16-byte aligned
    assert x_mis.data_ptr() % 16 != 0 and x_mis.is_contiguous()
    x_al = x_mis.clone()
    w = torch.randn(128, generator=gen).to(DEV)
    b = torch.randn(128, generator=gen).to(DEV)
    dout = torch.randn(300, 128, generator=gen).to(DEV)
    o1, m1, i1 = fln.forward_with_both_affine(x_mis, (128,), w, b, 1e-5)
    o2, m2, i2 = fln.forward_with_both_affine(x_al, (128,), w, b, 1e-5)
    for got, exp, what in ((o1, o2, "out"), (m1, m2, "mean"), (i1, i2, "invvar")):
        _close(got, exp, dict(rtol=1e-5, atol=1e-5), what)
    g1 = fln.backward_with_both_affine(dout, m1, i1, x_mis, (128,), w, b, 1e-5)
    g2 = fln.backward_with_both_affine(dout, m2, i2, x_al, (128,), w, b, 1e-5)
    for got, exp, what in zip(g1, g2, ("grad_input", "grad_gamma", "grad_beta")):
        _close(got, exp, dict(rtol=1e-4, atol=1e-4), what)


def test_empty_rows():
    say("[gpu] layer_norm n1=0")
    x = torch.empty(0, 64, device=DEV)
    w, b = torch.ones(64, device=DEV), torch.zeros(64, device=DEV)
    out, mean, invvar = fln.forward_with_both_affine(x, (64,), w, b, 1e-5)
    assert out.shape == (0, 64) and mean.shape == (0,) and invvar.shape == (0,)
    gi, gw, gb = fln.backward_with_both_affine(x, mean, invvar, x, (64,), w, b, 1e-5)
    torch.cuda.synchronize()
    assert gi.shape == (0, 64)
    assert torch.equal(gw, torch.zeros_like(w)) and torch.equal(gb, torch.zeros_like(b))


def test_backward_is_deterministic():
    say("[gpu] layer_norm backward determinism")
    gen = torch.Generator().manual_seed(11)
    x = torch.randn(5000, 384, generator=gen).to(DEV, torch.bfloat16)
    dout = torch.randn(5000, 384, generator=gen).to(DEV, torch.bfloat16)
    w = torch.randn(384, generator=gen).to(DEV, torch.bfloat16)
    b = torch.randn(384, generator=gen).to(DEV, torch.bfloat16)
    _, mean, invvar = fln.forward_with_both_affine(x, (384,), w, b, 1e-5)
    r1 = fln.backward_with_both_affine(dout, mean, invvar, x, (384,), w, b, 1e-5)
    r2 = fln.backward_with_both_affine(dout, mean, invvar, x, (384,), w, b, 1e-5)
    for a, c in zip(r1, r2):
        assert torch.equal(a, c)


def test_fused_layer_norm_module_autograd_matches_torch():
    say("[gpu] FusedLayerNorm module autograd")
    layer_norm._reset_loader_for_tests()
    gen = torch.Generator().manual_seed(12)
    m = layer_norm.FusedLayerNorm(128).to(DEV)
    with torch.no_grad():
        m.weight.copy_(torch.randn(128, generator=gen))
        m.bias.copy_(torch.randn(128, generator=gen))
    x = torch.randn(64, 50, 128, generator=gen).to(DEV).requires_grad_(True)
    before = _lib.launch_count(_lib.K_LAYER_NORM_BWD)
    y = m(x)
    y.backward(torch.ones_like(y) * 0.5 + x.detach())
    assert _lib.launch_count(_lib.K_LAYER_NORM_BWD) == before + 1
    xr = x.detach().clone().requires_grad_(True)
    wr = m.weight.detach().clone().requires_grad_(True)
    br = m.bias.detach().clone().requires_grad_(True)
    yr = F.layer_norm(xr, (128,), wr, br, 1e-5)
    yr.backward(torch.ones_like(yr) * 0.5 + x.detach())
    _close(y, yr, dict(rtol=1e-5, atol=1e-5), "module output")
    _close(x.grad, xr.grad, dict(rtol=1e-5, atol=1e-5), "module grad_input")
    _close(m.weight.grad, wr.grad, dict(rtol=1e-4, atol=1e-3), "module grad weight")
    _close(m.bias.grad, br.grad, dict(rtol=1e-4, atol=1e-3), "module grad bias")
    # bf16 input: parameters cast to bf16 inside, gradients land in f32 params
    m.zero_grad()
    xb = x.detach().to(torch.bfloat16).requires_grad_(True)
    yb = m(xb)
    assert yb.dtype == torch.bfloat16
    yb.float().sum().backward()
    assert m.weight.grad.dtype == torch.float32 and xb.grad.dtype == torch.bfloat16


def test_pair_layer_norm_n1024_properties():
    """The pair LayerNorm of the N=1024 workload: 1,048,576 rows x 128, bf16."""
    say("[gpu] layer_norm 1048576 x 128 bf16")
    gen = torch.Generator(device=DEV).manual_seed(13)
    x = (torch.randn(1024, 1024, 128, generator=gen, device=DEV) * 3 + 1).to(torch.bfloat16)
    w = torch.randn(128, generator=gen, device=DEV).to(torch.bfloat16)
    b = torch.randn(128, generator=gen, device=DEV).to(torch.bfloat16)
    out, mean, invvar = fln.forward_with_both_affine(x, (128,), w, b, 1e-5)
    # per-row statistics vs torch in f32 on the device
    var, mu = torch.var_mean(x.float().view(-1, 128), dim=1, unbiased=False)
    _close(mean, mu, dict(rtol=1e-5, atol=1e-5), "mean")
    _close(invvar, torch.rsqrt(var + 1e-5), dict(rtol=1e-5, atol=1e-5), "invvar")
    exp = F.layer_norm(x.float(), (128,), w.float(), b.float(), 1e-5)
    err = (out.float() - exp).abs() / (exp.abs() + 1e-2)
    assert float(err.max()) <= 2 ** -7, float(err.max())
    # backward: per-row sum of grad_input is 0 (shift invariance); with
    # dout = 1 and no gamma, grad_beta = n1 and grad_gamma = sum of xhat (~0)
    dout = torch.ones_like(x)
    gi, gw, gb = fln.backward_with_bias_affine(dout, mean, invvar, x, (128,), b, 1e-5)
    assert gw is None
    assert float(gi.float().abs().max()) < 1e-2
    torch.testing.assert_close(gb.float(), torch.full((128,), 1048576.0, device=DEV),
                               rtol=0, atol=0)
    gi, gw, gb = fln.backward_with_both_affine(x, mean, invvar, x, (128,), w, b, 1e-5)
    xhat = (x.float().view(-1, 128) - mean[:, None]) * invvar[:, None]
    # each stored element is rounded once to bf16 (relative error <= 2^-8)
    gf = gi.float().view(-1, 128)
    assert bool((gf.sum(dim=1).abs() <= gf.abs().sum(dim=1) * 2 ** -8 + 1e-3).all())
    torch.testing.assert_close(gb.float(), x.float().view(-1, 128).sum(0), rtol=2 ** -7, atol=1.0)
    torch.testing.assert_close(gw.float(), (x.float().view(-1, 128) * xhat).sum(0),
                               rtol=2 ** -7, atol=1.0)
