"""fp32 pair-stack modules with reduced-precision products allowed.

With ``torch.backends.cuda.matmul.allow_tf32`` set (the reference's inference
default: ``enable_tf32``, opendde/config/model_base.py:35, applied at
opendde/model/opendde.py:106), the fp32 triangle modules and the transition
run their products on the bf16 MFMA in three parts: each operand as a bf16
pair hi + lo, hi*hi + hi*lo + lo*hi with fp32 accumulation (about 2^-16 of
relative error per product, against TF32's 2^-11).  That covers every
projection, the attention core, the outputs, the transition's GEMMs and the
triangle contraction where Np is a multiple of 256.  The softmax, the
LayerNorms, the gates, the exact fallback rows and the residuals stay fp32.

Checks: the fp32 tier's bar (max-abs <= 1e-4) against the fp32 oracle (or,
where scaled-up weights make the reference's own TF32 mode miss that bar by
far, at least 8x closer than it), and output bits that differ from the
true-fp32 products' (so the three-part form did run).
"""

import pytest
import torch

from helpers import assert_fp32, margin, params_of, say, seeded, token_pair_mask
from oracle import reference as ref
from opendde_amd import workload as wl
from opendde_amd.pairformer import PairformerBlock
from opendde_amd.triangular import TriangleAttention

pytestmark = pytest.mark.gpu
DEV = "cuda"
STD = 0.1


def _tf32(t: torch.Tensor) -> torch.Tensor:
    """t rounded to TF32 (10 stored mantissa bits, nearest)."""
    i = t.float().contiguous().view(torch.int32)
    return ((i + 0x1000) & ~0x1FFF).view(torch.float32)


def _tf32_core(q, k, v, biases):
    """The oracle's attention core with the reference's TF32 mode: each
    matmul's operands rounded to TF32 (softmax and accumulation in fp32)."""
    a = torch.matmul(_tf32(q), _tf32(k).transpose(-1, -2))
    for b in biases:
        a = a + b
    a = torch.softmax(a, dim=-1)
    return torch.matmul(_tf32(a), _tf32(v))


def _run(mod, z, mask, tf32):
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = tf32
    try:
        with torch.no_grad():
            return mod(z, mask, triangle_attention="hip")
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old


@pytest.mark.parametrize("c,h", [(128, 4), (64, 2), (256, 8), (384, 12)])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("n", [17, 65, 130])
def test_three_part_core_matches_fp32_oracle(c, h, starting, n, monkeypatch):
    """Against the fp32 oracle: within the fp32 tier's bar (max-abs 1e-4), or,
    where the weights are scaled up so that logits reach tens of nats (c 384,
    12 heads), at least 8x closer to it than the reference's own TF32 mode
    (the oracle with its core's matmul operands rounded to TF32)."""
    _check_three_part_attention(c, h, starting, n, monkeypatch)


@pytest.mark.parametrize("c,h,starting", [(128, 4, True), (64, 2, True), (128, 2, False),
                                          (64, 4, False)])
def test_three_part_staged_projection_matches_fp32_oracle(c, h, starting, monkeypatch):
    """n = 260: the projection reads its split weights through LDS staging
    (from n = 256), for C of 64 and 128 and heads x 32 of 64 and 128."""
    _check_three_part_attention(c, h, starting, 260, monkeypatch)


def _check_three_part_attention(c, h, starting, n, monkeypatch):
    say(f"[gpu] three-part core c={c} h={h} n={n} start={starting}")
    mod = seeded(TriangleAttention(c, 32, h, starting=starting), 900 + c + h + n, STD)
    z = torch.randn(n, n, c, generator=torch.Generator().manual_seed(n + c))
    mask = token_pair_mask(n, max(1, n // 10), seed=n, random=True)
    exp = ref.triangle_attention(z, mask, params_of(mod), h, starting=starting)
    monkeypatch.setattr(ref, "attention_core", _tf32_core)
    tf = ref.triangle_attention(z, mask, params_of(mod), h, starting=starting)
    monkeypatch.undo()
    mod = mod.to(DEV)
    got = _run(mod, z.to(DEV), mask.to(DEV), True)
    exact = _run(mod, z.to(DEV), mask.to(DEV), False)
    err = float((got.double().cpu() - exp.double()).abs().max())
    err_tf32 = float((tf.double() - exp.double()).abs().max())
    what = f"triatt three-part c={c} h={h} n={n} start={starting}"
    say(f"    {what}: max-abs {err:.3e} (reference TF32 mode {err_tf32:.3e})")
    margin(f"{what} (reference TF32 mode: {err_tf32:.3e})", max_abs=err, bar=1e-4)
    assert torch.isfinite(got).all()
    assert err <= max(1e-4, err_tf32 / 8), f"{what}: {err:.3e} against TF32 {err_tf32:.3e}"
    assert not torch.equal(got, exact), "the three-part form did not run"


def test_three_part_core_exact_rows():
    # large logits (the fast path's overflow bound fails: exact rows) and
    # fully masked rows (mean of v), as in the fp32 tests
    n, pad = 72, 7
    mod = seeded(TriangleAttention(128, 32, 4), 31, 0.6)
    z = torch.randn(n, n, 128, generator=torch.Generator().manual_seed(32))
    mask = token_pair_mask(n, pad)
    exp = ref.triangle_attention(z, mask, params_of(mod), 4)
    got = _run(mod.to(DEV), z.to(DEV), mask.to(DEV), True)
    r = float((got[: n - pad].double().cpu() - exp[: n - pad].double()).abs().max() /
              exp[: n - pad].double().abs().max())
    say(f"    large-logit rel max err {r:.2e}")
    assert torch.isfinite(got).all() and r < 1e-3
    mod2 = seeded(TriangleAttention(128, 32, 4), 35, STD)
    z2 = torch.randn(40, 40, 128, generator=torch.Generator().manual_seed(36))
    mask2 = token_pair_mask(40, 5)
    exp2 = ref.triangle_attention(z2, mask2, params_of(mod2), 4)
    got2 = _run(mod2.to(DEV), z2.to(DEV), mask2.to(DEV), True)
    assert_fp32(got2, exp2, "three-part fully masked rows")


@pytest.mark.timeout(300)
def test_three_part_block_n1024_matches_fp32_oracle():
    """One N=1024 trunk block (51 random pads, c_s 384) in fp32 arithmetic
    with reduced-precision products allowed, against the oracle run in fp32
    on the GPU with TF32 off."""
    cfg = wl.TRUNK_N1024
    z0, s0, mask, gen = wl.make_inputs(cfg)
    blk = PairformerBlock(n_heads=cfg.n_heads_single, c_z=cfg.c_z, c_s=cfg.c_s,
                          c_hidden_mul=cfg.c_hidden_mul, c_hidden_pair_att=cfg.head_dim,
                          no_heads_pair=cfg.heads)
    wl.init_module_(blk, gen)
    blk = blk.eval().to(DEV)
    z0, s0, mask = z0.to(DEV), s0.to(DEV), mask.to(DEV)
    params = {k: v.detach().float() for k, v in blk.named_parameters()}
    old = torch.backends.cuda.matmul.allow_tf32
    try:
        torch.backends.cuda.matmul.allow_tf32 = False
        with torch.no_grad():
            sr, zr = ref.pairformer_block(s0, z0.clone(), mask, params, no_heads_pair=cfg.heads,
                                          n_heads=cfg.n_heads_single, chunk_size=64)
        torch.backends.cuda.matmul.allow_tf32 = True
        with torch.no_grad():
            sh, zh = blk(s0, z0.clone(), mask, triangle_multiplicative="hip",
                         triangle_attention="hip", inplace_safe=True)
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old
    dz = float((zh.double() - zr.double()).abs().max())
    ds = float((sh.double() - sr.double()).abs().max())
    say(f"    three-part N=1024 block: z max-abs {dz:.3e}, s max-abs {ds:.3e}")
    margin("three-part fp32 block n1024 z", max_abs=dz, bar=1e-4)
    margin("three-part fp32 block n1024 s", max_abs=ds, bar=1e-4)
    assert torch.isfinite(zh).all() and torch.isfinite(sh).all()
    assert dz <= 1e-4 and ds <= 1e-4


def _tf32_combine(a, b, outgoing):
    """The oracle's contraction with the reference's TF32 mode: a and b
    rounded to TF32 before the sum over k (accumulated in fp32)."""
    return _orig_combine(_tf32(a), _tf32(b), outgoing)


_orig_combine = ref.combine_projections


@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n,c,ch", [(256, 128, 128), (250, 64, 128), (512, 128, 128),
                                    (300, 128, 128), (260, 64, 64), (260, 128, 64),
                                    (260, 64, 128)])
def test_three_part_contraction_matches_fp32_oracle(outgoing, n, c, ch, monkeypatch):
    """fp32 triangle multiplication with TF32 allowed: the projections' and
    the output's products in three bf16 parts, the contraction's too where Np
    (n rounded up to 128) is a multiple of 256 (n 250, 256, 512), true fp32
    contraction products otherwise (n 260 and 300: Np 384).  From n = 256
    the projection and the output stage their split weights in LDS (n 260:
    C and Ch of 64 and 128).  Within the fp32 tier's
    bar of the fp32 oracle, or at least 8x closer to it than the reference's
    TF32 mode (the oracle with the contraction's operands rounded to TF32)."""
    from opendde_amd.triangular import (TriangleMultiplicationIncoming,
                                        TriangleMultiplicationOutgoing)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(c, ch), 950 + n + c + ch, STD)
    z = torch.randn(n, n, c, generator=torch.Generator().manual_seed(n + 7))
    mask = token_pair_mask(n, max(1, n // 10), seed=n + 1, random=True)
    exp = ref.triangle_multiplication(z, mask, params_of(mod), outgoing=outgoing)
    monkeypatch.setattr(ref, "combine_projections", _tf32_combine)
    tf = ref.triangle_multiplication(z, mask, params_of(mod), outgoing=outgoing)
    monkeypatch.undo()
    mod = mod.to(DEV)
    res = []
    for tf32 in (True, False):
        old = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = tf32
        try:
            with torch.no_grad():
                res.append(mod(z.to(DEV), mask.to(DEV), triangle_multiplicative="hip"))
        finally:
            torch.backends.cuda.matmul.allow_tf32 = old
    got, exact = res
    err = float((got.double().cpu() - exp.double()).abs().max())
    err_tf32 = float((tf.double() - exp.double()).abs().max())
    what = f"trimul three-part n={n} c={c} ch={ch} out={outgoing}"
    say(f"    {what}: max-abs {err:.3e} (reference TF32 mode {err_tf32:.3e})")
    margin(f"{what} (reference TF32 mode: {err_tf32:.3e})", max_abs=err, bar=1e-4)
    assert torch.isfinite(got).all()
    assert err <= max(1e-4, err_tf32 / 8), f"{what}: {err:.3e} against TF32 {err_tf32:.3e}"
    assert not torch.equal(got, exact), "the three-part form did not run"


# pair rows (from 16384: LDS-staged weights, 4- and 8-wave tiles, ragged last
# tiles) and single-track rows (hidden chunks split over workgroups), every
# width of the fp32 row kernel
@pytest.mark.parametrize("c,rows", [(128, 16384), (128, 40000), (64, 16400), (64, 33000),
                                    (128, 1000), (256, 130), (384, 130), (384, 17), (64, 257)])
def test_three_part_transition_matches_fp32_oracle(c, rows):
    from opendde_amd.pairformer import Transition
    mod = seeded(Transition(c, 4), 760 + c, 0.7 * STD * (128 / c) ** 0.5)
    x = torch.randn(rows, c, generator=torch.Generator().manual_seed(c + 3))
    exp = ref.transition(x, params_of(mod))
    mod = mod.to(DEV)
    xg = x.to(DEV)
    res = []
    for tf32 in (True, False):
        old = torch.backends.cuda.matmul.allow_tf32
        torch.backends.cuda.matmul.allow_tf32 = tf32
        try:
            with torch.no_grad():
                res.append(mod.hip_apply(xg))
        finally:
            torch.backends.cuda.matmul.allow_tf32 = old
    got, exact = res
    err = float((got.double().cpu() - exp.double()).abs().max())
    what = f"transition three-part c={c} rows={rows}"
    say(f"    {what}: max-abs {err:.3e}")
    margin(what, max_abs=err, bar=1e-4)
    assert torch.isfinite(got).all()
    assert err <= 1e-4, f"{what}: {err:.3e}"
    assert not torch.equal(got, exact), "the three-part form did not run"


def test_three_part_transition_pair_bias_in_place():
    # the fused pair-bias epilogue (true fp32) after three-part GEMMs, in place
    from opendde_amd.pairformer import AttentionPairBias, Transition
    n, c = 131, 128
    tr = seeded(Transition(c, 4), 770, STD)
    apb = seeded(AttentionPairBias(n_heads=16, c_a=384, c_z=c, create_offset_ln_z=True), 771, 0.1)
    x = torch.randn(n, n, c, generator=torch.Generator().manual_seed(772))
    z_new = x + ref.transition(x, params_of(tr))
    pz = params_of(apb)
    exp_bias = ref.linear(ref.layer_norm(z_new, pz["layernorm_z.weight"], pz.get("layernorm_z.bias")),
                          pz["linear_nobias_z.weight"]).permute(2, 0, 1)
    tr, apb = tr.to(DEV), apb.to(DEV)
    xg = x.to(DEV)
    dest = torch.full((16, n, n), float("nan"), device=DEV)
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = True
    try:
        with torch.no_grad():
            out = tr.hip_apply(xg, out=xg, add_residual=True,
                               pair_bias=apb.pair_bias_spec(dest.view(16, -1)))
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old
    assert out.data_ptr() == xg.data_ptr()
    dz = float((out.double().cpu() - z_new.double()).abs().max())
    db = float((dest.double().cpu() - exp_bias.double()).abs().max())
    margin("transition three-part in place z", max_abs=dz, bar=1e-4)
    margin("transition three-part pair bias", max_abs=db, bar=1e-4)
    assert dz <= 1e-4 and db <= 1e-4
