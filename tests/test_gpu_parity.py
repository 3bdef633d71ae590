"""GPU parity: the HIP kernels (called through the C ABI by the drop-in
modules) against the CPU oracle on identical seeded inputs and weights.

Tiers: fp32 kernels max-abs <= 1e-4 vs the fp32 oracle; bf16 kernels
rel-L2 <= 1e-2 and max-abs <= 5e-2 vs the fp32 oracle fed the same
(bf16-representable) input.
"""

import pytest
import torch

from helpers import (assert_bf16, assert_fp32, margin, params_of, rel_l2, say, seeded,
                     token_pair_mask)
from oracle import reference as ref
from opendde_amd import _lib
from opendde_amd.pairformer import PairformerBlock
from opendde_amd.triangular import (Attention, TriangleAttention, TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing)

pytestmark = pytest.mark.gpu
DEV = "cuda"
STD = 0.1  # larger than the workload's 0.02 so that every term is visible


@pytest.fixture(autouse=True)
def _announce(request):
    say(f"[gpu] {request.node.nodeid}")
    yield
    torch.cuda.synchronize()


def _z(n, c, seed, dtype=torch.float32):
    z = torch.randn(n, n, c, generator=torch.Generator().manual_seed(seed))
    return z.to(dtype)


# ---------------------------------------------------------------- attention


@pytest.mark.parametrize("n", [17, 64, 130, 300])
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_fp32(n, starting):
    # from n = 256 the projection stages its weights in LDS (n = 300: a
    # padded grid of 320)
    mod = seeded(TriangleAttention(128, 32, 4, starting=starting), 100 + n, STD)
    z = _z(n, 128, n)
    mask = token_pair_mask(n, max(1, n // 10))
    exp = ref.triangle_attention(z, mask, params_of(mod), 4, starting=starting)
    before = _lib.launch_count(_lib.K_TRIATT_CORE)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert _lib.launch_count(_lib.K_TRIATT_CORE) == before + 1
    assert_fp32(got, exp, f"triatt n={n} start={starting}")


@pytest.mark.parametrize("n", [17, 64, 130])
@pytest.mark.parametrize("starting", [True, False])
def test_triangle_attention_bf16(n, starting):
    mod = seeded(TriangleAttention(128, 32, 4, starting=starting), 200 + n, STD)
    z = _z(n, 128, n + 1, torch.bfloat16)
    mask = token_pair_mask(n, max(1, n // 10))
    exp = ref.triangle_attention(z.float(), mask, params_of(mod), 4, starting=starting)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert got.dtype == torch.bfloat16
    assert_bf16(got, exp, f"triatt bf16 n={n} start={starting}")


@pytest.mark.parametrize("c,h", [(64, 2), (256, 8), (384, 12)])
def test_triangle_attention_channel_shapes(c, h):
    n = 40
    mod = seeded(TriangleAttention(c, 32, h), 300 + c, STD)
    z = _z(n, c, c)
    mask = token_pair_mask(n, 3)
    exp = ref.triangle_attention(z, mask, params_of(mod), h)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="cuequivariance")
    assert_fp32(got, exp, f"triatt c={c} h={h}")


def _check_bf16_paths(c, h, starting, n):
    """z in bf16, and z in fp32 under bf16 autocast with an in-place
    residual add through the ending-node strides."""
    mod = seeded(TriangleAttention(c, 32, h, starting=starting), 800 + c + h + n, STD * 0.5)
    z = _z(n, c, c + h + n)
    mask = token_pair_mask(n, max(1, n // 10), seed=n + 2, random=True)
    zb = z.to(torch.bfloat16)
    exp = ref.triangle_attention(zb.float(), mask, params_of(mod), h, starting=starting)
    mod = mod.to(DEV)
    got = mod(zb.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert got.dtype == torch.bfloat16
    assert_bf16(got, exp, f"triatt bf16 c={c} h={h} n={n} start={starting}")
    # the block's form: a starting-node module applied through swapped strides
    mod.starting = True
    exp32 = ref.triangle_attention(z, mask, params_of(mod), h, starting=starting)
    z2 = z.to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        mod.hip_apply(z2, mask.to(DEV), transpose=not starting, out=z2, add_residual=True)
    assert_bf16(z2 - z.to(DEV), exp32, f"triatt fp32-z c={c} h={h} n={n} start={starting}")


@pytest.mark.parametrize("c,h", [(384, 12), (256, 8), (128, 8), (384, 4)])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("n", [40, 130])
def test_triangle_attention_wide_bf16(c, h, starting, n):
    """Wide channels (C or H*32 >= 256) take the LayerNorm-pass + NT GEMM
    projection and output."""
    _check_bf16_paths(c, h, starting, n)


@pytest.mark.parametrize("c,h", [(128, 4), (64, 2), (128, 2), (64, 4)])
@pytest.mark.parametrize("starting", [True, False])
@pytest.mark.parametrize("n", [40, 130])
def test_triangle_attention_weight_stationary_bf16(c, h, starting, n):
    """C and H*32 in {64, 128} take the weight-stationary projection and the
    output kernel with the gate (sigmoid(LN(z) W_g^T)) fused in, for z in
    bf16 and in fp32."""
    _check_bf16_paths(c, h, starting, n)


def test_triangle_attention_no_mask_and_in_place_add():
    n = 48
    mod = seeded(TriangleAttention(128, 32, 4), 7, STD).to(DEV)
    z = _z(n, 128, 8).to(DEV)
    upd = mod(z, None, triangle_attention="hip")
    exp = ref.triangle_attention(z.cpu(), None, params_of(mod), 4)
    assert_fp32(upd, exp, "triatt no mask")
    z2 = z.clone()
    out = mod.hip_apply(z2, None, out=z2, add_residual=True)
    assert out.data_ptr() == z2.data_ptr()
    assert_fp32(z2, z.cpu() + exp, "triatt in-place add")


def test_attention_core_slot_matches_oracle():
    # Attention.forward with the accelerated kwarg -> hip_triangular_attn slot
    n, c, h = 45, 128, 4
    tri = seeded(TriangleAttention(128, 32, 4), 11, STD)
    att = tri.mha
    x = torch.randn(n, n, c, generator=torch.Generator().manual_seed(12))
    mask = token_pair_mask(n, 5)
    mask_bias = (1e9 * (mask - 1))[..., :, None, None, :]
    tb = (x @ tri.linear.weight.t()).movedim(-1, -3).unsqueeze(-4)
    q = (x @ att.linear_q.weight.t()).view(n, n, h, 32).transpose(-2, -3) / 32 ** 0.5
    k = (x @ att.linear_k.weight.t()).view(n, n, h, 32).transpose(-2, -3)
    v = (x @ att.linear_v.weight.t()).view(n, n, h, 32).transpose(-2, -3)
    o = ref.attention_core(q, k, v, [mask_bias, tb]).transpose(-2, -3)
    g = torch.sigmoid(x @ att.linear_g.weight.t()).view(n, n, h, 32)
    exp = (o * g).reshape(n, n, h * 32) @ att.linear_o.weight.t()
    before = _lib.launch_count(_lib.K_TRIATT_RELAYOUT)
    att = att.to(DEV)
    got = att(x.to(DEV), x.to(DEV), biases=[mask_bias.to(DEV), tb.to(DEV)],
              triangle_attention="hip")
    assert _lib.launch_count(_lib.K_TRIATT_RELAYOUT) == before + 1
    assert_fp32(got, exp, "core slot")


# ---------------------------------------------------------- multiplication


@pytest.mark.parametrize("n", [17, 64, 130, 300])
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_fp32(n, outgoing):
    # from n = 256 the output kernel stages its weights in LDS (n = 300: a
    # padded grid of 320)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(128, 128), 400 + n, STD)
    z = _z(n, 128, 3 * n)
    mask = token_pair_mask(n, max(1, n // 10), seed=n, random=True)
    exp = ref.triangle_multiplication(z, mask, params_of(mod), outgoing)
    before = _lib.launch_count(_lib.K_TRIMUL_CONTRACT)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_multiplicative="hip")
    assert _lib.launch_count(_lib.K_TRIMUL_CONTRACT) == before + 1
    assert_fp32(got, exp, f"trimul n={n} out={outgoing}")


@pytest.mark.parametrize("n", [17, 64, 130])
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_bf16(n, outgoing):
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(128, 128), 500 + n, STD)
    z = _z(n, 128, 5 * n, torch.bfloat16)
    mask = token_pair_mask(n, max(1, n // 10), seed=n, random=True)
    exp = ref.triangle_multiplication(z.float(), mask, params_of(mod), outgoing)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_multiplicative="hip")
    assert_bf16(got, exp, f"trimul bf16 n={n} out={outgoing}")


@pytest.mark.parametrize("c,ch", [(64, 128), (64, 64), (384, 384), (128, 256)])
def test_triangle_multiplication_channel_shapes(c, ch):
    n = 40
    mod = seeded(TriangleMultiplicationIncoming(c, ch), 600 + c + ch, STD)
    z = _z(n, c, c + ch)
    exp = ref.triangle_multiplication(z, None, params_of(mod), False)
    got = mod.to(DEV)(z.to(DEV), None, triangle_multiplicative="hip")
    assert_fp32(got, exp, f"trimul c={c} ch={ch}")


@pytest.mark.parametrize("c,ch", [(64, 64), (64, 128), (128, 64)])
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_staged_weights_fp32(c, ch, outgoing):
    # n = 260 (from 256 the fp32 projection and output stage their weights
    # in LDS): C and Ch of 64 and 128
    n = 260
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(c, ch), 650 + c + ch, STD)
    z = _z(n, c, c + ch + 1)
    mask = token_pair_mask(n, 13, seed=n, random=True)
    exp = ref.triangle_multiplication(z, mask, params_of(mod), outgoing)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_multiplicative="hip")
    assert_fp32(got, exp, f"trimul staged n={n} c={c} ch={ch} out={outgoing}")


@pytest.mark.parametrize("c,h", [(64, 2), (128, 2), (64, 4)])
def test_triangle_attention_staged_weights_fp32(c, h):
    # n = 260: the fp32 projection stages its weights in LDS, for C of 64
    # and 128 and heads x 32 of 64 and 128
    n = 260
    mod = seeded(TriangleAttention(c, 32, h), 310 + c + h, STD)
    z = _z(n, c, c + h)
    mask = token_pair_mask(n, 13, seed=n + 1, random=True)
    exp = ref.triangle_attention(z, mask, params_of(mod), h)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert_fp32(got, exp, f"triatt staged n={n} c={c} h={h}")


@pytest.mark.parametrize("c,ch", [(384, 384), (256, 256), (128, 256), (384, 64)])
@pytest.mark.parametrize("outgoing", [True, False])
@pytest.mark.parametrize("n", [40, 130])
def test_triangle_multiplication_wide_bf16(c, ch, outgoing, n):
    """Wide channels (C or Ch >= 256) take the LayerNorm-pass + NT GEMM path;
    z in bf16, and z in fp32 under bf16 autocast with an in-place residual
    add."""
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(c, ch), 700 + c + ch + n, STD * 0.5)
    z = _z(n, c, c + 3 * ch + n)
    mask = token_pair_mask(n, max(1, n // 10), seed=n + 1, random=True)
    zb = z.to(torch.bfloat16)
    exp = ref.triangle_multiplication(zb.float(), mask, params_of(mod), outgoing)
    mod = mod.to(DEV)
    got = mod(zb.to(DEV), mask.to(DEV), triangle_multiplicative="hip")
    assert got.dtype == torch.bfloat16
    assert_bf16(got, exp, f"trimul wide bf16 c={c} ch={ch} n={n} out={outgoing}")
    exp32 = ref.triangle_multiplication(z, mask, params_of(mod), outgoing)
    z2 = z.to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod.hip_apply(z2, mask.to(DEV), out=z2, add_residual=True)
    assert got.data_ptr() == z2.data_ptr()
    assert_bf16(z2 - z.to(DEV), exp32, f"trimul wide fp32-z c={c} ch={ch} n={n} out={outgoing}")


@pytest.mark.parametrize("n", [70, 300])
def test_triangle_multiplication_in_place_add(n):
    # n = 70: the output kernel unsplit in place; n = 300: staged weights
    mod = seeded(TriangleMultiplicationOutgoing(128, 128), 9, STD).to(DEV)
    z = _z(n, 128, 10).to(DEV)
    mask = token_pair_mask(n, 6).to(DEV)
    exp = z.cpu() + ref.triangle_multiplication(z.cpu(), mask.cpu(), params_of(mod), True)
    z2 = z.clone()
    out = mod(z2, mask, inplace_safe=True, _add_with_inplace=True, triangle_multiplicative="hip")
    assert out.data_ptr() == z2.data_ptr()
    assert_fp32(z2, exp, f"trimul in-place add n={n}")


# ------------------------------------------------------------------- block


@pytest.mark.parametrize("inplace", [False, True])
def test_pairformer_block_fp32(inplace):
    n = 36
    blk = seeded(PairformerBlock(n_heads=16, c_z=128, c_s=384), 21, 0.05)
    g = torch.Generator().manual_seed(22)
    z = torch.randn(n, n, 128, generator=g)
    s = torch.randn(n, 384, generator=g)
    mask = token_pair_mask(n, 4)
    se, ze = ref.pairformer_block(s, z, mask, params_of(blk), no_heads_pair=4, n_heads=16)
    blk = blk.to(DEV)
    with torch.no_grad():
        sg, zg = blk(s.to(DEV), z.to(DEV).clone(), mask.to(DEV), triangle_multiplicative="hip",
                     triangle_attention="hip", inplace_safe=inplace)
    assert_fp32(zg, ze, "block z")
    assert_fp32(sg, se, "block s")


# ------------------------------------------- fast-path fallbacks (exact core)


def _rel(got, exp):
    g, e = got.double().cpu(), exp.double().cpu()
    return float((g - e).abs().max() / e.abs().max())


def test_triangle_attention_large_logits_take_exact_path():
    # weights large enough that |q| max|k| exceeds the fast path's overflow
    # bound: the rows are recomputed with a running max.
    # Only rows that keep some key are compared: for a fully masked row with
    # logits of hundreds of nats the reference's float32 result depends on how
    # -1e9 + logit rounds (ulp 64), not on a well-defined limit.
    n, pad = 72, 7
    mod = seeded(TriangleAttention(128, 32, 4), 31, 0.6)
    z = _z(n, 128, 32)
    mask = token_pair_mask(n, pad)
    exp = ref.triangle_attention(z, mask, params_of(mod), 4)
    exp64 = ref.triangle_attention(z.double(), mask.double(), params_of(mod, torch.float64), 4)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="hip")
    kept = slice(0, n - pad)
    r = _rel(got[kept], exp[kept])
    r_hip = _rel(got[kept], exp64[kept])
    r_ref = _rel(exp[kept], exp64[kept])
    say(f"    large-logit rel max err {r:.2e} vs the fp32 oracle; against float64: "
        f"HIP {r_hip:.2e}, fp32 oracle {r_ref:.2e}")
    margin("triatt large logits, kept rows, rel max err vs float64 [fp32]", hip=r_hip,
           fp32_oracle=r_ref)
    # logits of hundreds of nats: a 1e-7 relative rounding difference in a
    # logit moves its weight by ~1e-5, so the fp32 oracle itself is ~1.5e-5
    # from the float64 result; the HIP path must be as close to it as the
    # reference's own fp32 arithmetic (within 3x), where the overflowing fast
    # path would be off by orders of magnitude
    assert torch.isfinite(got).all() and r < 1e-3
    assert r_hip <= 3 * r_ref


def test_triangle_attention_underflowing_rows_take_exact_path():
    # LN offset 8 on every channel and tri-bias weights -0.5 make every logit
    # about -8*0.5*128 = -512 nats: exp2 of the raw logits underflows to 0 and
    # the rows must be recomputed with a running max.
    n = 40
    mod = seeded(TriangleAttention(128, 32, 4), 33, 0.05)
    with torch.no_grad():
        mod.layer_norm.bias.fill_(8.0)
        mod.linear.weight.fill_(-0.5)
    z = _z(n, 128, 34)
    exp = ref.triangle_attention(z, None, params_of(mod), 4)
    got = mod.to(DEV)(z.to(DEV), None, triangle_attention="hip")
    r = _rel(got, exp)
    say(f"    underflow rel max err {r:.2e}")
    assert torch.isfinite(got).all() and r < 1e-5


@pytest.mark.parametrize("n_pad", [0, 5, 39])
def test_triangle_attention_fully_masked_rows_are_mean_of_v(n_pad):
    # padded tokens give fully masked rows: the reference's float32 softmax of
    # identical -1e9 logits is uniform, i.e. the mean of v over all keys
    n = 40
    mod = seeded(TriangleAttention(128, 32, 4), 35, STD)
    z = _z(n, 128, 36)
    mask = token_pair_mask(n, n_pad)
    exp = ref.triangle_attention(z, mask, params_of(mod), 4)
    got = mod.to(DEV)(z.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert_fp32(got, exp, f"fully masked rows n_pad={n_pad}")


# -------------------------------------------------------------- transition


# c = 384 takes 128-row tiles with a split output GEMM up to 16384 rows (the
# single track) and 256-row tiles above: both sides of that boundary
@pytest.mark.parametrize("c,rows", [(128, 1000), (64, 257), (256, 130), (384, 1000), (384, 130),
                                    (384, 16384), (384, 20000)])
def test_transition_bf16(c, rows):
    from opendde_amd.pairformer import Transition
    # weights scaled so the output stays O(1) at every width (std ~0.6, max
    # ~3; the absolute bound of the bf16 tier is scale dependent)
    mod = seeded(Transition(c, 4), 700 + c, 0.7 * STD * (128 / c) ** 0.5)
    x = torch.randn(rows, c, generator=torch.Generator().manual_seed(c)).to(torch.bfloat16)
    exp = ref.transition(x.float(), params_of(mod))
    before = _lib.launch_count(_lib.K_TRANSITION)
    mod = mod.to(DEV)
    got = mod.hip_apply(x.to(DEV))
    assert _lib.launch_count(_lib.K_TRANSITION) == before + 1
    assert_bf16(got, exp, f"transition c={c} rows={rows}")


# at c = 64 and 128 from 16384 rows the weights are staged in LDS, shared by
# 64-row (4-wave) or, from 32768 rows, 128-row (8-wave) workgroup tiles: both
# forms, exact and ragged last tiles
@pytest.mark.parametrize("c,rows", [(128, 1000), (64, 257), (256, 130), (384, 130), (384, 17),
                                    (128, 16384), (128, 40000), (64, 16400), (64, 33000)])
def test_transition_fp32(c, rows):
    # fp32 arithmetic (no autocast): the fp32 tier's max-abs 1e-4
    from opendde_amd.pairformer import Transition
    mod = seeded(Transition(c, 4), 730 + c, 0.7 * STD * (128 / c) ** 0.5)
    x = torch.randn(rows, c, generator=torch.Generator().manual_seed(c + 1))
    exp = ref.transition(x, params_of(mod))
    before = _lib.launch_count(_lib.K_TRANSITION)
    mod = mod.to(DEV)
    xg = x.to(DEV)
    assert mod.hip_supported(xg)
    got = mod.hip_apply(xg)
    assert _lib.launch_count(_lib.K_TRANSITION) == before + 1
    assert got.dtype == torch.float32
    assert_fp32(got, exp, f"transition fp32 c={c} rows={rows}")
    # in place, with the residual
    got2 = mod.hip_apply(xg, out=xg, add_residual=True)
    assert got2.data_ptr() == xg.data_ptr()
    assert_fp32(got2, x + exp, f"transition fp32 in place c={c} rows={rows}")


@pytest.mark.parametrize("c,ln_offset,n", [(128, True, 37), (64, False, 37), (384, True, 37),
                                            (128, True, 131), (64, False, 182)])
def test_transition_fp32_pair_bias_projection(c, ln_offset, n):
    # the fp32 tier's pair bias from the fused epilogue, against the oracle
    # (n = 131 and 182: the LDS-staged forms)
    from opendde_amd.pairformer import AttentionPairBias, Transition
    tr = seeded(Transition(c, 4), 740, STD * (128 / c) ** 0.5)
    apb = seeded(AttentionPairBias(n_heads=16, c_a=384, c_z=c, create_offset_ln_z=ln_offset), 741,
                 0.1 * (128 / c) ** 0.5)
    x = torch.randn(n, n, c, generator=torch.Generator().manual_seed(7))
    z_new = x + ref.transition(x, params_of(tr))
    pz = params_of(apb)
    exp_bias = ref.linear(ref.layer_norm(z_new, pz["layernorm_z.weight"], pz.get("layernorm_z.bias")),
                          pz["linear_nobias_z.weight"]).permute(2, 0, 1)
    tr, apb = tr.to(DEV), apb.to(DEV)
    xg = x.to(DEV)
    dest = torch.full((16, n, n), float("nan"), device=DEV)
    out = tr.hip_apply(xg, out=xg, add_residual=True, pair_bias=apb.pair_bias_spec(dest.view(16, -1)))
    assert_fp32(out, z_new, f"fp32 transition update c={c}")
    assert_fp32(dest, exp_bias, f"fp32 pair bias c={c} offset={ln_offset}")


@pytest.mark.parametrize("c", [128, 384])
def test_transition_fp32_residual_under_autocast_in_place(c):
    from opendde_amd.pairformer import Transition
    mod = seeded(Transition(c, 4), 711, STD * (128 / c) ** 0.5).to(DEV)
    x = torch.randn(64, 64, c, generator=torch.Generator().manual_seed(3))
    exp = x + ref.transition(x, params_of(mod))
    xg = x.to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        assert mod.hip_supported(xg)
        out = mod.hip_apply(xg, out=xg, add_residual=True)
    assert out.data_ptr() == xg.data_ptr() and out.dtype == torch.float32
    assert_bf16(out - x.to(DEV), exp - x, "transition in-place update")


@pytest.mark.parametrize("x_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("c,ln_offset", [(128, True), (384, True), (384, False)])
def test_transition_pair_bias_projection(x_dtype, c, ln_offset):
    # the single track's pair bias linear_nobias_z(layernorm_z(z)) computed
    # from the rows the transition writes (fused epilogue at c = 128, a pass
    # after the GEMMs at c = 384)
    from opendde_amd.pairformer import AttentionPairBias, Transition
    n = 75  # 5625 rows: ragged against the row tiles
    # smaller transition weights keep z's update O(1): with bf16 storage the
    # written z also carries the rounding of |z| ~ 4 values (ulp 2^-5)
    tr = seeded(Transition(c, 4), 720, STD / 2 * (128 / c) ** 0.5)
    apb = seeded(AttentionPairBias(n_heads=16, c_a=384, c_z=c, create_offset_ln_z=ln_offset), 721,
                 0.1 * (128 / c) ** 0.5)
    x = torch.randn(n, n, c, generator=torch.Generator().manual_seed(5)).to(x_dtype)
    xf = x.float()
    z_new = xf + ref.transition(xf, params_of(tr))
    pz = params_of(apb)
    exp_bias = ref.linear(ref.layer_norm(z_new, pz["layernorm_z.weight"], pz.get("layernorm_z.bias")),
                          pz["linear_nobias_z.weight"]).permute(2, 0, 1)
    tr, apb = tr.to(DEV), apb.to(DEV)
    xg = x.to(DEV)
    dest = torch.full((16, n, n), float("nan"), device=DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        out = tr.hip_apply(xg, out=xg, add_residual=True,
                           pair_bias=apb.pair_bias_spec(dest.view(16, -1)))
    assert_bf16(out.float() - xf.to(DEV), z_new - xf, f"transition update ({x_dtype}, c={c})")
    assert_bf16(dest, exp_bias, f"pair bias ({x_dtype}, c={c}, offset={ln_offset})")


def test_pairformer_block_bf16_autocast():
    # the bench's mode: float32 residual stream, bf16 module arithmetic
    n = 70
    blk = seeded(PairformerBlock(n_heads=16, c_z=128, c_s=384), 41, 0.05)
    g = torch.Generator().manual_seed(42)
    z = torch.randn(n, n, 128, generator=g)
    s = torch.randn(n, 384, generator=g)
    mask = token_pair_mask(n, 6, seed=1, random=True)
    se, ze = ref.pairformer_block(s, z, mask, params_of(blk), no_heads_pair=4, n_heads=16)
    blk = blk.to(DEV)
    before = _lib.launch_count(_lib.K_TRANSITION)
    ln_z_calls = []
    hook = blk.attention_pair_bias.layernorm_z.register_forward_hook(
        lambda *_: ln_z_calls.append(1))
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        sg, zg = blk(s.to(DEV), z.to(DEV).clone(), mask.to(DEV), triangle_multiplicative="hip",
                     triangle_attention="hip", inplace_safe=True)
    hook.remove()
    # the pair transition (with the fused pair bias) and the single transition
    assert _lib.launch_count(_lib.K_TRANSITION) == before + 2
    assert not ln_z_calls, "pair bias should come from the fused transition epilogue"
    assert zg.dtype == torch.float32
    assert_bf16(zg - z.to(DEV), ze - z, "block update z (bf16 arithmetic)")
    assert_bf16(sg - s.to(DEV), se - s, "block update s (bf16 arithmetic)")


# ------------------------------------------------- bf16 accuracy of tri-mul
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_bf16_rounding_budget(outgoing):
    """The bf16 multiplication's input projections multiply LN_in(z) rounded
    to fp16 (11 mantissa bits) by the bf16 weights (exact in fp16), and
    LN_out is folded into W_z, so p enters the output projection as stored.
    With LN_in(z) rounded to bf16 and LN_out(p) rounded again, the relative
    error of the update against the fp32 oracle is about 5.0e-3 at this size;
    with them about 4.1e-3.  Over the 48-block trunk that margin is what
    keeps the accumulated update within max-abs 5e-2.  Also: without the f32
    copy of linear_z the fold rounds the weight twice and stays within the
    tier."""
    n = 192
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(128, 128), 900 + outgoing, 0.02)  # the workload's weight scale
    z = _z(n, 128, 901)
    exp = ref.triangle_multiplication(z, None, params_of(mod), outgoing)
    mod = mod.to(DEV)
    zg = z.to(DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got = mod.hip_apply(zg, None)
    rl = rel_l2(got, exp)
    say(f"    trimul bf16 n={n} out={outgoing} rel_l2={rl:.3e}")
    assert rl <= 4.6e-3, f"rel-L2 {rl:.3e}: bf16 rounding budget exceeded"
    from opendde_amd import kernels as K
    w = mod
    with torch.autocast("cuda", dtype=torch.bfloat16):
        got2 = K.triangle_multiplication(
            zg, None, outgoing=outgoing, norm_in_weight=w.layer_norm_in.weight,
            norm_in_bias=w.layer_norm_in.bias,
            p_in_weight=torch.cat([w.linear_a_p.weight, w.linear_b_p.weight]),
            g_in_weight=torch.cat([w.linear_a_g.weight, w.linear_b_g.weight]),
            norm_out_weight=w.layer_norm_out.weight, norm_out_bias=w.layer_norm_out.bias,
            p_out_weight=w.linear_z.weight, g_out_weight=w.linear_g.weight,
            f32_out_weight=False)
    assert_bf16(got2, exp, f"trimul bf16 without the f32 linear_z, out={outgoing}")
