"""A NaN in the pair tensor: the HIP path must put NaN exactly where the
reference's torch arithmetic does (the oracle restates it), and leave every
other element within the tier's tolerance.

The library is compiled with ``-fno-honor-nans`` (no NaN quieting around
v_max); this pins that the fused kernels still propagate a NaN input through
LayerNorm, the projections, the contraction, both attention cores and the
transition to the same rows and columns as the reference (a NaN in z[i0, j0]
spreads to row i0 and column i0 of the update).  All tokens are kept here: a
padded row's output is the uniform softmax's mean(V), which no bias reaches,
so a NaN bias would not reach it either, while the reference's -1e9 + NaN
would.
"""

import pytest
import torch

from helpers import BF16_MAX_ABS, FP32_MAX_ABS, params_of, say, seeded
from oracle import reference as ref
from opendde_amd.pairformer import PairformerBlock, Transition
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing)

pytestmark = pytest.mark.gpu
DEV = "cuda"
N, C = 48, 128
I0, J0, C0 = 5, 17, 9


def _z(seed=0):
    z = torch.randn(N, N, C, generator=torch.Generator().manual_seed(seed))
    z[I0, J0, C0] = float("nan")
    return z


def _check(got, exp, tol, what):
    got = got.float().cpu()
    gn, en = torch.isnan(got), torch.isnan(exp)
    say(f"    {what}: NaN at {int(en.sum())} reference positions, {int(gn.sum())} here")
    assert int(en.sum()) > 0, f"{what}: the NaN did not reach the reference's output"
    assert torch.equal(gn, en), f"{what}: NaN positions differ"
    fin = ~en
    if not bool(fin.any()):
        return  # the NaN reached every element (a whole block spreads it everywhere)
    assert torch.isfinite(got[fin]).all(), f"{what}: an Inf appeared"
    ma = float((got[fin] - exp[fin]).abs().max())
    assert ma <= tol, f"{what}: max-abs {ma:.3e} on the finite elements"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("kind", ["mul_out", "mul_in", "att_start", "att_end", "transition"])
def test_nan_in_z_reaches_the_same_positions(kind, bf16):
    say(f"[gpu] NaN propagation {kind} bf16={bf16}")
    z = _z()
    mask = torch.ones(N, N)
    if kind.startswith("mul"):
        mod = seeded((TriangleMultiplicationOutgoing if kind == "mul_out"
                      else TriangleMultiplicationIncoming)(C, 128), 1, 0.1)
        exp = ref.triangle_multiplication(z, mask, params_of(mod), outgoing=kind == "mul_out")
        run = lambda m, x: m(x, mask.to(DEV), triangle_multiplicative="hip")
    elif kind.startswith("att"):
        mod = seeded(TriangleAttention(C, 32, 4, starting=kind == "att_start"), 2, 0.1)
        exp = ref.triangle_attention(z, mask, params_of(mod), 4, starting=kind == "att_start")
        run = lambda m, x: m(x, mask.to(DEV), triangle_attention="hip")
    else:
        mod = seeded(Transition(C, 4), 3, 0.1)
        exp = ref.transition(z, params_of(mod))
        run = lambda m, x: m.hip_apply(x)
    mod = mod.to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=bf16):
        got = run(mod, z.to(DEV))
    _check(got, exp, BF16_MAX_ABS if bf16 else FP32_MAX_ABS, kind)


def test_nan_in_z_through_a_block():
    """One whole block in the bench's mode (fp32 residual, bf16 arithmetic,
    in place): z and the single track s."""
    say("[gpu] NaN propagation through a block")
    blk = seeded(PairformerBlock(n_heads=16, c_z=C, c_s=384), 4, 0.05)
    z = _z(1)
    s = torch.randn(N, 384, generator=torch.Generator().manual_seed(2))
    mask = torch.ones(N, N)
    se, ze = ref.pairformer_block(s, z, mask, params_of(blk), no_heads_pair=4, n_heads=16)
    blk = blk.to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        sg, zg = blk(s.to(DEV), z.to(DEV), mask.to(DEV), triangle_multiplicative="hip",
                     triangle_attention="hip", inplace_safe=True)
    _check(zg - z.to(DEV), ze - z, BF16_MAX_ABS, "block z")
    _check(sg - s.to(DEV), se - s, BF16_MAX_ABS, "block s")
