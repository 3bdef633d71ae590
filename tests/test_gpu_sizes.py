"""Pair sizes at and around the kernels' tile edges, down to one token.

The kernels tile pairs in 16-, 64- and 128-row blocks, keys in 32-key blocks
padded to 64, and the contraction in 128- and 256-wide tiles (rows padded to
128).  Every module is compared with the oracle at N on either side of those
edges, including N = 1 and 2 (a single pair row, a single key block mostly
padding), in fp32 arithmetic (max-abs <= 1e-4) and bf16 arithmetic under
autocast with an fp32 z (the bench's mode; the bf16 tier on the update).
The token mask pads the last token where N > 2, so every size also has a
fully masked row and column.
"""

import pytest
import torch

from helpers import assert_bf16, assert_fp32, params_of, say, seeded, token_pair_mask
from oracle import reference as ref
from opendde_amd.pairformer import PairformerBlock
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing)

pytestmark = pytest.mark.gpu
DEV = "cuda"
SIZES = [1, 2, 3, 15, 16, 33, 63, 65, 127, 129, 255, 257]


def _inputs(n, seed):
    z = torch.randn(n, n, 128, generator=torch.Generator().manual_seed(seed))
    mask = token_pair_mask(n, 1 if n > 2 else 0)
    return z, mask


@pytest.mark.parametrize("n", SIZES)
@pytest.mark.parametrize("kind", ["att_start", "att_end", "mul_out", "mul_in"])
def test_module_sizes(n, kind):
    say(f"[gpu] size sweep {kind} n={n}")
    z, mask = _inputs(n, 1000 + n)
    if kind.startswith("att"):
        mod = seeded(TriangleAttention(128, 32, 4, starting=kind == "att_start"), n, 0.1)
        exp = ref.triangle_attention(z, mask, params_of(mod), 4, starting=kind == "att_start")
        run = lambda m, x: m(x, mask.to(DEV), triangle_attention="hip")  # noqa: E731
    else:
        mod = seeded((TriangleMultiplicationOutgoing if kind == "mul_out"
                      else TriangleMultiplicationIncoming)(128, 128), n, 0.1)
        exp = ref.triangle_multiplication(z, mask, params_of(mod), outgoing=kind == "mul_out")
        run = lambda m, x: m(x, mask.to(DEV), triangle_multiplicative="hip")  # noqa: E731
    mod = mod.to(DEV)
    with torch.no_grad():
        got = run(mod, z.to(DEV))
        assert_fp32(got, exp, f"{kind} n={n}")
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got16 = run(mod, z.to(DEV))
    assert got16.dtype == torch.float32
    assert_bf16(got16, exp, f"{kind} bf16 n={n}")


@pytest.mark.parametrize("n", [1, 2, 17, 65, 129])
def test_block_sizes(n):
    """A whole block (c_s 384, 16 single heads) in fp32 and in the bench's mode."""
    say(f"[gpu] size sweep block n={n}")
    z, mask = _inputs(n, 2000 + n)
    s = torch.randn(n, 384, generator=torch.Generator().manual_seed(3000 + n))
    blk = seeded(PairformerBlock(n_heads=16, c_z=128, c_s=384), 4000 + n, 0.05)
    se, ze = ref.pairformer_block(s, z, mask, params_of(blk), no_heads_pair=4, n_heads=16)
    blk = blk.to(DEV)
    with torch.no_grad():
        sg, zg = blk(s.to(DEV), z.to(DEV), mask.to(DEV), triangle_multiplicative="hip",
                     triangle_attention="hip", inplace_safe=True)
        assert_fp32(zg, ze, f"block n={n} z")
        assert_fp32(sg, se, f"block n={n} s")
        with torch.autocast("cuda", dtype=torch.bfloat16):
            sb, zb = blk(s.to(DEV), z.to(DEV), mask.to(DEV), triangle_multiplicative="hip",
                         triangle_attention="hip", inplace_safe=True)
    assert_bf16(zb - z.to(DEV), ze - z, f"block bf16 n={n} z update")
    assert_bf16(sb - s.to(DEV), se - s, f"block bf16 n={n} s update")
