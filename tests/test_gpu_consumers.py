"""GPU parity of the pair stack at the shapes of its other consumers.

The reference builds ``PairformerBlock`` / ``PairformerStack`` with other
dimensions outside the trunk (opendde/config/model_base.py:20-30,131-216;
``hidden_scale_up=True`` sets the triangle heads to c_z/32 and the
multiplication hidden width to c_z, modules/pairformer.py:91-93):
* the OpenDDE v1 trunk and the confidence head's stack: c_z = 384, c_s = 384,
  12 triangle heads, c_hidden_mul = 384 (confidence.py:98-104);
* the MSA module's pair stack: c_z = 384, c_s = 0 (pairformer.py:804-808);
* the template embedder's stack: c = 64, c_s = 0, 2 blocks, 2 heads,
  c_hidden_mul = 64 (pairformer.py:1678-1685).
Each runs through the HIP triangle kernels (and, in the bf16 mode, the HIP
pair transition: fused at c = 64, LayerNorm pass + two GEMMs at c = 384) and
is compared with the CPU oracle: fp32 to max-abs 1e-4, bf16 autocast to the
bf16 tier on the block's update.
"""

import pytest
import torch

from helpers import assert_bf16, assert_fp32, params_of, say, seeded, token_pair_mask
from oracle import reference as ref
from opendde_amd import _lib
from opendde_amd.pairformer import PairformerBlock, PairformerStack

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _fp32_matmul():
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = old
    torch.cuda.synchronize()


def _inputs(n, c_z, c_s, seed, n_pad):
    g = torch.Generator().manual_seed(seed)
    z = torch.randn(n, n, c_z, generator=g)
    s = torch.randn(n, c_s, generator=g) if c_s else None
    return z, s, token_pair_mask(n, n_pad, seed=seed, random=True)


def _run(mod, s, z, mask, autocast):
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16, enabled=autocast):
        return mod(None if s is None else s.to(DEV), z.to(DEV).clone(), mask.to(DEV),
                   triangle_multiplicative="hip", triangle_attention="hip", inplace_safe=True)


CONSUMERS = {
    # name: (c_z, c_s, n_blocks, expected triangle heads, n)
    "opendde_v1_trunk_block": (384, 384, 1, 12, 48),
    "msa_pair_stack_block": (384, 0, 1, 12, 40),
    "template_stack": (64, 0, 2, 2, 56),
    "confidence_stack": (384, 384, 2, 12, 36),
}


@pytest.mark.parametrize("autocast", [False, True], ids=["fp32", "bf16"])
@pytest.mark.parametrize("name", list(CONSUMERS))
def test_consumer_stack_matches_oracle(name, autocast):
    c_z, c_s, n_blocks, heads, n = CONSUMERS[name]
    say(f"[gpu] consumer {name} c_z={c_z} c_s={c_s} blocks={n_blocks} "
        f"{'bf16' if autocast else 'fp32'}")
    # weights ~ N(0, std^2) sized so the block updates are O(1) (std 0.2-0.8,
    # max 1-5) at every width, as in the trunk workload
    std = 0.035 if c_z == 384 else 0.05
    stack = seeded(PairformerStack(n_blocks=n_blocks, n_heads=16, c_z=c_z, c_s=c_s,
                                   hidden_scale_up=True), 50 + c_z + c_s, std)
    blk = stack.blocks[0]
    assert blk.tri_att_start.mha.no_heads == heads
    assert blk.tri_mul_out.c_hidden == c_z
    z, s, mask = _inputs(n, c_z, c_s, 60 + n, n // 8)
    p = params_of(stack)
    se, ze = ref.pairformer_stack(s, z, mask, p, n_blocks, no_heads_pair=heads, n_heads=16)
    stack = stack.to(DEV)
    before = (_lib.launch_count(_lib.K_TRIATT_CORE), _lib.launch_count(_lib.K_TRIMUL_CONTRACT),
              _lib.launch_count(_lib.K_TRANSITION))
    sg, zg = _run(stack, s, z, mask, autocast)
    torch.cuda.synchronize()
    assert _lib.launch_count(_lib.K_TRIATT_CORE) == before[0] + 2 * n_blocks
    assert _lib.launch_count(_lib.K_TRIMUL_CONTRACT) == before[1] + 2 * n_blocks
    # the HIP transition runs in both modes (bf16 and fp32 arithmetic), for
    # the pair track and (with c_s > 0) the single track
    per_block = 2 if c_s else 1
    assert _lib.launch_count(_lib.K_TRANSITION) == before[2] + per_block * n_blocks
    if autocast:
        assert_bf16(zg - z.to(DEV), ze - z, f"{name} z update")
        if c_s:
            assert_bf16(sg - s.to(DEV), se - s, f"{name} s update")
    else:
        assert_fp32(zg, ze, f"{name} z")
        if c_s:
            assert_fp32(sg, se, f"{name} s")


def test_template_stack_uses_fused_transition():
    """At c = 64 the pair transition also runs in HIP (bf16 arithmetic)."""
    say("[gpu] template stack transition launch")
    blk = seeded(PairformerBlock(c_z=64, c_s=0, hidden_scale_up=True), 77, 0.05).to(DEV)
    z, _, mask = _inputs(40, 64, 0, 78, 4)
    before = _lib.launch_count(_lib.K_TRANSITION)
    _run(blk, None, z, mask, True)
    torch.cuda.synchronize()
    assert _lib.launch_count(_lib.K_TRANSITION) == before + 1
