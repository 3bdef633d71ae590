"""GPU parity at the path's own workload sizes.

* N=128 PairformerBlock (c_s 384, 16 single heads), fp32 kernels vs the CPU
  oracle: max-abs <= 1e-4.
* N=384 triangle attention (starting node, last 38 tokens padded), bf16 vs
  the fp32 CPU oracle on the same bf16-rounded input.
* N=768 triangle multiplication, outgoing and incoming, bf16 vs the fp32 CPU
  oracle; N=1024 and 1200 (the large contraction tiles) vs the fp32 oracle
  run on the GPU.
* One block of the N=1024 trunk workload (51 random pads) in the bench's
  mode (fp32 residual, bf16 arithmetic) vs the oracle run in fp32 on the GPU
  (at this size the CPU oracle takes minutes), and one block at the shipped
  model's pair width (c_z 384, 12 heads, hidden 384) the same way; plus
  size-independent properties: the ending node through swapped strides
  equals the starting node on the transposed copy bit for bit, and repeated
  runs are bitwise deterministic.
* One block of the N=1024 trunk workload with fp32 arithmetic throughout
  (the reference's default inference precision) vs the oracle run in fp32 on
  the GPU: max-abs <= 1e-4 on the updates.
* N=2048, 4 blocks with the single track (c_s 384), bf16: runs without
  running out of memory and stays finite (every block's parity is in
  test_gpu_trunk.py).
"""

import pytest
import torch

from helpers import assert_bf16, assert_fp32, params_of, say, token_pair_mask
from oracle import reference as ref
from opendde_amd import _lib
from opendde_amd import workload as wl
from opendde_amd.pairformer import PairformerBlock, PairformerStack
from opendde_amd.triangular import (TriangleAttention, TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _fp32_checker():
    say("[gpu] config-size test")
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = old
    torch.cuda.synchronize()
    torch.cuda.empty_cache()


def _block(cfg, gen, c_s=None):
    c_s = cfg.c_s if c_s is None else c_s
    blk = PairformerBlock(n_heads=cfg.n_heads_single, c_z=cfg.c_z, c_s=c_s,
                          c_hidden_mul=cfg.c_hidden_mul, c_hidden_pair_att=cfg.head_dim,
                          no_heads_pair=cfg.heads)
    wl.init_module_(blk, gen)
    return blk.eval()


def test_block_n128_fp32():
    cfg = wl.BLOCK_N128
    z, s, mask, gen = wl.make_inputs(cfg)
    blk = _block(cfg, gen)
    say(f"    block n={cfg.n} fp32")
    se, ze = ref.pairformer_block(s, z, mask, params_of(blk), no_heads_pair=cfg.heads,
                                  n_heads=cfg.n_heads_single)
    blk = blk.to(DEV)
    before = _lib.launch_count(_lib.K_TRANSITION)
    with torch.no_grad():
        sg, zg = blk(s.to(DEV), z.to(DEV), mask.to(DEV), triangle_multiplicative="hip",
                     triangle_attention="hip")
    # the pair and single transitions both run on the fp32 HIP kernel
    assert _lib.launch_count(_lib.K_TRANSITION) == before + 2
    assert_fp32(zg, ze, "block n128 z")
    assert_fp32(sg, se, "block n128 s")


def test_triangle_attention_n384_bf16():
    cfg = wl.TRIATT_N384
    z, _, mask, gen = wl.make_inputs(cfg)
    mod = TriangleAttention(cfg.c_z, cfg.head_dim, cfg.heads)
    wl.init_module_(mod, gen)
    zb = z.to(torch.bfloat16)
    say(f"    triatt n={cfg.n} bf16 pads={cfg.n_pad}")
    exp = ref.triangle_attention(zb.float(), mask, params_of(mod), cfg.heads, chunk_size=64)
    got = mod.to(DEV)(zb.to(DEV), mask.to(DEV), triangle_attention="hip")
    assert got.dtype == torch.bfloat16
    assert_bf16(got, exp, "triatt n384 bf16")


@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_n768_bf16(outgoing):
    cfg = wl.TRIMUL_N768
    z, _, mask, gen = wl.make_inputs(cfg)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = cls(cfg.c_z, cfg.c_hidden_mul)
    wl.init_module_(mod, gen)
    zb = z.to(torch.bfloat16)
    say(f"    trimul n={cfg.n} bf16 outgoing={outgoing}")
    exp = ref.triangle_multiplication(zb.float(), mask, params_of(mod), outgoing)
    got = mod.to(DEV)(zb.to(DEV), mask.to(DEV), triangle_multiplicative="hip")
    assert_bf16(got, exp, f"trimul n768 bf16 outgoing={outgoing}")


def _gpu_params(mod):
    return {k: v.detach().float() for k, v in mod.named_parameters()}


@pytest.mark.parametrize("n", [740, 1024, 1200])
@pytest.mark.parametrize("outgoing", [True, False])
def test_triangle_multiplication_large_contraction_bf16(n, outgoing):
    """Np = 768, 1024 and 1280 (3 x 3, 4 x 4 and 5 x 5 tiles of 256 x 256)
    take the large contraction kernel (N = 740 with a random pad mask); bf16 z
    against the fp32 oracle run on the GPU."""
    gen = wl.generator(900 + n)
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = cls(128, 128)
    wl.init_module_(mod, gen)
    mod = mod.to(DEV)
    zb = torch.randn(n, n, 128, generator=gen).to(torch.bfloat16).to(DEV)
    mask = token_pair_mask(n, n // 20, seed=n, random=True).to(DEV)
    say(f"    trimul n={n} bf16 outgoing={outgoing} (large contraction tiles)")
    with torch.no_grad():
        exp = ref.triangle_multiplication(zb.float(), mask, _gpu_params(mod), outgoing)
        before = _lib.launch_count(_lib.K_TRIMUL_CONTRACT)
        got = mod(zb, mask, triangle_multiplicative="hip")
    assert _lib.launch_count(_lib.K_TRIMUL_CONTRACT) == before + 1
    assert_bf16(got, exp, f"trimul n={n} bf16 outgoing={outgoing}")


def test_trunk_block_n1024_bench_mode():
    cfg = wl.TRUNK_N1024
    z, s, mask, gen = wl.make_inputs(cfg)
    blk = _block(cfg, gen).to(DEV)
    z, s, mask = z.to(DEV), s.to(DEV), mask.to(DEV)
    say(f"    trunk block n={cfg.n} pads={cfg.n_pad}")
    with torch.no_grad():
        se, ze = ref.pairformer_block(s, z, mask, _gpu_params(blk), no_heads_pair=cfg.heads,
                                      n_heads=cfg.n_heads_single, chunk_size=64)
        runs = []
        for _ in range(2):
            with torch.autocast("cuda", dtype=torch.bfloat16):
                runs.append(blk(s, z.clone(), mask, triangle_multiplicative="hip",
                                triangle_attention="hip", inplace_safe=True))
    (sg, zg), (sg2, zg2) = runs
    assert torch.equal(zg, zg2) and torch.equal(sg, sg2), "block is not deterministic"
    assert_bf16(zg - z, ze - z, "trunk block z update")
    assert_bf16(sg - s, se - s, "trunk block s update")


def test_trunk_block_n1024_fp32():
    """One block of the benchmark workload (N=1024, 51 random pads, c_s 384)
    with fp32 arithmetic throughout -- the reference's default inference
    precision (opendde/config/model_base.py:36-37) -- in place, against the
    oracle run in fp32 on the GPU (TF32 off): max-abs <= 1e-4 on the updates."""
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    try:
        cfg = wl.TRUNK_N1024
        z, s, mask, gen = wl.make_inputs(cfg)
        blk = _block(cfg, gen).to(DEV)
        z, s, mask = z.to(DEV), s.to(DEV), mask.to(DEV)
        say(f"    fp32 trunk block n={cfg.n} pads={cfg.n_pad}")
        with torch.no_grad():
            se, ze = ref.pairformer_block(s, z, mask, _gpu_params(blk), no_heads_pair=cfg.heads,
                                          n_heads=cfg.n_heads_single, chunk_size=64)
            counts = [_lib.launch_count(k) for k in (_lib.K_TRIATT_CORE, _lib.K_TRIMUL_CONTRACT,
                                                     _lib.K_TRANSITION, _lib.K_BIAS_ATTN)]
            sg, zg = blk(s, z.clone(), mask, triangle_multiplicative="hip",
                         triangle_attention="hip", inplace_safe=True)
            torch.cuda.synchronize()
        after = [_lib.launch_count(k) for k in (_lib.K_TRIATT_CORE, _lib.K_TRIMUL_CONTRACT,
                                                _lib.K_TRANSITION, _lib.K_BIAS_ATTN)]
        assert [a - b for a, b in zip(after, counts)] == [2, 2, 2, 1]
        assert zg.dtype == torch.float32
        assert_fp32(zg - z, ze - z, "fp32 trunk block z update")
        assert_fp32(sg - s, se - s, "fp32 trunk block s update")
    finally:
        torch.backends.cuda.matmul.allow_tf32 = old


def test_opendde_v1_width_block_n1024_bench_mode():
    """One block at the shipped model's pair width (c_z 384, hidden_scale_up:
    12 triangle heads, multiplication hidden 384) at N = 1024 with 51 random
    pads, in the bench's mode: the wide kernels at their full size (256 x 256
    gate tiles, the transposing LayerNorm at Np = 1024, the large contraction
    tiles) against the oracle run in fp32 on the GPU."""
    cfg = wl.PairConfig("opendde_v1_block_n1024", 1024, c_z=384, heads=12,
                        c_hidden_mul=384, n_pad=51, random_pad=True, seed=3)
    z, s, mask, gen = wl.make_inputs(cfg)
    blk = PairformerBlock(n_heads=cfg.n_heads_single, c_z=cfg.c_z, c_s=cfg.c_s,
                          hidden_scale_up=True)
    wl.init_module_(blk, gen)
    blk = blk.eval().to(DEV)
    assert blk.tri_att_start.mha.no_heads == 12 and blk.tri_mul_out.c_hidden == 384
    z, s, mask = z.to(DEV), s.to(DEV), mask.to(DEV)
    say(f"    v1-width block n={cfg.n} c_z={cfg.c_z} pads={cfg.n_pad}")
    with torch.no_grad():
        se, ze = ref.pairformer_block(s, z, mask, _gpu_params(blk), no_heads_pair=12,
                                      n_heads=cfg.n_heads_single, chunk_size=32)
        with torch.autocast("cuda", dtype=torch.bfloat16):
            sg, zg = blk(s, z.clone(), mask, triangle_multiplicative="hip",
                         triangle_attention="hip", inplace_safe=True)
    assert_bf16(zg - z, ze - z, "v1-width block z update")
    assert_bf16(sg - s, se - s, "v1-width block s update")


def test_ending_node_strides_equal_transposed_starting_node_n1024():
    cfg = wl.TRUNK_N1024
    z, _, mask, gen = wl.make_inputs(cfg, with_s=False)
    mod = TriangleAttention(cfg.c_z, cfg.head_dim, cfg.heads)
    wl.init_module_(mod, gen)
    mod = mod.to(DEV)
    zb, m = z.to(DEV).to(torch.bfloat16), mask.to(DEV)
    say("    ending node via strides vs transposed copy, n=1024")
    end = mod.hip_apply(zb, m, transpose=True)
    start_t = mod.hip_apply(zb.transpose(0, 1).contiguous(), m.t().contiguous())
    assert torch.equal(end, start_t.transpose(0, 1)), "orientation symmetry is not exact"


def test_stress_n2048_four_blocks():
    """N=2048 x 4 blocks with the single track (c_s 384): the pair-bias
    epilogue and the single-track attention core at the bias's largest size
    ([16, 2048, 2048] fp32)."""
    cfg = wl.STRESS_N2048
    z, s, mask, gen = wl.make_inputs(cfg)
    stack = PairformerStack(n_blocks=cfg.n_blocks, n_heads=cfg.n_heads_single, c_z=cfg.c_z,
                            c_s=cfg.c_s)
    wl.init_module_(stack, gen)
    stack = stack.eval().to(DEV)
    z, s, mask = z.to(DEV), s.to(DEV), mask.to(DEV)
    say(f"    stress n={cfg.n} blocks={cfg.n_blocks} c_s={cfg.c_s}")
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()
    base = torch.cuda.memory_allocated()
    before = _lib.launch_count(_lib.K_BIAS_ATTN)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        ss, zs = stack(s, z.clone(), mask, triangle_multiplicative="hip",
                       triangle_attention="hip", inplace_safe=True)
    torch.cuda.synchronize()
    peak = (torch.cuda.max_memory_allocated() - base) / 2 ** 30
    say(f"    n=2048 4 blocks: peak {peak:.1f} GiB above the inputs")
    assert _lib.launch_count(_lib.K_BIAS_ATTN) == before + cfg.n_blocks
    assert torch.isfinite(zs).all() and torch.isfinite(ss).all()
    assert peak < 32, f"peak memory {peak:.1f} GiB"
    # parity of all four blocks against the fp32 oracle: test_gpu_trunk.py
