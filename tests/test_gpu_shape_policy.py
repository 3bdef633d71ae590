"""Calls outside the fused kernels' coverage, and leading batch dims.

Policy, the reference's (opendde/model/triangular/layers.py:455-468,
triangular.py:482-486): an accelerated request on a GPU tensor whose shape or
dtype the kernels do not cover runs the module's torch path.  Its result
equals the ``"torch"`` request's bit for bit, and no kernel of the library
launches.  Leading batch dims run as one library call per module, and its
output equals the per-view calls bit for bit (the same kernels on the same
views; the workspace is shared in stream order).
"""

import math

import pytest
import torch

from helpers import say, seeded, token_pair_mask
from opendde_amd import _lib
from opendde_amd import workload as wl
from opendde_amd.pairformer import PairformerBlock
from opendde_amd.triangular import (Attention, TriangleAttention,
                                    TriangleMultiplicationIncoming,
                                    TriangleMultiplicationOutgoing, kernel_triangular_mult)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _launches():
    return [_lib.launch_count(k) for k in _lib.KERNEL_NAMES]


def _pair(n, c, dtype=torch.float32, seed=0, lead=()):
    g = wl.generator(seed)
    return torch.randn(tuple(lead) + (n, n, c), generator=g).to(DEV, dtype)


def _hip_equals_torch(run, what):
    """run(kernel_name) -> tensor; the 'hip' request must take the torch path."""
    say(f"[gpu] shape policy: {what}")
    before = _launches()
    got = run("hip")
    torch.cuda.synchronize()
    assert _launches() == before, f"{what}: a library kernel launched"
    exp = run("torch")
    assert torch.equal(got, exp), f"{what}: hip request differs from the torch path"


def test_attention_head_dim_16_runs_torch_path():
    mod = seeded(TriangleAttention(c_in=128, c_hidden=16, no_heads=4), 1).to(DEV)
    z, mask = _pair(40, 128), token_pair_mask(40, 5).to(DEV)
    with torch.no_grad():
        _hip_equals_torch(lambda k: mod(z, mask=mask, triangle_attention=k), "head dim 16")


def test_attention_unsupported_channels_run_torch_path():
    mod = seeded(TriangleAttention(c_in=96, c_hidden=32, no_heads=4, starting=False), 2).to(DEV)
    z, mask = _pair(40, 96), token_pair_mask(40, 3).to(DEV)
    with torch.no_grad():
        _hip_equals_torch(lambda k: mod(z, mask=mask, triangle_attention=k), "attention c=96")


def test_multiplication_unsupported_hidden_runs_torch_path():
    mod = seeded(TriangleMultiplicationOutgoing(c_z=128, c_hidden=96), 3).to(DEV)
    z, mask = _pair(40, 128), token_pair_mask(40, 4).to(DEV)
    with torch.no_grad():
        _hip_equals_torch(lambda k: mod(z, mask=mask, triangle_multiplicative=k),
                          "multiplication c_hidden=96")


def test_fp16_runs_torch_path():
    mod = seeded(TriangleMultiplicationIncoming(c_z=128, c_hidden=128), 4).to(DEV).half()
    z, mask = _pair(40, 128, torch.float16), token_pair_mask(40, 2).to(DEV, torch.float16)
    with torch.no_grad():
        _hip_equals_torch(lambda k: mod(z, mask=mask, triangle_multiplicative=k), "fp16 z")


def test_attention_slot_head_dim_16_runs_torch_path():
    """The reference's Attention with the accelerated slot requested and a
    per-head dim the core does not take (layers.py:455-481)."""
    mha = seeded(Attention(64, 64, 64, 16, 4), 5).to(DEV)
    x = _pair(24, 64, seed=6)[:, :, :]
    g = wl.generator(7)
    mask_bias = (1e9 * (token_pair_mask(24, 3).to(DEV) - 1))[:, None, None, :]
    tri_bias = torch.randn(1, 4, 24, 24, generator=g).to(DEV)
    with torch.no_grad():
        _hip_equals_torch(lambda k: mha(x, x, biases=[mask_bias, tri_bias], triangle_attention=k),
                          "attention slot head dim 16")


def test_block_unsupported_channels_runs_torch_path():
    """c_z = 96: every pair module (both multiplications, both attentions and
    the transition) is outside the kernels' channel set."""
    blk = seeded(PairformerBlock(n_heads=16, c_z=96, c_s=0, c_hidden_mul=96,
                                 c_hidden_pair_att=32, no_heads_pair=4), 8).to(DEV)
    z, mask = _pair(32, 96, seed=9), token_pair_mask(32, 4).to(DEV)
    with torch.no_grad():
        _hip_equals_torch(lambda k: blk(None, z.clone(), mask, triangle_multiplicative=k,
                                        triangle_attention=k)[1], "block c_z=96")


def _count_calls(monkeypatch, name):
    lib = _lib.load()
    orig = getattr(lib, name)
    calls = []

    def wrapped(*args):
        calls.append(1)
        return orig(*args)

    monkeypatch.setattr(lib, name, wrapped)
    return calls


@pytest.mark.parametrize("dtype,transpose", [(torch.bfloat16, False), (torch.float32, True)])
def test_batched_triangle_attention_is_one_call(monkeypatch, dtype, transpose):
    n, c = 72, 128
    mod = seeded(TriangleAttention(c_in=c, c_hidden=32, no_heads=4), 10).to(DEV)
    z = _pair(n, c, dtype, seed=11, lead=(2, 1))
    mask = torch.stack([token_pair_mask(n, 5), token_pair_mask(n, 9, seed=1, random=True)])
    mask = mask[:, None].to(DEV)  # [2, 1, N, N]: a different mask per view
    say(f"[gpu] batched triangle attention {dtype} transpose={transpose}")
    with torch.no_grad():
        per = torch.stack([mod.hip_apply(z[b, 0], mask[b, 0], transpose=transpose)
                           for b in range(2)])[:, None]
        calls = _count_calls(monkeypatch, "odde_triatt_fwd")
        got = mod.hip_apply(z, mask, transpose=transpose)
        assert len(calls) == 1
        assert torch.equal(got, per)
        # a broadcast [N, N] mask (batch stride 0) and the in-place residual form
        per_b = []
        for b in range(2):
            zb = z[b, 0].clone()
            per_b.append(mod.hip_apply(zb, mask[0, 0], transpose=transpose, out=zb,
                                       add_residual=True))
        zi = z.clone()
        mod.hip_apply(zi, mask[0, 0], transpose=transpose, out=zi, add_residual=True)
        assert torch.equal(zi, torch.stack(per_b)[:, None])
        assert not torch.equal(zi, z)


@pytest.mark.parametrize("outgoing,dtype", [(True, torch.bfloat16), (False, torch.float32)])
def test_batched_triangle_multiplication_is_one_call(monkeypatch, outgoing, dtype):
    n, c = 72, 128
    cls = TriangleMultiplicationOutgoing if outgoing else TriangleMultiplicationIncoming
    mod = seeded(cls(c_z=c, c_hidden=128), 12).to(DEV)
    z = _pair(n, c, dtype, seed=13, lead=(3,))
    mask = torch.stack([token_pair_mask(n, p, seed=p, random=True) for p in (0, 6, 11)]).to(DEV)
    say(f"[gpu] batched triangle multiplication outgoing={outgoing} {dtype}")
    with torch.no_grad():
        per = torch.stack([mod.hip_apply(z[b], mask[b]) for b in range(3)])
        calls = _count_calls(monkeypatch, "odde_trimul_fwd")
        got = mod(z, mask=mask, triangle_multiplicative="hip")
        assert len(calls) == 1
        assert torch.equal(got, per)
        assert math.isfinite(float(got.float().abs().max()))


def test_permuted_batch_runs_on_a_copy(monkeypatch):
    """Leading dims that no view collapses (a permuted 2-D batch): the modules
    run the kernels on a contiguous copy (one library call) instead of
    raising, and the in-place form writes the result back into z."""
    n, c = 40, 128
    att = seeded(TriangleAttention(c_in=c, c_hidden=32, no_heads=4), 14).to(DEV)
    mul = seeded(TriangleMultiplicationOutgoing(c_z=c, c_hidden=128), 15).to(DEV)
    base = _pair(n, c, seed=16, lead=(3, 2))
    z = base.transpose(0, 1)  # [2, 3, N, N, C], not collapsible by a view
    mask = token_pair_mask(n, 4).to(DEV)
    say("[gpu] permuted 2-D batch")
    with torch.no_grad():
        exp_att = att.hip_apply(z.contiguous(), mask)
        calls = _count_calls(monkeypatch, "odde_triatt_fwd")
        got_att = att(z, mask=mask, triangle_attention="hip")
        assert len(calls) == 1 and torch.equal(got_att, exp_att)
        exp_mul = z.contiguous()
        mul.hip_apply(exp_mul, mask, out=exp_mul, add_residual=True)
        zi = z.clone().transpose(0, 1).contiguous().transpose(0, 1)  # same permuted layout
        calls = _count_calls(monkeypatch, "odde_trimul_fwd")
        got = mul(zi, mask=mask, inplace_safe=True, _add_with_inplace=True,
                  triangle_multiplicative="hip")
        assert len(calls) == 1 and got is zi and torch.equal(zi, exp_mul)


def test_kernel_triangular_mult_slot_is_one_call(monkeypatch):
    """The reference's function slot with leading dims: one library call with
    batch strides, equal to the per-view calls bit for bit."""
    n, c = 48, 128
    mod = seeded(TriangleMultiplicationIncoming(c_z=c, c_hidden=128), 17).to(DEV)
    x = _pair(n, c, torch.bfloat16, seed=18, lead=(2, 2))
    mask = token_pair_mask(n, 6, seed=2, random=True).to(DEV, torch.bfloat16)
    p_in = torch.cat([mod.linear_a_p.weight, mod.linear_b_p.weight]).bfloat16()
    g_in = torch.cat([mod.linear_a_g.weight, mod.linear_b_g.weight]).bfloat16()
    args = (mod.layer_norm_in.weight, mod.layer_norm_in.bias, p_in, g_in,
            mod.layer_norm_out.weight, mod.layer_norm_out.bias, mod.linear_z.weight.bfloat16(),
            mod.linear_g.weight.bfloat16(), 1e-5)
    say("[gpu] kernel_triangular_mult slot, leading dims (2, 2)")
    with torch.no_grad():
        per = torch.stack([torch.stack([kernel_triangular_mult(x[a, b], "incoming", mask, *args)
                                        for b in range(2)]) for a in range(2)])
        calls = _count_calls(monkeypatch, "odde_trimul_fwd")
        got = kernel_triangular_mult(x, "incoming", mask, *args)
        assert len(calls) == 1
        assert got.shape == x.shape and torch.equal(got, per)
