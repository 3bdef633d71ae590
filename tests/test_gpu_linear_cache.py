"""The single track's linears under bf16 autocast take bf16 weights cast once
per parameter version (layers.Linear) instead of on every call: the result
must be exactly what autocast's own F.linear gives, and an in-place weight
update must be seen."""

import pytest
import torch
import torch.nn.functional as F

from helpers import say, seeded
from opendde_amd.layers import Linear, LinearNoBias
from opendde_amd.pairformer import SingleAttention

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("bias", [True, False])
def test_linear_under_autocast_equals_autocast_linear(bias):
    say(f"[gpu] cached bf16 linear bias={bias}")
    lin = seeded((Linear if bias else LinearNoBias)(384, 384), 3).to(DEV)
    if bias:
        with torch.no_grad():
            lin.bias.normal_(0, 0.1)
    x = torch.randn(1024, 384, device=DEV)
    for _ in range(2):
        with torch.autocast("cuda", dtype=torch.bfloat16):
            got = lin(x)
            exp = F.linear(x, lin.weight, lin.bias)
        assert got.dtype == torch.bfloat16 and torch.equal(got, exp)
        with torch.no_grad():
            lin.weight.mul_(1.5)  # a new version: the cached copy must not be reused


@pytest.mark.parametrize("bias", [True, False])
def test_linear_under_autocast_trains_its_parameters(bias):
    """With gradients on, the cached (detached) casts must not be used: the
    backward reaches weight and bias exactly as autocast's F.linear does."""
    say(f"[gpu] linear backward under autocast bias={bias}")
    lin = seeded((Linear if bias else LinearNoBias)(384, 256), 5).to(DEV)
    x = torch.randn(512, 384, device=DEV, requires_grad=True)
    gy = torch.randn(512, 256, device=DEV)
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y = lin(x)
    y.backward(gy.to(y.dtype))
    assert lin.weight.grad is not None and x.grad is not None
    if bias:
        assert lin.bias.grad is not None
    got = [lin.weight.grad.clone(), x.grad.clone()] + ([lin.bias.grad.clone()] if bias else [])
    lin.zero_grad()
    x.grad = None
    with torch.autocast("cuda", dtype=torch.bfloat16):
        y2 = F.linear(x, lin.weight, lin.bias)
    y2.backward(gy.to(y2.dtype))
    exp = [lin.weight.grad, x.grad] + ([lin.bias.grad] if bias else [])
    assert torch.equal(y, y2)
    for g, e in zip(got, exp):
        assert torch.equal(g, e)


def test_single_attention_shared_cast_is_bit_identical():
    say("[gpu] single attention with one shared bf16 input cast")
    att = seeded(SingleAttention(384, 384, 384, 24, 16), 4).to(DEV)
    with torch.no_grad():
        att.linear_o.weight.normal_(0, 0.02)
        att.linear_g.weight.normal_(0, 0.02)
    a = torch.randn(200, 384, device=DEV)
    bias = torch.randn(16, 200, 200, device=DEV)

    def plain(m, q_x):  # the same forward without the shared cast or the weight cache
        def heads(t):
            return t.view(t.shape[:-1] + (m.num_heads, -1)).transpose(-2, -3)
        q = heads(F.linear(q_x, m.linear_q.weight, m.linear_q.bias)) / (m.c_hidden ** 0.5)
        k = heads(F.linear(q_x, m.linear_k.weight))
        v = heads(F.linear(q_x, m.linear_v.weight))
        o = F.scaled_dot_product_attention(q.float(), k.float(), v.float(),
                                           attn_mask=bias.float(), scale=1.0).to(q.dtype)
        o = o.transpose(-2, -3)
        g = torch.sigmoid(F.linear(q_x, m.linear_g.weight))
        o = o * g.view(g.shape[:-1] + (m.num_heads, -1))
        return F.linear(o.reshape(o.shape[:-2] + (-1,)), m.linear_o.weight)

    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        got = att(a, a, attn_bias=bias, hip=False)
        exp = plain(att, a)
    assert torch.equal(got, exp)
