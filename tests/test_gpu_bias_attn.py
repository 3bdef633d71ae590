"""GPU parity of the single track's fp32 attention core with an additive
pair bias (primitives._attention, opendde/model/modules/primitives.py:
220-258: q, k, v and the bias upcast to fp32, SDPA with scale 1), as used by
AttentionPairBias (16 heads of 24 at c_s = 384).

Against the oracle's attention core in float64 on the CPU (fp32 inputs:
max-abs <= 1e-4 for O(1) outputs); bf16 inputs are compared with the same
float64 attention of the bf16-rounded inputs, at the bf16 rounding of the
output.  Cases: every supported head dim, ragged query and key counts
against the 64-query / 64-key blocks, no bias, and strided q, k, v views
(the heads of a [N, H*D] projection) at the pair stack's size.
"""

import pytest
import torch

from helpers import say
from oracle import reference as ref
from opendde_amd import _lib, kernels as K

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(h, nq, nk, d, seed, bias=True):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(h, nq, d, generator=g) / d ** 0.5
    k = torch.randn(h, nk, d, generator=g)
    v = torch.randn(h, nk, d, generator=g)
    b = torch.randn(h, nq, nk, generator=g) * 2.0 if bias else None
    return q, k, v, b


def _expected(q, k, v, b):
    biases = [] if b is None else [b.double()]
    return ref.attention_core(q.double(), k.double(), v.double(), biases).float()


@pytest.mark.parametrize("h,nq,nk,d", [(3, 17, 130, 24), (2, 64, 64, 8), (4, 100, 37, 16),
                                       (1, 129, 200, 32), (2, 70, 65, 48), (2, 33, 128, 64),
                                       # key blocks split unevenly over the four key groups
                                       (2, 40, 300, 32), (1, 64, 513, 24)])
def test_bias_attention_fp32_matches_oracle(h, nq, nk, d):
    say(f"[gpu] bias attn h={h} nq={nq} nk={nk} d={d}")
    q, k, v, b = _inputs(h, nq, nk, d, 10 + nq + d)
    exp = _expected(q, k, v, b)
    before = _lib.launch_count(_lib.K_BIAS_ATTN)
    got = K.bias_attention(q.to(DEV), k.to(DEV), v.to(DEV), b.to(DEV)).cpu()
    assert _lib.launch_count(_lib.K_BIAS_ATTN) == before + 1
    torch.testing.assert_close(got, exp, rtol=0, atol=1e-4)


def test_bias_attention_no_bias_and_bf16_inputs():
    say("[gpu] bias attn no bias / bf16")
    q, k, v, _ = _inputs(2, 90, 77, 24, 5, bias=False)
    exp = _expected(q, k, v, None)
    got = K.bias_attention(q.to(DEV), k.to(DEV), v.to(DEV), None).cpu()
    torch.testing.assert_close(got, exp, rtol=0, atol=1e-4)
    q, k, v, b = _inputs(3, 50, 140, 24, 6)
    qb, kb, vb = (t.to(torch.bfloat16) for t in (q, k, v))
    exp = _expected(qb.float(), kb.float(), vb.float(), b)
    got = K.bias_attention(qb.to(DEV), kb.to(DEV), vb.to(DEV), b.to(DEV))
    assert got.dtype == torch.bfloat16
    torch.testing.assert_close(got.float().cpu(), exp, rtol=1e-2, atol=1e-2)


def test_bias_attention_strided_heads_at_pair_stack_size():
    """16 heads of 24 taken as strided views of [N, 384] projections (the
    layout SingleAttention hands over), N = 1024, against torch's fp32 SDPA
    on the GPU."""
    say("[gpu] bias attn N=1024 strided")
    n, h, d = 1024, 16, 24
    g = torch.Generator().manual_seed(7)
    qx = torch.randn(n, h * d, generator=g).to(DEV) / d ** 0.5
    kx = torch.randn(n, h * d, generator=g).to(DEV)
    vx = torch.randn(n, h * d, generator=g).to(DEV)
    b = (torch.randn(h, n, n, generator=g) * 2.0).to(DEV)
    heads = lambda t: t.view(n, h, d).transpose(0, 1)  # noqa: E731
    q, k, v = heads(qx), heads(kx), heads(vx)
    exp = torch.nn.functional.scaled_dot_product_attention(q.contiguous(), k.contiguous(),
                                                           v.contiguous(), attn_mask=b, scale=1.0)
    got = K.bias_attention(q, k, v, b)
    torch.testing.assert_close(got, exp, rtol=0, atol=1e-4)


def test_bias_attention_contiguous_but_misaligned_kv():
    """k and v that are contiguous but start 4 bytes past a 16-byte boundary
    (a view one element into a buffer) are copied to aligned memory, not
    rejected."""
    say("[gpu] bias attn misaligned k/v")
    q, k, v, b = _inputs(2, 40, 72, 24, 9)
    exp = _expected(q, k, v, b)
    kbuf = torch.empty(k.numel() + 1, device=DEV)
    vbuf = torch.empty(v.numel() + 1, device=DEV)
    kd = kbuf[1:].view(k.shape)
    vd = vbuf[1:].view(v.shape)
    kd.copy_(k)
    vd.copy_(v)
    assert kd.is_contiguous() and kd.data_ptr() % 16 == 4
    got = K.bias_attention(q.to(DEV), kd, vd, b.to(DEV)).cpu()
    torch.testing.assert_close(got, exp, rtol=0, atol=1e-4)


def test_bias_attention_scale_gate_and_token_major_out():
    """The query scale applied inside the core, the output gate
    sigmoid(gate) (Attention._wrap_up, primitives.py:772-776) at the store,
    and the output written through strides into a token-major [N, H, D]
    buffer: against the oracle's float64 attention of the scaled queries,
    times the float64 sigmoid of the gate."""
    say("[gpu] bias attn scale + gate + token-major out")
    h, nq, nk, d = 3, 70, 130, 24
    q, k, v, b = _inputs(h, nq, nk, d, 21)
    q = q * d ** 0.5  # unscaled queries; the kernel applies 1 / sqrt(d)
    gate = torch.randn(h, nq, d, generator=torch.Generator().manual_seed(22)) * 2.0
    exp = (_expected(q / d ** 0.5, k, v, b).double() * torch.sigmoid(gate.double())).float()
    buf = torch.full((nq, h, d), float("nan"), device=DEV)
    K.bias_attention(q.to(DEV), k.to(DEV), v.to(DEV), b.to(DEV), scale=1.0 / d ** 0.5,
                     gate=gate.to(DEV), out=buf.transpose(0, 1))
    torch.testing.assert_close(buf.transpose(0, 1).cpu(), exp, rtol=0, atol=1e-4)


def test_single_attention_fused_path_matches_its_torch_path():
    """SingleAttention under bf16 autocast with hip=True (one GEMM for q, k,
    v and g, scale and gate inside the core, token-major output) against
    the same module's torch path (hip=False: separate bf16 projections,
    fp32 SDPA, gating in bf16). The two round differently in bf16, so the
    tolerance is bf16's on O(1) outputs; one core launch."""
    from opendde_amd.pairformer import SingleAttention
    say("[gpu] single attention fused path")
    n, c, heads = 300, 384, 16
    g = torch.Generator().manual_seed(31)
    m = SingleAttention(c, c, c, c // heads, heads, gating=True, q_linear_bias=True)
    with torch.no_grad():
        for p in m.parameters():
            p.copy_(torch.randn(p.shape, generator=g) * (0.05 if p.dim() > 1 else 0.5))
    m = m.to(DEV)
    x = torch.randn(n, c, generator=g).to(DEV)
    bias = (torch.randn(heads, n, n, generator=g) * 2.0).to(DEV)
    with torch.no_grad(), torch.autocast("cuda", dtype=torch.bfloat16):
        before = _lib.launch_count(_lib.K_BIAS_ATTN)
        got = m(x, x, bias, hip=True)
        assert _lib.launch_count(_lib.K_BIAS_ATTN) == before + 1
        exp = m(x, x, bias, hip=False)
    assert got.dtype == exp.dtype == torch.bfloat16
    torch.testing.assert_close(got.float(), exp.float(), rtol=2e-2, atol=2e-2)
