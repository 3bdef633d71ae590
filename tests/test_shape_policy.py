"""Host-side pieces of the shape policy (no GPU): which calls the kernels
cover, the one-time fallback note, and how leading batch dims and masks are
flattened for the one-call batch (kernels._batch_view / kernels._mask_view).
The GPU side is in test_gpu_shape_policy.py."""

import logging

import pytest
import torch

from opendde_amd import hook
from opendde_amd import kernels as K

CPU = torch.device("cpu")


def _z(n=8, c=128, dtype=torch.float32, lead=()):
    return torch.zeros(tuple(lead) + (n, n, c), dtype=dtype)


def test_attention_coverage():
    assert K.triangle_attention_unsupported(_z(), heads=4, head_dim=32) is None
    assert K.triangle_attention_unsupported(_z(c=384), heads=12, head_dim=32) is None
    assert "per-head dim 16" in K.triangle_attention_unsupported(_z(), heads=4, head_dim=16)
    assert "c=96" in K.triangle_attention_unsupported(_z(c=96), heads=4, head_dim=32)
    assert "heads=3" in K.triangle_attention_unsupported(_z(), heads=3, head_dim=32)
    assert "float16" in K.triangle_attention_unsupported(_z(dtype=torch.float16), 4, 32)
    why = K.triangle_attention_unsupported(_z(dtype=torch.bfloat16), 4, 32,
                                           compute_dtype=torch.float32)
    assert "fp32 arithmetic" in why


def test_multiplication_and_transition_coverage():
    assert K.triangle_multiplication_unsupported(_z(), 128) is None
    assert K.triangle_multiplication_unsupported(_z(c=64), 384) is None
    assert "c_hidden=96" in K.triangle_multiplication_unsupported(_z(), 96)
    assert "c=32" in K.triangle_multiplication_unsupported(_z(c=32), 128)
    x = torch.zeros(10, 128)
    assert K.transition_unsupported(x, 128, 4) is None
    assert "n=2" in K.transition_unsupported(x, 128, 2)
    assert "c=96" in K.transition_unsupported(torch.zeros(10, 96), 96, 4)
    assert "non-contiguous" in K.transition_unsupported(torch.zeros(128, 10).t(), 128, 4)


def test_attention_core_coverage():
    assert K.attention_core_unsupported(torch.zeros(2, 4, 8, 32)) is None
    assert "per-head dim 24" in K.attention_core_unsupported(torch.zeros(2, 4, 8, 24))
    assert "float64" in K.attention_core_unsupported(torch.zeros(2, 4, 8, 32, dtype=torch.float64))


def test_fallback_note_logs_once(caplog):
    hook._fallbacks_noted.clear()
    with caplog.at_level(logging.WARNING, logger="opendde_amd.hook"):
        hook.note_fallback("TriangleAttention", "per-head dim 16")
        hook.note_fallback("TriangleAttention", "per-head dim 16")
        hook.note_fallback("TriangleAttention", "c=96")
    msgs = [r.getMessage() for r in caplog.records]
    assert len(msgs) == 2 and "torch path" in msgs[0]
    hook._fallbacks_noted.clear()


def test_batch_view_flattens_leading_dims_without_copy():
    z = _z(lead=(2, 3))
    v, b, sb = K._batch_view(z, "z")
    assert b == 6 and sb == 8 * 8 * 128 and v.data_ptr() == z.data_ptr()
    v, b, sb = K._batch_view(_z(), "z")
    assert (b, sb) == (1, 0)
    # a transposed pair view keeps its leading stride
    zt = z.transpose(-2, -3)
    v, b, sb = K._batch_view(zt, "z")
    assert b == 6 and v.stride()[1:3] == (128, 8 * 128)
    with pytest.raises(ValueError, match="collapse"):
        K._batch_view(_z(lead=(2, 3)).transpose(0, 1), "z")
    with pytest.raises(ValueError, match="square"):
        K._batch_view(torch.zeros(4, 5, 128), "z")
    assert K._batch_view(_z(n=0, lead=(2,)), "z")[1] == 0


def test_mask_view_broadcasts_over_the_batch():
    n = 8
    m = torch.ones(n, n)
    got, s0, s1, sb = K._mask_view(m, (3,), n, CPU)
    assert got.shape == (3, n, n) and (s0, s1, sb) == (n, 1, 0)
    per = torch.rand(2, 1, n, n) > 0.5
    got, s0, s1, sb = K._mask_view(per, (2, 1), n, CPU)
    assert got.dtype == torch.float32 and sb == n * n
    assert torch.equal(got[1], per[1, 0].float())
    got, _, _, sb = K._mask_view(m, (), n, CPU)
    assert got.shape == (1, n, n) and sb == 0
    with pytest.raises(ValueError, match="broadcast"):
        K._mask_view(torch.ones(4, n, n), (3,), n, CPU)
    with pytest.raises(ValueError, match="leading dims"):
        K._mask_view(torch.ones(2, 2, n, n), (2,), n, CPU)


def test_pair_layout_predicate():
    z = _z(lead=(2, 3))
    assert K.pair_layout_ok(z)
    assert K.pair_layout_ok(z[1])  # one view of a batch
    assert K.pair_layout_ok(z.transpose(-2, -3))  # the ending-node strides
    assert not K.pair_layout_ok(z.transpose(0, 1))  # leading dims that no view collapses
    assert not K.pair_layout_ok(torch.zeros(8, 8, 256)[..., ::2])  # channel stride 2
    assert not K.pair_layout_ok(torch.zeros(8, 8, 130)[..., 1:129])  # rows not 16-byte aligned
    assert K.pair_layout_ok(_z(n=0))


def test_weight_cache_entry_dies_with_its_parameter():
    import gc
    w = torch.nn.Parameter(torch.randn(64, 64))
    w2 = torch.nn.Parameter(torch.randn(8, 64))
    n0 = K.cache_size()
    a = K.prepared(w, torch.bfloat16)
    b = K.prepared_cat((w, w2), torch.bfloat16)
    assert K.cache_size() == n0 + 2 and a.dtype == torch.bfloat16 and b.shape == (72, 64)
    assert K.prepared(w, torch.bfloat16) is a  # a hit while the version holds
    K.prepared_cat((w2, torch.nn.Parameter(torch.randn(4, 64))), torch.bfloat16)
    gc.collect()
    assert K.cache_size() == n0 + 2  # its temporary source died: entry gone
    del w
    gc.collect()
    assert K.cache_size() == n0  # both remaining entries named the freed parameter


def test_linear_takes_the_cached_cast_only_without_gradients():
    from opendde_amd.layers import Linear
    lin = Linear(16, 8)
    assert lin._needs_grad()
    with torch.no_grad():
        assert not lin._needs_grad()
    lin.requires_grad_(False)
    assert not lin._needs_grad()
