"""Kernel-selection hook and drop-in module behaviour on the CPU.

Mirrors the reference's behavioural tests for this path:
tests/test_runtime_fallbacks.py:53-103 (accelerated requests on CPU tensors
fall back to torch; invalid names raise) and
tests/test_inference_config.py:141-265 (``auto`` resolution, explicit
accelerated requests that cannot run raise with the runtime's reason,
explicit torch skips the library probe).  Also pins the checkpoint contract
(parameter names) and the torch path of the drop-in modules against the
oracle.
"""

from types import SimpleNamespace

import pytest
import torch

from helpers import params_of, seeded, token_pair_mask
from oracle import reference as ref
from opendde_amd import hook
from opendde_amd import kernels as K
from opendde_amd import triangular
from opendde_amd.pairformer import PairformerBlock, PairformerStack, Transition

ACCEL = ["hip", "cuequivariance"]


# ------------------------------------------------------ CPU fallback policy


@pytest.mark.parametrize("kernel", ACCEL)
def test_cpu_triangle_attention_accelerated_falls_back_to_torch(monkeypatch, kernel):
    monkeypatch.setattr(triangular, "hip_triangular_attn",
                        lambda *a, **k: pytest.fail("CPU tensor reached the HIP slot"))
    attention = triangular.Attention(c_q=4, c_k=4, c_v=4, c_hidden=4, no_heads=1)
    q_x = torch.randn(2, 17, 4)
    biases = [torch.zeros(2, 1, 17, 17), torch.zeros(2, 1, 17, 17)]
    expected = attention(q_x, q_x, biases=biases, triangle_attention="torch")
    output = attention(q_x, q_x, biases=biases, triangle_attention=kernel)
    torch.testing.assert_close(output, expected)


@pytest.mark.parametrize("kernel", ACCEL)
@pytest.mark.parametrize("c_hidden", [2, 4])
def test_cpu_triangle_multiplication_accelerated_falls_back_to_torch(monkeypatch, kernel,
                                                                     c_hidden):
    monkeypatch.setattr(K, "triangle_multiplication",
                        lambda *a, **k: pytest.fail("CPU tensor reached the HIP kernel"))
    layer = triangular.TriangleMultiplicationOutgoing(c_z=4, c_hidden=c_hidden)
    z = torch.randn(3, 3, 4)
    expected = layer(z, triangle_multiplicative="torch")
    output = layer(z, triangle_multiplicative=kernel)
    torch.testing.assert_close(output, expected)


@pytest.mark.parametrize("kernel", ACCEL)
def test_cpu_triangle_attention_module_falls_back_to_torch(monkeypatch, kernel):
    monkeypatch.setattr(K, "triangle_attention",
                        lambda *a, **k: pytest.fail("CPU tensor reached the HIP kernel"))
    mod = seeded(triangular.TriangleAttention(16, 8, 2), 1, 0.1)
    z = torch.randn(20, 20, 16)
    mask = token_pair_mask(20, 3)
    expected = mod(z, mask, triangle_attention="torch")
    torch.testing.assert_close(mod(z, mask, triangle_attention=kernel), expected)


@pytest.mark.parametrize("kernel", ACCEL)
def test_cpu_pairformer_block_accelerated_equals_torch(kernel):
    blk = seeded(PairformerBlock(n_heads=4, c_z=32, c_s=32, c_hidden_mul=32,
                                 c_hidden_pair_att=8, no_heads_pair=2), 3, 0.1)
    g = torch.Generator().manual_seed(4)
    z = torch.randn(10, 10, 32, generator=g)
    s = torch.randn(10, 32, generator=g)
    mask = token_pair_mask(10, 2)
    with torch.no_grad():
        se, ze = blk(s, z.clone(), mask)
        sg, zg = blk(s, z.clone(), mask, triangle_multiplicative=kernel,
                     triangle_attention=kernel)
    torch.testing.assert_close(zg, ze)
    torch.testing.assert_close(sg, se)


def test_cpu_triangle_multiplication_rejects_invalid_backend():
    layer = triangular.TriangleMultiplicationOutgoing(c_z=4, c_hidden=2)
    with pytest.raises(ValueError, match="triangle_multiplicative"):
        layer(torch.randn(3, 3, 4), triangle_multiplicative="invalid")


def test_cpu_triangle_attention_rejects_invalid_backend():
    attention = triangular.Attention(c_q=4, c_k=4, c_v=4, c_hidden=4, no_heads=1)
    q_x = torch.randn(2, 17, 4)
    with pytest.raises(ValueError, match="Invalid triangle_attention"):
        attention(q_x, q_x, biases=[], triangle_attention="invalid")


def test_hip_kernels_refuse_cpu_tensors():
    # the product entry points never compute on the CPU
    z = torch.randn(8, 8, 64)
    w = torch.randn(64, 64)
    with pytest.raises((RuntimeError, ValueError)):
        K.triangle_multiplication(
            z, None, outgoing=True, norm_in_weight=torch.ones(64), norm_in_bias=torch.zeros(64),
            p_in_weight=torch.randn(128, 64), g_in_weight=torch.randn(128, 64),
            norm_out_weight=torch.ones(64), norm_out_bias=torch.zeros(64), p_out_weight=w,
            g_out_weight=w)


# ------------------------------------------------------- config-level hook


def _cfg(mul, att):
    return SimpleNamespace(triangle_multiplicative=mul, triangle_attention=att)


def test_validate_triangle_kernels_rejects_unknown_values():
    hook.validate_triangle_kernels("auto", "cuequivariance")
    hook.validate_triangle_kernels("torch", "hip")
    with pytest.raises(ValueError):
        hook.validate_triangle_kernels("unsupported", "torch")
    with pytest.raises(ValueError):
        hook.validate_triangle_kernels("torch", "unsupported")


def test_auto_resolves_to_torch_on_cpu():
    cfg = hook.apply_runtime_compatibility(_cfg("auto", "auto"), torch.device("cpu"))
    assert (cfg.triangle_multiplicative, cfg.triangle_attention) == ("torch", "torch")


def test_auto_resolves_to_hip_when_runtime_usable(monkeypatch):
    monkeypatch.setattr(hook, "get_hip_runtime_status",
                        lambda device, probe_library: hook.HipRuntimeStatus())
    cfg = hook.apply_runtime_compatibility(_cfg("auto", "torch"), torch.device("cpu"))
    assert (cfg.triangle_multiplicative, cfg.triangle_attention) == ("hip", "torch")


@pytest.mark.parametrize("kernel", ACCEL)
def test_explicit_accelerated_reports_runtime_reason(monkeypatch, kernel):
    monkeypatch.setattr(hook, "get_hip_runtime_status",
                        lambda device, probe_library: hook.HipRuntimeStatus("no gfx950 here"))
    with pytest.raises(RuntimeError, match="no gfx950 here"):
        hook.apply_runtime_compatibility(_cfg(kernel, "torch"), torch.device("cpu"))


def test_explicit_accelerated_on_cpu_device_raises():
    with pytest.raises(RuntimeError, match="GPU"):
        hook.apply_runtime_compatibility(_cfg("hip", "hip"), torch.device("cpu"))


def test_explicit_torch_kernels_skip_library_probe(monkeypatch):
    seen = []

    def status(device, probe_library):
        seen.append(probe_library)
        return hook.HipRuntimeStatus("unused")

    monkeypatch.setattr(hook, "get_hip_runtime_status", status)
    hook.apply_runtime_compatibility(_cfg("torch", "torch"), torch.device("cpu"))
    assert seen == [False]


def test_apply_runtime_compatibility_needs_resolved_device():
    with pytest.raises(TypeError):
        hook.apply_runtime_compatibility(_cfg("auto", "auto"), "cuda:0")


# -------------------------------------------------- checkpoint contract


def test_parameter_names_are_the_reference_checkpoint_names():
    names = set(PairformerBlock().state_dict())
    expected = set()
    for mod in ("tri_att_start", "tri_att_end"):
        expected |= {f"{mod}.layer_norm.weight", f"{mod}.layer_norm.bias", f"{mod}.linear.weight"}
        expected |= {f"{mod}.mha.linear_{x}.weight" for x in "qkvog"}
    for mod in ("tri_mul_out", "tri_mul_in"):
        expected |= {f"{mod}.layer_norm_{x}.{p}" for x in ("in", "out") for p in ("weight", "bias")}
        expected |= {f"{mod}.linear_{x}.weight" for x in ("a_p", "a_g", "b_p", "b_g", "z", "g")}
    for mod in ("pair_transition", "single_transition"):
        expected |= {f"{mod}.layernorm1.weight", f"{mod}.layernorm1.bias"}
        expected |= {f"{mod}.linear_no_bias{x}.weight" for x in ("", "_a", "_b")}
    apb = "attention_pair_bias"
    expected |= {f"{apb}.layernorm_a.weight", f"{apb}.layernorm_a.bias",
                 f"{apb}.layernorm_z.weight", f"{apb}.layernorm_z.bias",
                 f"{apb}.linear_nobias_z.weight", f"{apb}.attention.linear_q.bias"}
    expected |= {f"{apb}.attention.linear_{x}.weight" for x in "qkvog"}
    assert names == expected
    stack = PairformerStack(n_blocks=2)
    assert set(stack.state_dict()) == {f"blocks.{i}.{k}" for i in range(2) for k in expected}


# ------------------------------------------ torch path of the product modules


def test_module_torch_paths_match_oracle():
    torch.manual_seed(0)
    n = 12
    z = torch.randn(n, n, 32)
    mask = token_pair_mask(n, 2)
    ta = seeded(triangular.TriangleAttention(32, 8, 2, starting=False), 5, 0.1)
    torch.testing.assert_close(
        ta(z, mask), ref.triangle_attention(z, mask, params_of(ta), 2, starting=False),
        atol=1e-5, rtol=1e-5)
    tm = seeded(triangular.TriangleMultiplicationIncoming(32, 16), 6, 0.1)
    torch.testing.assert_close(
        tm(z, mask), ref.triangle_multiplication(z, mask, params_of(tm), False),
        atol=1e-5, rtol=1e-5)
    tr = seeded(Transition(32, 4), 7, 0.1)
    torch.testing.assert_close(tr(z), ref.transition(z, params_of(tr)), atol=1e-5, rtol=1e-5)


def test_outer_product_mean_module_torch_path_matches_oracle():
    """The module's torch path (the reference's math, used on CPU tensors)
    equals the oracle, with and without a mask and with row chunking."""
    from opendde_amd.outer_product_mean import OuterProductMean
    mod = seeded(OuterProductMean(16, 24, 32), 5, 0.1).double()
    g = torch.Generator().manual_seed(6)
    m = torch.randn(7, 9, 16, generator=g, dtype=torch.float64)
    mask = (torch.rand(7, 9, generator=g) > 0.3).double()
    p = {k: v for k, v in mod.named_parameters()}
    for mk in (mask, None):
        exp = ref.outer_product_mean(m, mk, p)
        torch.testing.assert_close(mod(m, mk), exp, rtol=1e-12, atol=1e-12)
        torch.testing.assert_close(mod(m, mk, chunk_size=4), exp, rtol=1e-12, atol=1e-12)
    with pytest.raises(ValueError):
        mod(m, mask, kernel="triton")
