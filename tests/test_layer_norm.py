"""Fast LayerNorm: module, loader and boundary behaviour on the CPU.

Ports of the reference's loader tests (tests/test_runtime_fallbacks.py:
167-289): CPU tensors use ``F.layer_norm`` without touching the loader; a
successful load is cached (one import); without a GPU the loader returns
``None`` and does not mark itself attempted; a failed load is cached and
logged once; the autograd function returns one gradient per input.  Plus the
``LAYERNORM_TYPE=fast_layernorm`` factory switch, the checkpoint names, the
eight-symbol surface and the C-ABI status paths (no device call is reached).
"""

import ctypes
import logging
import os
import subprocess
import sys
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from opendde_amd import _lib
from opendde_amd import fast_layer_norm as fln
from opendde_amd import layer_norm

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture
def reset_loader():
    layer_norm._reset_loader_for_tests()
    yield layer_norm
    layer_norm._reset_loader_for_tests()


def test_fused_layer_norm_uses_torch_for_cpu(monkeypatch):
    monkeypatch.setattr(layer_norm, "_load_fast_layer_norm_cuda_v2",
                        lambda: pytest.fail("CPU LayerNorm loaded the HIP library"))
    for scale, offset in ((True, True), (True, False), (False, True), (False, False)):
        module = layer_norm.FusedLayerNorm(4, create_scale=scale, create_offset=offset)
        x = torch.randn(2, 4)
        torch.testing.assert_close(
            module(x), F.layer_norm(x, module.normalized_shape, module.weight, module.bias,
                                    module.eps))


def test_fused_layer_norm_parameters():
    m = layer_norm.FusedLayerNorm([3, 4], eps=1e-6)
    assert m.normalized_shape == torch.Size([3, 4]) and m.eps == 1e-6
    assert torch.equal(m.weight, torch.ones(3, 4)) and torch.equal(m.bias, torch.zeros(3, 4))
    assert set(m.state_dict()) == {"weight", "bias"}
    m = layer_norm.FusedLayerNorm(8, create_scale=False)
    assert m.weight is None and set(m.state_dict()) == {"bias"}


def test_loaded_extension_is_cached(monkeypatch, reset_loader):
    imports = []
    real = layer_norm.importlib.import_module

    def counting_import(name, package=None):
        imports.append((name, package))
        return real(name, package)

    monkeypatch.setattr(layer_norm.torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(layer_norm.importlib, "import_module", counting_import)
    ext = layer_norm._load_fast_layer_norm_cuda_v2()
    assert ext is fln
    assert layer_norm._load_fast_layer_norm_cuda_v2() is ext
    assert imports == [(".fast_layer_norm", layer_norm.__package__)]


def test_loader_without_gpu_does_not_mark_attempted(monkeypatch, reset_loader):
    monkeypatch.setattr(layer_norm.torch.cuda, "is_available", lambda: False)
    assert layer_norm._load_fast_layer_norm_cuda_v2() is None
    assert not layer_norm._fast_layer_norm_load_attempted


def test_load_failure_is_cached_and_logged_once(caplog, monkeypatch, reset_loader):
    calls = []

    def broken_import(name, package=None):
        calls.append(name)
        return SimpleNamespace()  # fails symbol validation

    monkeypatch.setattr(layer_norm.torch.cuda, "is_available", lambda: True)
    monkeypatch.setattr(layer_norm.importlib, "import_module", broken_import)
    caplog.set_level(logging.WARNING, logger=layer_norm.__name__)
    assert layer_norm._load_fast_layer_norm_cuda_v2() is None
    assert layer_norm._load_fast_layer_norm_cuda_v2() is None
    assert len(calls) == 1
    assert layer_norm._fast_layer_norm_load_attempted
    assert layer_norm.fast_layer_norm_cuda_v2 is None
    assert "missing required symbols" in str(layer_norm._fast_layer_norm_load_error)
    assert sum("Fast LayerNorm HIP library is unavailable" in r.message
               for r in caplog.records) == 1


def test_backward_returns_one_gradient_per_input(monkeypatch):
    extension = SimpleNamespace(
        forward_with_both_affine=lambda x, shape, w, b, eps: (
            x.clone(), x.new_zeros(x.shape[:-1]), x.new_ones(x.shape[:-1])),
        backward_with_both_affine=lambda g, mean, invvar, x, shape, w, b, eps: (
            g, torch.zeros_like(w), torch.zeros_like(b)),
    )
    monkeypatch.setattr(layer_norm, "fast_layer_norm_cuda_v2", extension)
    x = torch.randn(2, 4, requires_grad=True)
    w = torch.ones(4, requires_grad=True)
    b = torch.zeros(4, requires_grad=True)
    out = layer_norm.FusedLayerNormAffineFunction.apply(x, w, b, torch.Size([4]), 1e-5)
    out.sum().backward()
    torch.testing.assert_close(x.grad, torch.ones_like(x))
    assert w.grad is not None and b.grad is not None


def test_dispatch_picks_the_symbol_for_the_affine_variant(monkeypatch):
    seen = []

    def fwd(name):
        def f(x, shape, *rest):
            seen.append((name, len(rest)))
            return x.clone(), x.new_zeros(x.shape[0]), x.new_ones(x.shape[0])
        return f

    ext = SimpleNamespace(**{s: fwd(s) for s in layer_norm._FAST_LAYER_NORM_REQUIRED_SYMBOLS
                             if s.startswith("forward")})
    monkeypatch.setattr(layer_norm, "fast_layer_norm_cuda_v2", ext)
    x = torch.randn(3, 4)
    w, b = torch.ones(4), torch.zeros(4)
    for wi, bi in ((None, None), (None, b), (w, None), (w, b)):
        layer_norm.FusedLayerNormAffineFunction.apply(x, wi, bi, torch.Size([4]), 1e-5)
    # (symbol, number of trailing args incl. eps)
    assert seen == [("forward_none_affine", 1), ("forward_with_bias_affine", 2),
                    ("forward_with_weight_affine", 2), ("forward_with_both_affine", 3)]


def test_extension_exposes_the_eight_symbols():
    assert layer_norm._validate_fast_layer_norm_extension(fln) is fln
    with pytest.raises(ImportError, match="missing required symbols"):
        layer_norm._validate_fast_layer_norm_extension(SimpleNamespace(forward_none_affine=len))


def test_entry_points_refuse_cpu_and_non_contiguous_inputs():
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fln.forward_none_affine(torch.randn(2, 4), (4,), 1e-5)
    with pytest.raises(RuntimeError, match="must be a CUDA tensor"):
        fln.backward_none_affine(torch.randn(2, 4), torch.zeros(2), torch.ones(2),
                                 torch.randn(2, 4), (4,), 1e-5)


def test_layernorm_type_env_selects_fused_layer_norm():
    code = ("from opendde_amd import layers; from opendde_amd.pairformer import PairformerBlock;"
            "import opendde_amd.layer_norm as L;"
            "m = layers.LayerNorm(8, create_offset=False);"
            "print(type(m).__name__, m.bias is None, m.eps);"
            "b = PairformerBlock(c_z=32, c_s=32, n_heads=4, c_hidden_mul=32,"
            " c_hidden_pair_att=8, no_heads_pair=2);"
            "print(type(b.tri_mul_out.layer_norm_in).__name__, len(b.state_dict()))")
    res = {}
    for value in ("fast_layernorm", "torch"):
        env = dict(os.environ, LAYERNORM_TYPE=value, PYTHONPATH=ROOT)
        out = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True,
                             text=True, check=True).stdout.split("\n")
        res[value] = out
    assert res["fast_layernorm"][0] == "FusedLayerNorm True 1e-05"
    assert res["fast_layernorm"][1].startswith("FusedLayerNorm ")
    assert res["torch"][0] == "OpenFoldLayerNorm True 1e-05"
    # same checkpoint keys either way
    assert res["fast_layernorm"][1].split()[1] == res["torch"][1].split()[1]


# ------------------------------------------------------------------ C ABI


def _bwd_args(n1, n2, dtype=_lib.BF16):
    a = _lib.LayerNormBwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype, a.n1, a.n2 = dtype, n1, n2
    return a


def test_abi_status_paths():
    lib = _lib.load()
    a = _lib.LayerNormArgs()
    a.struct_size = ctypes.sizeof(a) - 8
    assert lib.odde_layer_norm_fwd(ctypes.byref(a), None) == -1
    assert "struct_size" in lib.odde_last_error().decode()
    a.struct_size = ctypes.sizeof(a)
    a.n1, a.n2, a.dtype, a.eps = 4, 0, _lib.F32, 1e-5
    assert lib.odde_layer_norm_fwd(ctypes.byref(a), None) == -1
    a.n2, a.dtype = 8, 7
    assert lib.odde_layer_norm_fwd(ctypes.byref(a), None) == -1
    assert "dtype" in lib.odde_last_error().decode()
    a.dtype = _lib.F16
    assert lib.odde_layer_norm_fwd(ctypes.byref(a), None) == -1
    assert "null" in lib.odde_last_error().decode()
    a.n1 = 0  # nothing to do: returns before any device call
    assert lib.odde_layer_norm_fwd(ctypes.byref(a), None) == 0

    b = _bwd_args(1000, 128)
    fake = ctypes.c_void_p(0x1000)
    for f in ("dout", "mean", "invvar", "x", "grad_input", "grad_gamma"):
        setattr(b, f, fake)
    assert lib.odde_layer_norm_bwd(ctypes.byref(b), None) == -3
    assert "workspace" in lib.odde_last_error().decode()
    b.grad_input = None
    assert lib.odde_layer_norm_bwd(ctypes.byref(b), None) == -1


@pytest.mark.parametrize("n1,n2,dtype", [(1 << 20, 128, _lib.BF16), (1000, 384, _lib.F32),
                                         (17, 37, _lib.F16), (5, 4096, _lib.BF16)])
def test_abi_backward_workspace_query(n1, n2, dtype):
    lib = _lib.load()
    b = _bwd_args(n1, n2, dtype)
    nb = ctypes.c_uint64(0)
    assert lib.odde_layer_norm_bwd_workspace_bytes(ctypes.byref(b), ctypes.byref(nb)) == 0
    # one partial row (2 x n2 f32) per part; at least the generic split's
    # parts (>= 256 rows each, <= 4096 parts), at most max(1024, that)
    rpp = max(256, -(-n1 // 4096))
    generic = -(-n1 // rpp)
    assert nb.value % (8 * n2) == 0
    parts = nb.value // (8 * n2)
    assert generic <= parts <= max(1024, generic)
    b.n1 = 0
    assert lib.odde_layer_norm_bwd_workspace_bytes(ctypes.byref(b), ctypes.byref(nb)) == 0
    assert nb.value == 0
