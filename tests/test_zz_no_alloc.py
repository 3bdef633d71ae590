"""The allocation-free LayerNorm backward (odde_layer_norm_bwd_noalloc)
against the workspace entry point (odde_layer_norm_bwd), both through the C
ABI: same kernels, so the results must be bit-identical.  Two calls in a row
with the second on a smaller input (the scratch array keeps the first call's
partial sums, which the second must not read), with and without the
parameter gradients, f32 and bf16.
"""

import ctypes

import pytest
import torch

from helpers import say
from opendde_amd import _lib

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else ctypes.c_void_p(0)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _inputs(n1, n2, dtype, seed):
    g = torch.Generator(device=DEV).manual_seed(seed)
    x = torch.randn(n1, n2, generator=g, device=DEV).to(dtype)
    dout = torch.randn(n1, n2, generator=g, device=DEV).to(dtype)
    gamma = (1 + 0.1 * torch.randn(n2, generator=g, device=DEV)).to(dtype)
    xf = x.float()
    mean = xf.mean(1)
    invvar = torch.rsqrt(xf.var(1, unbiased=False) + 1e-5)
    return x, dout, gamma, mean.contiguous(), invvar.contiguous()


def _run(entry, x, dout, gamma, mean, invvar, params):
    n1, n2 = x.shape
    gi = torch.empty_like(x)
    gg = torch.empty_like(gamma) if params else None
    gb = torch.empty_like(gamma) if params else None
    a = _lib.LayerNormBwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype = _lib.F32 if x.dtype == torch.float32 else _lib.BF16
    a.n1, a.n2 = n1, n2
    a.dout, a.mean, a.invvar, a.x, a.gamma = (_ptr(t) for t in (dout, mean, invvar, x, gamma))
    a.grad_input, a.grad_gamma, a.grad_beta = _ptr(gi), _ptr(gg), _ptr(gb)
    lib = _lib.load()
    ws = None
    if entry == "odde_layer_norm_bwd":
        nb = ctypes.c_uint64(0)
        _lib.check(lib.odde_layer_norm_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)),
                   "workspace query")
        ws = torch.empty(max(int(nb.value), 256), dtype=torch.uint8, device=DEV)
        a.workspace, a.workspace_bytes = _ptr(ws), ws.numel()
    _lib.check(getattr(lib, entry)(ctypes.byref(a), _stream()), entry)
    torch.cuda.synchronize()
    return gi, gg, gb


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("params", [True, False])
def test_noalloc_layer_norm_bwd_matches_workspace_entry_point(dtype, params):
    # second call smaller: (rows, n2) and its row-kernel grid both shrink;
    # n2 = 100 (not a whole number of 16-byte vectors in bf16) takes the
    # generic kernels and their column-partial rows
    for k, (n1, n2) in enumerate([(300_000, 128), (5_000, 128), (2_000, 100)]):
        say(f"[gpu] no-alloc LN backward call {k}: n1={n1} n2={n2} {dtype} params={params}")
        x, dout, gamma, mean, invvar = _inputs(n1, n2, dtype, 17 + k)
        want = _run("odde_layer_norm_bwd", x, dout, gamma, mean, invvar, params)
        before = _lib.launch_count(_lib.K_LAYER_NORM_BWD)
        got = _run("odde_layer_norm_bwd_noalloc", x, dout, gamma, mean, invvar, params)
        assert _lib.launch_count(_lib.K_LAYER_NORM_BWD) == before + 1
        for name, g_, w_ in zip(("grad_input", "grad_gamma", "grad_beta"), got, want):
            if w_ is None:
                assert g_ is None
                continue
            assert torch.equal(g_, w_), f"call {k}: {name} differs from the workspace entry point"
