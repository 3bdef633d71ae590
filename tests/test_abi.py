"""C-ABI boundary checks that need no GPU: the library loads, exports every
symbol include/opendde_amd.h declares, its struct layouts match the ctypes
mirrors (sizes and field offsets as gcc computes them from the header), and
invalid arguments come back as status codes with a message (no device call
is reached on those paths)."""

import ctypes
import os
import re
import subprocess
import tempfile

import pytest

from opendde_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "opendde_amd.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(odde_[a-z_0-9]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    declared = _declared_functions()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"missing export {name}"
    assert set(declared) == set(_lib.SYMBOLS), "ctypes binding and header disagree"
    assert lib.odde_abi_version() == _lib.ABI_VERSION


@pytest.mark.parametrize("cname,pyty", [("odde_triatt_args", _lib.TriattArgs),
                                        ("odde_triatt_core_args", _lib.TriattCoreArgs),
                                        ("odde_trimul_args", _lib.TrimulArgs),
                                        ("odde_transition_args", _lib.TransitionArgs),
                                        ("odde_layer_norm_args", _lib.LayerNormArgs),
                                        ("odde_layer_norm_bwd_args", _lib.LayerNormBwdArgs),
                                        ("odde_opm_args", _lib.OpmArgs),
                                        ("odde_bias_attn_args", _lib.BiasAttnArgs)])
def test_struct_layout_matches_header(cname, pyty):
    fields = [f for f, _ in pyty._fields_]
    src = ["#include <stdio.h>", "#include <stddef.h>", f'#include "{HEADER}"', "int main(void){",
           f'printf("%zu\\n", sizeof({cname}));']
    src += [f'printf("%zu\\n", offsetof({cname}, {f}));' for f in fields]
    src += ["return 0;}"]
    with tempfile.TemporaryDirectory() as d:
        c = os.path.join(d, "t.c")
        exe = os.path.join(d, "t")
        open(c, "w").write("\n".join(src))
        subprocess.run(["gcc", "-std=c99", c, "-o", exe], check=True)
        vals = [int(x) for x in subprocess.run([exe], capture_output=True, text=True,
                                               check=True).stdout.split()]
    assert vals[0] == ctypes.sizeof(pyty)
    for f, off in zip(fields, vals[1:]):
        assert getattr(pyty, f).offset == off, f


def _status(fn, args):
    lib = _lib.load()
    rc = getattr(lib, fn)(ctypes.byref(args), ctypes.c_void_p(0))
    return rc, lib.odde_last_error().decode()


def test_bad_arguments_return_status_and_message():
    a = _lib.TriattArgs()
    a.struct_size = ctypes.sizeof(a) - 4
    rc, msg = _status("odde_triatt_fwd", a)
    assert rc == -1 and "struct_size" in msg
    a.struct_size = ctypes.sizeof(a)
    a.n, a.c, a.heads, a.head_dim = 64, 128, 4, 16
    rc, msg = _status("odde_triatt_fwd", a)
    assert rc == -2 and "head_dim" in msg
    a.head_dim = 32
    a.z_dtype = a.compute_dtype = 0
    rc, msg = _status("odde_triatt_fwd", a)
    assert rc == -1 and "null" in msg
    a.batch = -1
    rc, msg = _status("odde_triatt_fwd", a)
    assert rc == -1 and "batch" in msg
    a.batch = 0
    t = _lib.TrimulArgs()
    t.struct_size = ctypes.sizeof(t)
    t.n, t.c, t.c_hidden = 32, 100, 128
    rc, msg = _status("odde_trimul_fwd", t)
    assert rc == -2 and "c_hidden" in msg
    tr = _lib.TransitionArgs()
    tr.struct_size = ctypes.sizeof(tr)
    tr.c, tr.n_factor, tr.rows = 128, 4, 10
    tr.x_dtype, tr.compute_dtype = 0, 1
    for f in ("x", "out", "ln_w", "ln_b", "w_a", "w_b", "w_o"):
        setattr(tr, f, ctypes.c_void_p(0x1000))
    tr.x_dtype, tr.compute_dtype = 1, 0  # bf16 rows with fp32 arithmetic
    rc, msg = _status("odde_transition_fwd", tr)
    assert rc == -2 and "float32 rows" in msg
    tr.x_dtype, tr.compute_dtype = 0, 1
    tr.c = 96
    rc, msg = _status("odde_transition_fwd", tr)
    assert rc == -2 and "c in" in msg
    tr.c = 128
    tr.pb_heads = 8
    rc, msg = _status("odde_transition_fwd", tr)
    assert rc == -2 and "16 heads" in msg
    tr.pb_heads = 16
    rc, msg = _status("odde_transition_fwd", tr)
    assert rc == -1 and "pair-bias" in msg
    # c = 384 runs as LN pass + two GEMMs with the hidden rows in a workspace
    tr.c, tr.pb_heads = 384, 0
    nb = ctypes.c_uint64(0)
    assert _lib.load().odde_transition_workspace_bytes(ctypes.byref(tr), ctypes.byref(nb)) == 0
    assert nb.value >= 2048 * 5 * 384 * 2
    rc, msg = _status("odde_transition_fwd", tr)
    assert rc == -3 and "workspace" in msg
    tr.c = 128
    assert _lib.load().odde_transition_workspace_bytes(ctypes.byref(tr), ctypes.byref(nb)) == 0
    assert nb.value == 0


def test_workspace_query_and_too_small_workspace():
    lib = _lib.load()
    t = _lib.TrimulArgs()
    t.struct_size = ctypes.sizeof(t)
    t.n, t.c, t.c_hidden = 100, 128, 128
    t.z_dtype, t.compute_dtype = 0, 1
    nb = ctypes.c_uint64(0)
    assert lib.odde_trimul_workspace_bytes(ctypes.byref(t), ctypes.byref(nb)) == 0
    np_ = 128
    assert nb.value >= 3 * 128 * np_ * np_ * 2
    # non-null pointers but no workspace -> EWORKSPACE before any launch
    fake = ctypes.c_void_p(0x1000)
    for f in ("z", "out", "norm_in_weight", "norm_in_bias", "norm_out_weight", "norm_out_bias",
              "p_in_weight", "g_in_weight", "p_out_weight", "g_out_weight"):
        setattr(t, f, fake)
    rc = lib.odde_trimul_fwd(ctypes.byref(t), ctypes.c_void_p(0))
    assert rc == -3 and "workspace" in lib.odde_last_error().decode()


def test_loader_caches_failure(monkeypatch):
    _lib.reset_loader_for_tests()
    monkeypatch.setattr(_lib, "LIB_PATH", "/nonexistent/libopendde_amd.so")
    with pytest.raises(ImportError):
        _lib.load()
    monkeypatch.setattr(_lib, "LIB_PATH", os.path.join(ROOT, "opendde_amd", "lib",
                                                        "libopendde_amd.so"))
    with pytest.raises(ImportError):  # cached failure, no second attempt
        _lib.load()
    _lib.reset_loader_for_tests()
    assert _lib.load() is not None


def _opm_args(S=100, N=70, c_m=64, c=32, c_z=128, mask=True):
    a = _lib.OpmArgs()
    a.struct_size = ctypes.sizeof(_lib.OpmArgs)
    a.n_seq, a.n_res, a.c_m, a.c_hidden, a.c_z = S, N, c_m, c, c_z
    a.m_dtype = a.out_dtype = a.compute_dtype = _lib.BF16
    a.mask = ctypes.c_void_p(256) if mask else None
    return a


def test_opm_workspace_query_and_limits():
    """a and b transposed (rows padded to 128 residues, 64 MSA rows) plus the
    transposed bf16 mask and the f32 norm matrix when a mask is given;
    unsupported sizes return -2."""
    lib = _lib.load()
    nb = ctypes.c_uint64(0)
    assert lib.odde_opm_workspace_bytes(ctypes.byref(_opm_args()), ctypes.byref(nb)) == 0
    np_, sp = 128, 128
    assert nb.value >= 2 * np_ * 32 * sp * 2 + np_ * sp * 2 + np_ * np_ * 4
    nb2 = ctypes.c_uint64(0)
    assert lib.odde_opm_workspace_bytes(ctypes.byref(_opm_args(mask=False)), ctypes.byref(nb2)) == 0
    assert nb2.value < nb.value
    for kw in (dict(c=16), dict(c_m=48), dict(c_z=96)):
        rc = lib.odde_opm_workspace_bytes(ctypes.byref(_opm_args(**kw)), ctypes.byref(nb))
        assert rc == -2, kw
        assert "outer_product_mean" in lib.odde_last_error().decode()
    rc, msg = _status("odde_opm_fwd", _opm_args())
    assert rc == -1 and "null tensor pointer" in msg


def test_noalloc_layer_norm_bwd_rejects_what_its_scratch_cannot_hold():
    # the partial column sums of n2 = 4096 over 2^20 rows need far more than
    # the 16 MiB scratch array: the call returns EUNSUPPORTED before any
    # device work (the pointers are never dereferenced)
    a = _lib.LayerNormBwdArgs()
    a.struct_size = ctypes.sizeof(a)
    a.dtype, a.n1, a.n2 = _lib.F32, 1 << 20, 4096
    for f in ("dout", "mean", "invvar", "x", "gamma", "grad_input", "grad_gamma", "grad_beta"):
        setattr(a, f, ctypes.c_void_p(0x1000))
    nb = ctypes.c_uint64(0)
    assert _lib.load().odde_layer_norm_bwd_workspace_bytes(ctypes.byref(a), ctypes.byref(nb)) == 0
    assert nb.value > 16 << 20
    rc, msg = _status("odde_layer_norm_bwd_noalloc", a)
    assert rc == -2 and "scratch" in msg
    a.struct_size = 8
    rc, msg = _status("odde_layer_norm_bwd_noalloc", a)
    assert rc == -1 and "struct_size" in msg


def test_probe_library_is_separate_and_exports_its_header():
    """The machine-rate probes live in the measurement library only: the
    product library exports none of them."""
    from opendde_amd import probe as pr
    text = open(os.path.join(ROOT, "include", "opendde_amd_probe.h")).read()
    declared = sorted(set(re.findall(r"\b(odde_probe_[a-z_0-9]+)\s*\(", text)))
    assert set(declared) == set(pr.SYMBOLS)
    plib = pr.load()
    for name in declared:
        assert hasattr(plib, name), f"missing export {name}"
    lib = _lib.load()
    for name in declared:
        assert not hasattr(lib, name), f"{name} exported by the product library"
