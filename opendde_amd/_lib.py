"""ctypes binding of ``libopendde_amd.so`` (C ABI in ``include/opendde_amd.h``).

Loading is lazy, lock-protected and cached, including a cached failure: the
first call that needs the library tries to load it once; later calls return
the cached handle or re-raise the cached error (the same policy as the
reference's optional-extension loader, opendde/model/layer_norm/layer_norm.py:
42-108).  There is no fallback here: a caller that asked for the HIP backend
on a GPU tensor gets an ``ImportError`` / ``RuntimeError`` if the library is
missing or a launch fails.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("OPENDDE_AMD_LIB", os.path.join(HERE, "lib", "libopendde_amd.so"))
ABI_VERSION = 1

F32, BF16, F16 = 0, 1, 2
# triangle modules: f32 data, the attention core's and the contraction's
# products as three bf16 parts
F32X3 = 3
K_TRIATT_PROJ, K_TRIATT_CORE, K_TRIATT_OUT = 0, 1, 2
K_TRIMUL_PROJ, K_TRIMUL_CONTRACT, K_TRIMUL_OUT = 3, 4, 5
K_TRIATT_RELAYOUT = 6
K_TRANSITION = 7
K_LAYER_NORM, K_LAYER_NORM_BWD = 8, 9
K_OPM = 10
K_BIAS_ATTN = 11
KERNEL_NAMES = {
    K_TRIATT_PROJ: "triatt_proj", K_TRIATT_CORE: "triatt_core", K_TRIATT_OUT: "triatt_out",
    K_TRIMUL_PROJ: "trimul_proj", K_TRIMUL_CONTRACT: "trimul_contract",
    K_TRIMUL_OUT: "trimul_out", K_TRIATT_RELAYOUT: "triatt_relayout",
    K_TRANSITION: "transition", K_LAYER_NORM: "layer_norm", K_LAYER_NORM_BWD: "layer_norm_bwd",
    K_OPM: "outer_product_mean", K_BIAS_ATTN: "bias_attn",
}

_i32, _i64, _u32, _u64, _f32 = ctypes.c_int32, ctypes.c_int64, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_float
_vp = ctypes.c_void_p


class TriattArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("n", _i32), ("c", _i32), ("heads", _i32), ("head_dim", _i32),
        ("z_dtype", _i32), ("compute_dtype", _i32), ("add_residual", _i32),
        ("z", _vp), ("z_s0", _i64), ("z_s1", _i64),
        ("mask", _vp), ("mask_s0", _i64), ("mask_s1", _i64),
        ("out", _vp), ("out_s0", _i64), ("out_s1", _i64),
        ("ln_w", _vp), ("ln_b", _vp),
        ("w_bias", _vp), ("w_q", _vp), ("w_k", _vp), ("w_v", _vp), ("w_g", _vp), ("w_o", _vp),
        ("inf", _f32), ("eps", _f32),
        ("workspace", _vp), ("workspace_bytes", _u64),
        ("batch", _i32), ("z_sb", _i64), ("mask_sb", _i64), ("out_sb", _i64),
    ]


class TriattCoreArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("batch", _i32), ("rows", _i32), ("heads", _i32), ("n", _i32),
        ("head_dim", _i32), ("dtype", _i32),
        ("q", _vp), ("q_sb", _i64), ("q_si", _i64), ("q_sh", _i64), ("q_sj", _i64),
        ("k", _vp), ("k_sb", _i64), ("k_si", _i64), ("k_sh", _i64), ("k_sj", _i64),
        ("v", _vp), ("v_sb", _i64), ("v_si", _i64), ("v_sh", _i64), ("v_sj", _i64),
        ("bias", _vp), ("b_sb", _i64), ("b_sh", _i64), ("b_sq", _i64), ("b_sk", _i64),
        ("mask", _vp), ("m_sb", _i64), ("m_si", _i64), ("m_sk", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_si", _i64), ("o_sh", _i64), ("o_sj", _i64),
        ("scale", _f32), ("inf_value", _f32),
        ("workspace", _vp), ("workspace_bytes", _u64),
    ]


class TrimulArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("n", _i32), ("c", _i32), ("c_hidden", _i32),
        ("z_dtype", _i32), ("compute_dtype", _i32), ("outgoing", _i32), ("add_residual", _i32),
        ("z", _vp), ("z_s0", _i64), ("z_s1", _i64),
        ("mask", _vp), ("mask_s0", _i64), ("mask_s1", _i64),
        ("out", _vp), ("out_s0", _i64), ("out_s1", _i64),
        ("norm_in_weight", _vp), ("norm_in_bias", _vp),
        ("norm_out_weight", _vp), ("norm_out_bias", _vp),
        ("p_in_weight", _vp), ("g_in_weight", _vp), ("p_out_weight", _vp), ("g_out_weight", _vp),
        ("eps", _f32),
        ("workspace", _vp), ("workspace_bytes", _u64),
        ("p_out_weight_f32", _vp),
        ("batch", _i32), ("z_sb", _i64), ("mask_sb", _i64), ("out_sb", _i64),
    ]


class TransitionArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("c", _i32), ("n_factor", _i32), ("x_dtype", _i32),
        ("compute_dtype", _i32), ("add_residual", _i32), ("rows", _i64),
        ("x", _vp), ("out", _vp), ("ln_w", _vp), ("ln_b", _vp),
        ("w_a", _vp), ("w_b", _vp), ("w_o", _vp), ("eps", _f32),
        ("pb_heads", _i32), ("pb_ln_w", _vp), ("pb_ln_b", _vp), ("pb_w", _vp), ("pb_out", _vp),
        ("pb_eps", _f32), ("workspace", _vp), ("workspace_bytes", _u64),
    ]


class LayerNormArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("dtype", _i32), ("n1", _i64), ("n2", _i32), ("eps", _f32),
        ("x", _vp), ("gamma", _vp), ("beta", _vp), ("out", _vp), ("mean", _vp), ("invvar", _vp),
    ]


class LayerNormBwdArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("dtype", _i32), ("n1", _i64), ("n2", _i32),
        ("dout", _vp), ("mean", _vp), ("invvar", _vp), ("x", _vp), ("gamma", _vp),
        ("grad_input", _vp), ("grad_gamma", _vp), ("grad_beta", _vp),
        ("workspace", _vp), ("workspace_bytes", _u64),
    ]


class OpmArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("n_seq", _i32), ("n_res", _i32), ("c_m", _i32),
        ("c_hidden", _i32), ("c_z", _i32), ("m_dtype", _i32), ("out_dtype", _i32),
        ("compute_dtype", _i32), ("add_residual", _i32),
        ("m", _vp), ("mask", _vp), ("ln_w", _vp), ("ln_b", _vp), ("w_12", _vp), ("w_out", _vp),
        ("b_out", _vp), ("ln_eps", _f32), ("eps", _f32), ("out", _vp),
        ("workspace", _vp), ("workspace_bytes", _u64),
    ]


class BiasAttnArgs(ctypes.Structure):
    _fields_ = [
        ("struct_size", _u32), ("n_q", _i32), ("n_k", _i32), ("heads", _i32),
        ("head_dim", _i32), ("dtype", _i32),
        ("q", _vp), ("q_sh", _i64), ("q_sn", _i64), ("k", _vp), ("k_sh", _i64), ("k_sn", _i64),
        ("v", _vp), ("v_sh", _i64), ("v_sn", _i64), ("bias", _vp), ("out", _vp),
        ("o_sh", _i64), ("o_sn", _i64), ("gate", _vp), ("g_sh", _i64), ("g_sn", _i64),
        ("q_scale", _f32),
    ]


# Every symbol include/opendde_amd.h declares, with its ctypes signature.
SYMBOLS = {
    "odde_abi_version": (_i32, []),
    "odde_last_error": (ctypes.c_char_p, []),
    "odde_triatt_workspace_bytes": (_i32, [ctypes.POINTER(TriattArgs), ctypes.POINTER(_u64)]),
    "odde_triatt_fwd": (_i32, [ctypes.POINTER(TriattArgs), _vp]),
    "odde_triatt_core_workspace_bytes": (_i32, [ctypes.POINTER(TriattCoreArgs), ctypes.POINTER(_u64)]),
    "odde_triatt_core_fwd": (_i32, [ctypes.POINTER(TriattCoreArgs), _vp]),
    "odde_trimul_workspace_bytes": (_i32, [ctypes.POINTER(TrimulArgs), ctypes.POINTER(_u64)]),
    "odde_trimul_fwd": (_i32, [ctypes.POINTER(TrimulArgs), _vp]),
    "odde_transition_workspace_bytes": (_i32, [ctypes.POINTER(TransitionArgs),
                                               ctypes.POINTER(_u64)]),
    "odde_transition_fwd": (_i32, [ctypes.POINTER(TransitionArgs), _vp]),
    "odde_layer_norm_fwd": (_i32, [ctypes.POINTER(LayerNormArgs), _vp]),
    "odde_layer_norm_bwd_workspace_bytes": (_i32, [ctypes.POINTER(LayerNormBwdArgs),
                                                   ctypes.POINTER(_u64)]),
    "odde_layer_norm_bwd": (_i32, [ctypes.POINTER(LayerNormBwdArgs), _vp]),
    "odde_layer_norm_bwd_noalloc": (_i32, [ctypes.POINTER(LayerNormBwdArgs), _vp]),
    "odde_opm_workspace_bytes": (_i32, [ctypes.POINTER(OpmArgs), ctypes.POINTER(_u64)]),
    "odde_opm_fwd": (_i32, [ctypes.POINTER(OpmArgs), _vp]),
    "odde_bias_attn_fwd": (_i32, [ctypes.POINTER(BiasAttnArgs), _vp]),
    "odde_launch_count": (_i64, [_i32]),
    "odde_timing_enable": (_i32, [_i32]),
    "odde_timing_reset": (_i32, []),
    "odde_timing_query": (_i32, [_i32, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(_i64)]),
}

_lib: Optional[ctypes.CDLL] = None
_load_error: Optional[BaseException] = None
_load_attempted = False
_lock = threading.Lock()


def _bind(lib: ctypes.CDLL) -> ctypes.CDLL:
    missing = [s for s in SYMBOLS if not hasattr(lib, s)]
    if missing:
        raise ImportError("libopendde_amd.so is missing symbols: " + ", ".join(missing))
    for name, (res, args) in SYMBOLS.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.odde_abi_version()
    if ver != ABI_VERSION:
        raise ImportError(f"libopendde_amd.so ABI version {ver}, expected {ABI_VERSION}")
    return lib


def load() -> ctypes.CDLL:
    """Return the bound library, loading it on first use (cached, incl. failure)."""
    global _lib, _load_error, _load_attempted
    if _load_attempted:
        if _lib is None:
            raise ImportError(f"opendde_amd HIP library unavailable: {_load_error}") from _load_error
        return _lib
    with _lock:
        if not _load_attempted:
            try:
                if not os.path.exists(LIB_PATH):
                    raise FileNotFoundError(
                        f"{LIB_PATH} not built (run `python -m opendde_amd.build`)")
                _lib = _bind(ctypes.CDLL(LIB_PATH))
            except BaseException as e:  # noqa: BLE001 - cached and re-raised
                _load_error = e
                _lib = None
            _load_attempted = True
    return load()


def available() -> bool:
    try:
        load()
        return True
    except ImportError:
        return False


def reset_loader_for_tests() -> None:
    global _lib, _load_error, _load_attempted
    with _lock:
        _lib, _load_error, _load_attempted = None, None, False


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().odde_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (status {rc}): {msg}")


def launch_count(kernel_id: int) -> int:
    return int(load().odde_launch_count(kernel_id))


def timing_enable(on: bool) -> None:
    load().odde_timing_enable(1 if on else 0)


def timing_reset() -> None:
    load().odde_timing_reset()


def timing_query(kernel_id: int):
    """(total_ms, launches) over the launches recorded since the last reset."""
    tot = ctypes.c_double(0.0)
    cnt = _i64(0)
    check(load().odde_timing_query(kernel_id, ctypes.byref(tot), ctypes.byref(cnt)), "timing_query")
    return tot.value, int(cnt.value)
