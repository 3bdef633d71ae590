"""ctypes binding of the measurement library ``libopendde_amd_probe.so``
(``include/opendde_amd_probe.h``): machine-rate probes that the benchmark
reports beside the kernels' figures.  Not part of the Pairformer path; the
product library ``libopendde_amd.so`` does not contain them.  Each call
launches on the given stream and returns at once; time it with events on
that stream."""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE_LIB_PATH = os.environ.get("OPENDDE_AMD_PROBE_LIB",
                                os.path.join(HERE, "lib", "libopendde_amd_probe.so"))
F32, BF16, BF16_RANDOM = 0, 1, 2

_vp = ctypes.c_void_p
_dp = ctypes.POINTER(ctypes.c_double)
SYMBOLS = {
    "odde_probe_last_error": (ctypes.c_char_p, []),
    "odde_probe_mfma": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, _vp, _dp,
                                         _vp]),
    "odde_probe_mix": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32, _vp, _dp,
                                        _vp]),
    "odde_probe_stream": (ctypes.c_int32, [ctypes.c_int32, _vp, _vp, ctypes.c_uint64, _vp]),
}

_lib: Optional[ctypes.CDLL] = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """The measurement library (loaded once); raises if it is not built."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(PROBE_LIB_PATH):
                raise ImportError(f"{PROBE_LIB_PATH} not built (python -m opendde_amd.build)")
            lib = ctypes.CDLL(PROBE_LIB_PATH)
            for name, (res, args) in SYMBOLS.items():
                fn = getattr(lib, name)
                fn.restype, fn.argtypes = res, args
            _lib = lib
        return _lib


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = load().odde_probe_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed ({rc}): {msg}")
