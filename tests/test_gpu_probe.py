"""The machine-rate probes the bench reports (no counterpart in the
reference): they launch, time through the library's events, and return the
flop counts their documentation states."""

import ctypes

import pytest
import torch

from helpers import say
from opendde_amd import _lib

pytestmark = pytest.mark.gpu


def _timed(fn):
    torch.cuda.synchronize()
    _lib.timing_reset()
    _lib.timing_enable(True)
    fn()
    torch.cuda.synchronize()
    _lib.timing_enable(False)
    tot, cnt = _lib.timing_query(_lib.K_PROBE)
    _lib.timing_reset()
    return tot, cnt


@pytest.mark.parametrize("parts", [1, 2, 3])
def test_mix_probe_runs_and_counts_attention_flops(parts):
    say(f"[gpu] mix probe parts={parts}")
    lib = _lib.load()
    sink = torch.zeros(256, device="cuda")
    fl = ctypes.c_double(0.0)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    tot, cnt = _timed(lambda: _lib.check(lib.odde_probe_mix(parts, 20, 8, ctypes.c_void_p(
        sink.data_ptr()), ctypes.byref(fl), stream), "odde_probe_mix"))
    assert cnt == 1 and tot > 0
    assert fl.value == 524288.0 * 20 * 4 * 8
    assert float(sink.abs().sum()) == 0.0  # the sink is never written


def test_probes_reject_bad_arguments():
    lib = _lib.load()
    fl = ctypes.c_double(0.0)
    assert lib.odde_probe_mix(4, 10, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1
    assert lib.odde_probe_mix(1, 0, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1
    assert lib.odde_probe_mfma(7, 10, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1
