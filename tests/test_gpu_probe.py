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


def test_stream_probe_modes():
    """Mode 1 copies exactly, mode 2 leaves its buffer's bits unchanged, mode
    0 reads without writing; each is one timed launch (ragged sizes cover the
    bounds of the grid-stride loop)."""
    lib = _lib.load()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for n in (4, 1000, (1 << 20) + 12):
        say(f"[gpu] stream probe n={n}")
        src = torch.randn(n, device="cuda")
        dst = torch.zeros(max(n, 256), device="cuda")
        ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
        for mode in (0, 1, 2):
            before = dst.clone()
            tot, cnt = _timed(lambda: _lib.check(lib.odde_probe_stream(
                mode, ptr(src), ptr(dst), n * 4, stream), "odde_probe_stream"))
            assert cnt == 1 and tot > 0
            if mode == 0:
                assert torch.equal(dst, before)
            elif mode == 1:
                assert torch.equal(dst[:n], src) and torch.equal(dst[n:], before[n:])
            else:
                assert torch.equal(dst, before)


def test_stream_probe_rejects_bad_arguments():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    assert lib.odde_probe_stream(3, p, p, 64, None) == -1
    assert lib.odde_probe_stream(1, p, p, 63, None) == -1
    assert lib.odde_probe_stream(1, None, p, 64, None) == -1
    assert lib.odde_probe_stream(0, p, p, 0, None) == -1
    assert lib.odde_probe_stream(1, ctypes.c_void_p(0x1004), p, 64, None) == -1

