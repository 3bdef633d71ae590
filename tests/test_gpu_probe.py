"""The machine-rate probes the bench reports (measurement library
libopendde_amd_probe.so, apart from the product library; no counterpart in
the reference): they launch on the given stream, return the flop counts their
documentation states, and reject bad arguments with a status and a message."""

import ctypes

import pytest
import torch

from helpers import say
from opendde_amd import _lib
from opendde_amd import probe as pr

pytestmark = pytest.mark.gpu


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _timed_ms(fn):
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    fn()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1)


@pytest.mark.parametrize("parts", [1, 2, 3, 4])
def test_mix_probe_runs_and_counts_attention_flops(parts):
    say(f"[gpu] mix probe parts={parts}")
    lib = pr.load()
    sink = torch.zeros(256, device="cuda")
    fl = ctypes.c_double(0.0)
    before = [_lib.launch_count(k) for k in _lib.KERNEL_NAMES]
    ms = _timed_ms(lambda: pr.check(lib.odde_probe_mix(parts, 20, 8, ctypes.c_void_p(
        sink.data_ptr()), ctypes.byref(fl), _stream()), "odde_probe_mix"))
    assert ms > 0
    assert fl.value == 524288.0 * 20 * 4 * 8
    # the product library is not involved
    assert [_lib.launch_count(k) for k in _lib.KERNEL_NAMES] == before


@pytest.mark.parametrize("code", [pr.BF16, pr.BF16_RANDOM, pr.F32])
def test_mfma_probe_counts_flops(code):
    say(f"[gpu] mfma probe dtype={code}")
    lib = pr.load()
    sink = torch.zeros(256, device="cuda")
    fl = ctypes.c_double(0.0)
    ms = _timed_ms(lambda: pr.check(lib.odde_probe_mfma(code, 50, 4, ctypes.c_void_p(
        sink.data_ptr()), ctypes.byref(fl), _stream()), "odde_probe_mfma"))
    assert ms > 0
    assert fl.value == 2.0 * 16 * 16 * (4 if code == pr.F32 else 32) * 8 * 50 * 4 * 4


def test_probes_reject_bad_arguments():
    lib = pr.load()
    fl = ctypes.c_double(0.0)
    assert lib.odde_probe_mix(5, 10, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1
    assert b"parts" in lib.odde_probe_last_error()
    assert lib.odde_probe_mix(1, 0, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1
    assert lib.odde_probe_mfma(7, 10, 1, ctypes.c_void_p(0x1000), ctypes.byref(fl), None) == -1


def test_stream_probe_modes():
    """Mode 1 copies exactly, mode 2 leaves its buffer's bits unchanged, mode
    0 reads without writing (ragged sizes cover the bounds of the grid-stride
    loop; dst holds at least the 256 floats mode 0 may write)."""
    lib = pr.load()
    ptr = lambda t: ctypes.c_void_p(t.data_ptr())  # noqa: E731
    for n in (4, 1000, (1 << 20) + 12):
        say(f"[gpu] stream probe n={n}")
        src = torch.randn(n, device="cuda")
        dst = torch.zeros(max(n, 256), device="cuda")
        for mode in (0, 1, 2):
            before = dst.clone()
            ms = _timed_ms(lambda: pr.check(lib.odde_probe_stream(
                mode, ptr(src), ptr(dst), n * 4, _stream()), "odde_probe_stream"))
            assert ms > 0
            if mode == 0:
                assert torch.equal(dst, before)
            elif mode == 1:
                assert torch.equal(dst[:n], src) and torch.equal(dst[n:], before[n:])
            else:
                assert torch.equal(dst, before)


def test_stream_probe_rejects_bad_arguments():
    lib = pr.load()
    p = ctypes.c_void_p(0x1000)
    assert lib.odde_probe_stream(3, p, p, 64, None) == -1
    assert lib.odde_probe_stream(1, p, p, 63, None) == -1
    assert lib.odde_probe_stream(1, None, p, 64, None) == -1
    assert lib.odde_probe_stream(0, p, p, 0, None) == -1
    assert lib.odde_probe_stream(1, ctypes.c_void_p(0x1004), p, 64, None) == -1
