"""Shared test helpers: seeded modules, oracle parameter dicts, tolerances."""

from __future__ import annotations

import sys

import torch

from opendde_amd import workload as wl

# Tolerances of the path: fp32 kernels max-abs 1e-4 against the fp32 oracle;
# bf16 kernels relative-L2 1e-2 and max-abs 5e-2 against the fp32 oracle.
FP32_MAX_ABS = 1e-4
BF16_REL_L2 = 1e-2
BF16_MAX_ABS = 5e-2


# Measured errors of the tolerance checks, printed by conftest's terminal
# summary at the end of the session (pytest hides a passing test's output, so
# the margins would otherwise be invisible in a plain ``pytest -q`` run).
MARGINS = []


def say(msg: str) -> None:
    """Unbuffered progress line that survives pytest's capture."""
    sys.__stderr__.write(msg + "\n")
    sys.__stderr__.flush()


def margin(what: str, **vals) -> None:
    """Record a measured error (and its bar) for the session summary."""
    MARGINS.append(what + ": " + " ".join(f"{k}={v:.3e}" if isinstance(v, float) else f"{k}={v}"
                                          for k, v in vals.items()))


def seeded(module: torch.nn.Module, seed: int, std: float = wl.STD) -> torch.nn.Module:
    wl.init_module_(module, wl.generator(seed), std)
    return module.eval()


def params_of(module: torch.nn.Module, dtype=torch.float32):
    return {k: v.detach().to("cpu", dtype) for k, v in module.named_parameters()}


def rel_l2(got: torch.Tensor, exp: torch.Tensor) -> float:
    g, e = got.double().cpu(), exp.double().cpu()
    return float((g - e).norm() / e.norm().clamp_min(1e-30))


def max_abs(got: torch.Tensor, exp: torch.Tensor) -> float:
    return float((got.double().cpu() - exp.double().cpu()).abs().max())


def assert_fp32(got, exp, what=""):
    ma = max_abs(got, exp)
    say(f"    {what} fp32 max_abs={ma:.3e}")
    margin(f"{what} [fp32]", max_abs=ma, bar=FP32_MAX_ABS)
    assert torch.isfinite(got).all(), f"{what}: non-finite output"
    assert ma <= FP32_MAX_ABS, f"{what}: max-abs {ma:.3e} > {FP32_MAX_ABS}"


def assert_bf16(got, exp, what=""):
    rl, ma = rel_l2(got, exp), max_abs(got, exp)
    say(f"    {what} bf16 rel_l2={rl:.3e} max_abs={ma:.3e}")
    margin(f"{what} [bf16]", rel_l2=rl, max_abs=ma, bars=f"{BF16_REL_L2:g}/{BF16_MAX_ABS:g}")
    assert torch.isfinite(got.float()).all(), f"{what}: non-finite output"
    assert rl <= BF16_REL_L2, f"{what}: rel-L2 {rl:.3e} > {BF16_REL_L2}"
    assert ma <= BF16_MAX_ABS, f"{what}: max-abs {ma:.3e} > {BF16_MAX_ABS}"


def token_pair_mask(n: int, n_pad: int, seed: int = 0, random: bool = False) -> torch.Tensor:
    t = wl.token_mask(n, n_pad, wl.generator(seed), random)
    return wl.pair_mask(t)
