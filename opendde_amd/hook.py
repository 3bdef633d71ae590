"""Kernel-selection hook for the triangle modules.

Mirrors the reference's hook (module kwarg ``triangle_attention`` /
``triangle_multiplicative``; config/CLI value ``auto``;
opendde/config/inference.py:23,83-170, opendde/utils/environment.py:84-97,
226-291, docs/kernels.md:23-51) with one accelerated backend: the gfx950 HIP
kernels.  ``"hip"`` names it; ``"cuequivariance"`` is accepted as an alias so
existing configs and call sites select the same accelerated slot unchanged.

Module-level policy (as in the reference): an accelerated request on a CPU
tensor runs the torch path (layers.py:455-459, triangular.py:482-486); on a
GPU tensor it runs the HIP kernels when they cover the call's shape and dtype
and the torch path otherwise, logged once per module and reason, as the
reference's slot falls back to torch for configurations its kernel lacks
(layers.py:466-468).  A missing or unloadable library is never a reason to
fall back: the call raises.  The reference's cuEq-only shape gates (J <= 16
for attention, c_hidden != c_z for multiplication) are not carried over: the
HIP kernels take those shapes.
"""

from __future__ import annotations

import logging
from dataclasses import dataclass
from typing import Optional

import torch

logger = logging.getLogger(__name__)

ACCELERATED = ("hip", "cuequivariance")
MODULE_KERNELS = ("torch",) + ACCELERATED
TRIANGLE_KERNELS = ("auto",) + MODULE_KERNELS


def is_accelerated(name: str) -> bool:
    return name in ACCELERATED


_fallbacks_noted: set = set()


def note_fallback(module: str, reason: str) -> None:
    """Log, once per (module, reason), that an accelerated request on a GPU
    tensor ran the torch path because the kernels do not cover the call."""
    key = (module, reason)
    if key not in _fallbacks_noted:
        _fallbacks_noted.add(key)
        logger.warning("%s: HIP kernels do not cover %s; running the torch path", module, reason)


def check_attention_kernel(name: str) -> None:
    if name not in MODULE_KERNELS:
        raise ValueError(
            "Invalid triangle_attention. Options: 'hip', 'cuequivariance', 'torch'.")


def check_multiplicative_kernel(name: str) -> None:
    if name not in MODULE_KERNELS:
        raise ValueError(
            "triangle_multiplicative must be 'hip', 'cuequivariance' or 'torch', "
            f"but got {name}")


def validate_triangle_kernels(triangle_multiplicative: str, triangle_attention: str) -> None:
    """Config-level name validation (reference: config/inference.py:83-95)."""
    if triangle_multiplicative not in TRIANGLE_KERNELS:
        raise ValueError(
            "Invalid triangle_multiplicative. Options: 'auto', 'hip', 'cuequivariance', 'torch'.")
    if triangle_attention not in TRIANGLE_KERNELS:
        raise ValueError(
            "Invalid triangle_attention. Options: 'auto', 'hip', 'cuequivariance', 'torch'.")


@dataclass(frozen=True)
class HipRuntimeStatus:
    """Whether the HIP backend can run on one resolved device."""

    unavailable_reason: Optional[str] = None

    @property
    def usable(self) -> bool:
        return self.unavailable_reason is None

    @property
    def auto_triangle_kernel(self) -> str:
        return "hip" if self.usable else "torch"


def get_hip_runtime_status(device: torch.device, *, probe_library: bool = True) -> HipRuntimeStatus:
    """Mirror of get_cuequivariance_runtime_status (environment.py:226-291)."""
    if device.type != "cuda":
        return HipRuntimeStatus("HIP triangle kernels require a GPU device; use torch kernels.")
    if torch.version.hip is None:
        return HipRuntimeStatus("HIP triangle kernels require a ROCm build of PyTorch.")
    try:
        arch = torch.cuda.get_device_properties(device).gcnArchName
    except Exception as exc:  # noqa: BLE001
        return HipRuntimeStatus(f"Could not query the GPU architecture: {exc}")
    if not arch.startswith("gfx950"):
        return HipRuntimeStatus(f"HIP triangle kernels are built for gfx950, found {arch}.")
    if not probe_library:
        return HipRuntimeStatus("HIP library availability was not requested.")
    from . import _lib
    try:
        _lib.load()
    except ImportError as exc:
        return HipRuntimeStatus(str(exc))
    return HipRuntimeStatus()


def resolve_auto_triangle_kernels(configs, status: HipRuntimeStatus):
    """Resolve ``auto`` once per run (reference: config/inference.py:104-124)."""
    mul, att = configs.triangle_multiplicative, configs.triangle_attention
    if "auto" not in {mul, att}:
        return configs
    k = status.auto_triangle_kernel
    if mul == "auto":
        configs.triangle_multiplicative = k
    if att == "auto":
        configs.triangle_attention = k
    logger.info("Resolved triangle kernels from auto to multiplicative=%s, attention=%s.",
                configs.triangle_multiplicative, configs.triangle_attention)
    return configs


def validate_triangle_kernel_runtime(configs, status: HipRuntimeStatus) -> None:
    """An explicit accelerated request that cannot run is an error
    (reference: config/inference.py:127-137)."""
    if not (is_accelerated(configs.triangle_multiplicative)
            or is_accelerated(configs.triangle_attention)):
        return
    if status.unavailable_reason is not None:
        raise RuntimeError(status.unavailable_reason)


def apply_runtime_compatibility(configs, device: torch.device):
    """Validate names, resolve ``auto`` and check an explicit accelerated
    request against the device (reference: config/inference.py:140-170)."""
    if not isinstance(device, torch.device):
        raise TypeError("device must be an already-resolved torch.device")
    validate_triangle_kernels(configs.triangle_multiplicative, configs.triangle_attention)
    requested = {configs.triangle_multiplicative, configs.triangle_attention}
    status = get_hip_runtime_status(device, probe_library=requested != {"torch"})
    configs = resolve_auto_triangle_kernels(configs, status)
    validate_triangle_kernel_runtime(configs, status)
    return configs
