"""Backend factory by name (mirrors multi_lora/backend/registry.py:10-17).

``"hip"`` is the MI355X backend.  ``"triton"`` — the reference's name for
its GPU segment-GEMM backend — selects the same HIP backend, so configs
written for the reference keep working.  The reference's per-segment
PyTorch path (``"torch"``) is not part of this package: it serves as the
test oracle only, and asking for it here is an error rather than a silent
CPU path.
"""

from __future__ import annotations

from .base import LoRABackend
from .hip_backend import HipLoRABackend

_GPU_NAMES = ("hip", "triton")


def get_lora_backend(name: str) -> LoRABackend:
    key = name.lower().strip()
    if key in _GPU_NAMES:
        return HipLoRABackend()
    if key == "torch":
        raise ValueError(
            "the per-segment PyTorch backend is not shipped; use lora_backend='hip' "
            "(the HIP kernels have no CPU path)"
        )
    raise ValueError(f"unknown lora backend: {name}; try hip")
