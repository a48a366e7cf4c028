from .base import LoRABackend
from .hip_backend import HipLoRABackend
from .registry import get_lora_backend

__all__ = ["LoRABackend", "HipLoRABackend", "get_lora_backend"]
