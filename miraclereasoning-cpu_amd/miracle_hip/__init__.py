"""MI355X-native per-token forward path for the Miracle model families.

Drop-in for the reference package's public surface (miracle_reasoning/__init__.py):
``MiracleModel``, ``ModelConfig``, a backend class, its error type and
``list_devices``.  The backend is ``HIPBackend`` (one MI355X, gfx950); there is
no CPU or OpenCL fallback.
"""
from .config import FAMILIES, ModelConfig
from .hip import Device, HIPBackend, HIPError, Tensor, list_devices
from .model import MiracleModel

__all__ = ["FAMILIES", "Device", "HIPBackend", "HIPError", "MiracleModel", "ModelConfig", "Tensor", "list_devices"]
