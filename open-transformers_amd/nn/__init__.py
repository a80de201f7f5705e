"""Neural-network operators of the ROCm backend (mirrors ``repop.nn``)."""

from . import flash_attention, functional, layer, loss

__all__ = ["flash_attention", "functional", "layer", "loss"]
