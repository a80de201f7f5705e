"""Neural-network operators of the ROCm backend (mirrors ``repop.nn``)."""

from . import embedding, flash_attention, functional, layer, loss

__all__ = ["embedding", "flash_attention", "functional", "layer", "loss"]
