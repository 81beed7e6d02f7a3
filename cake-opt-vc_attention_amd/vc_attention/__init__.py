"""vc_attention surface (Config / LayoutCache / attention) with the gfx950 hip backend."""
from .core import Config, LayoutCache, attention

__all__ = ["Config", "LayoutCache", "attention"]
