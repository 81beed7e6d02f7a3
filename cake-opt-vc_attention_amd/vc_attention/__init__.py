"""vc_attention surface (Config / LayoutCache / attention) with the gfx950 hip backend,
and the backend's known-answer preflight."""
from .core import Config, LayoutCache, attention
from .hip_backend import preflight

__all__ = ["Config", "LayoutCache", "attention", "preflight"]
