"""MI355X-native causal depthwise conv1d; import surface of the reference package
(causal_conv1d_triton/__init__.py:1-3)."""

from .causal_conv1d import causal_conv1d_fn

__all__ = ["causal_conv1d_fn"]
