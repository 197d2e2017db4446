"""sageattention for AMD Instinct MI355X (gfx950): quantized attention as a drop-in `sageattn`.

`sageattn` deliberately has no `attn_mask` parameter in its signature: callers such as ComfyUI
probe for its absence (`sageattention/__init__.py:4-11` of the reference).
"""
from .core import sageattn  # noqa: F401

__version__ = "0.1.0+mi355"
__all__ = ["sageattn"]
