"""MI355X-native Laya inference: the laya-cuda API over a HIP (gfx950) runtime.

Import is light: the native library loads when the first Runtime is built.
"""
from .engine import Engine
from .batching import BatchEngine

__all__ = ["Engine", "BatchEngine"]
__version__ = "0.1.0+mi355x"
