"""MI355X shared-prefix decision engine: Python side of libcujev.so.

Same public surface as the reference's python/cujev/__init__.py
(Engine, Branch, Timing, EngineError)."""
from ._lib import Branch, Engine, EngineError, Timing

__all__ = ["Engine", "Branch", "Timing", "EngineError"]
