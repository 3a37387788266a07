from __future__ import annotations

from .luminav import LuminaV

__all__ = ["LuminaV"]
