"""MI355X-native LuminaV optimizer step (drop-in for `luminamoon.LuminaV` on ROCm tensors)."""
from __future__ import annotations

from .optimizer import LuminaV
from .optimizer.version import PACKAGE_VERSION as __version__

__all__ = ["LuminaV", "__version__"]
