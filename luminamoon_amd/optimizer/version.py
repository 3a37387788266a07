"""Algorithm-specification versions and their capability gates.

Follows python/luminamoon/optimizer/version.py:20-69 (matrix) and :114-140 (validation) of the
reference. The reference's offline version cache and module loader have no counterpart here:
every supported specification is served by the same kernels, gated only by the matrix below.
"""
from __future__ import annotations

import re
from typing import Any, Dict, List

ALGORITHM_SPEC_VERSION = "1.6.0"
DEFAULT_LUMINAV_VERSION = ALGORITHM_SPEC_VERSION
PACKAGE_VERSION = "0.1.0"
SUPPORTED_VERSIONS: List[str] = ["1.6.0", "1.5.5", "1.5.4", "1.5.3"]

VERSION_CAPABILITIES: Dict[str, Dict[str, Any]] = {
    "1.6.0": {"version": "1.6.0", "allowed_buffers": (1, 2, "T1", "T2"), "supports_bucket_fusion": True,
              "supports_prewarm_jit": True, "supports_triangle_family": True,
              "description": "Triangle Family (T1 & T2 tanh-free envelope) & Pade rational bounds"},
    "1.5.5": {"version": "1.5.5", "allowed_buffers": (1, 2), "supports_bucket_fusion": True,
              "supports_prewarm_jit": True, "supports_triangle_family": False,
              "description": "Contiguous Bucket Fusion (fuse_tensors)"},
    "1.5.4": {"version": "1.5.4", "allowed_buffers": (1, 2), "supports_bucket_fusion": False,
              "supports_prewarm_jit": False, "supports_triangle_family": False,
              "description": "Bitwise-BF16 State Promotion inside FP16 container & unified denominator epsilon"},
    "1.5.3": {"version": "1.5.3", "allowed_buffers": (1, 2), "supports_bucket_fusion": False,
              "supports_prewarm_jit": False, "supports_triangle_family": False,
              "description": "Single-Buffer TD-CLM Envelope & Pade [13/6] rational tanh"},
}

_ALIASES = ("latest", "default", "reference", "canonical", "baseline")


def validate_version(version: str) -> str:
    v = str(version).strip().lower()
    if v in _ALIASES:
        return DEFAULT_LUMINAV_VERSION
    if v in ("cargo", "package"):
        return PACKAGE_VERSION
    if v.startswith("v"):
        v = v[1:]
    m = re.match(r"^(\d+)\.(\d+)(?:\.(\d+))?(?:[.-]?(post\d+|dev\d+|rc\d+))?$", v)
    if not m:
        raise ValueError(
            f"Invalid LuminaV version format: '{version}'. Expected semantic or PEP 440 version e.g. '1.6.0' or '1.0.2.post1'."
        )
    major, minor, patch, suffix = m.group(1), m.group(2), m.group(3) or "0", m.group(4) or ""
    return f"{major}.{minor}.{patch}" + (f".{suffix}" if suffix else "")


def get_capabilities(version: str) -> Dict[str, Any]:
    v = validate_version(version)
    if v not in VERSION_CAPABILITIES:
        raise ValueError(
            f"Unknown LuminaV algorithm specification '{version}'. Supported: {list(VERSION_CAPABILITIES.keys())}"
        )
    return dict(VERSION_CAPABILITIES[v])


class HybridVersionMethod:
    """Descriptor that dispatches to an instance method or a class method depending on access."""

    def __init__(self, inst_fn, cls_fn):
        self.inst_fn, self.cls_fn = inst_fn, cls_fn

    def __get__(self, obj, owner):
        if obj is None:
            return self.cls_fn.__get__(owner, owner) if hasattr(self.cls_fn, "__get__") else self.cls_fn
        return self.inst_fn.__get__(obj, owner)
