"""Argument helpers shared by the LuminaV constructor and step.

Behaviour follows python/luminamoon/optimizer/validation.py (dtype check :55-70, Levenshtein
:145-162, suggestion :165-185, number check :188-193) of the reference.
"""
from __future__ import annotations

import math
from typing import Any, Optional, Tuple


def is_valid_number(val: Any) -> bool:
    return not isinstance(val, bool) and isinstance(val, (int, float)) and math.isfinite(float(val))


def levenshtein(a: str, b: str) -> int:
    a, b = a.lower(), b.lower()
    if not a:
        return len(b)
    if not b:
        return len(a)
    prev = list(range(len(b) + 1))
    for i, ca in enumerate(a, 1):
        cur = [i] + [0] * len(b)
        for j, cb in enumerate(b, 1):
            cur[j] = min(prev[j] + 1, cur[j - 1] + 1, prev[j - 1] + (ca != cb))
        prev = cur
    return prev[-1]


def suggest_closest(value: str, candidates: Tuple[str, ...], max_dist: int = 3) -> Optional[str]:
    """Closest candidate within max_dist edits; a prefix match is a fallback when nothing is close."""
    key = value.strip().lower()
    if not key:
        return None
    best, best_dist = None, max_dist + 1
    for cand in candidates:
        dist = levenshtein(key, cand)
        if dist < best_dist:
            best, best_dist = cand, dist
        elif dist > max_dist and len(key) >= 2 and best is None and (cand.startswith(key) or key.startswith(cand)):
            best = cand
    return best


def validate_supported_dtype(tensor: Any, name: str = "param") -> None:
    if not hasattr(tensor, "dtype"):
        return
    s = str(tensor.dtype).lower()
    if "float32" in s or "bfloat16" in s or "float16" in s or s in ("f4", "<f4", "=f4", "f2", "<f2", "=f2"):
        return
    raise ValueError(
        f"Unsupported dtype '{s}' for '{name}'. Supported dtypes are "
        "torch.float32 (float32), torch.bfloat16 (bfloat16), and torch.float16 (float16)."
    )
