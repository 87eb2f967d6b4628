"""INT-Crush quantized-linear forward for AMD MI355X (gfx950).

Drop-in counterpart of the ComfyUI-INT-Crush plugin package
(reference __init__.py:1-32): importing the package registers the INT4/INT8
layouts with ComfyUI when ComfyUI is present, and exposes the loader nodes.
The compute path is the hand-written HIP library libintcrush_gfx950.so,
reached through _hip_runtime.
"""
from __future__ import annotations

import logging

from . import _hip_runtime  # noqa: F401  (loads the gfx950 kernels, sets flags)

_log = logging.getLogger(__name__)

NODE_CLASS_MAPPINGS: dict = {}
NODE_DISPLAY_NAME_MAPPINGS: dict = {}

try:
    from .quant_layout import register_intcrush_layouts

    register_intcrush_layouts()
    from ._loaders import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS  # noqa: F811
except ImportError as _exc:  # pragma: no cover - ops layer not importable
    _log.debug("INT-Crush: ops/loader layer unavailable: %s", _exc)

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
