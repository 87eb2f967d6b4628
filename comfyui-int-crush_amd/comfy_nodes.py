"""ComfyUI node discovery module (reference comfy_nodes.py:1-13)."""
from ._loaders import NODE_CLASS_MAPPINGS, NODE_DISPLAY_NAME_MAPPINGS

__all__ = ["NODE_CLASS_MAPPINGS", "NODE_DISPLAY_NAME_MAPPINGS"]
