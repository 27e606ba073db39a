"""Module naming and lookup for BC4 linears (``texelator/adapters.py`` of the reference).

``artifact_key`` and ``layer_index`` keep the reference's naming so that artifact files written
here and by the reference carry the same names for the same modules.
"""
from __future__ import annotations

import hashlib
import re

from torch import nn

DEFAULT_SUFFIXES = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")

_LAYER_PATTERNS = (
    re.compile(r"(?:^|\.)(?:layers|h|blocks)\.(\d+)(?:\.|$)"),
    re.compile(r"(?:^|\.)decoder\.layers\.(\d+)(?:\.|$)"),
)


def layer_index(name: str) -> int | None:
    """Decoder layer number embedded in a module name (``adapters.py:45-50``)."""
    for pattern in _LAYER_PATTERNS:
        found = pattern.search(name)
        if found:
            return int(found.group(1))
    return None


def artifact_key(name: str) -> str:
    """File stem for a module's encoded matrix: readable name plus a 10-hex-digit hash of the
    full name (``adapters.py:53-56``)."""
    readable = re.sub(r"[^A-Za-z0-9_.-]+", "_", name).replace(".", "__")
    return f"{readable}--{hashlib.sha256(name.encode()).hexdigest()[:10]}"


def resolve_parent(model: nn.Module, module_name: str) -> tuple[nn.Module, str]:
    """(parent module, attribute name) of a dotted module path (``adapters.py:90-96``)."""
    if "." not in module_name:
        if not hasattr(model, module_name):
            raise RuntimeError(f"model module does not exist: {module_name}")
        return model, module_name
    parent_name, child = module_name.rsplit(".", 1)
    return model.get_submodule(parent_name), child
