"""Module lookup used when installing BC4 linears (``texelator/adapters.py:90-96``)."""
from __future__ import annotations

from torch import nn


def resolve_parent(model: nn.Module, module_name: str) -> tuple[nn.Module, str]:
    if "." not in module_name:
        if not hasattr(model, module_name):
            raise RuntimeError(f"model module does not exist: {module_name}")
        return model, module_name
    parent_name, child = module_name.rsplit(".", 1)
    return model.get_submodule(parent_name), child
