"""Module naming and lookup for BC4 linears (``texelator/adapters.py`` of the reference).

``artifact_key`` and ``layer_index`` keep the reference's naming so that artifact files written
here and by the reference carry the same names for the same modules.
"""
from __future__ import annotations

import hashlib
import re
from dataclasses import asdict, dataclass
from typing import Iterable

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


@dataclass(frozen=True)
class LinearSpec:
    """One target linear of a model, with the metadata fields an artifact entry records
    (``adapters.py:28-40``): ``supported`` is False when K is not a multiple of 16."""

    module_name: str
    artifact_key: str
    layer: int
    op: str
    M: int
    K: int
    bias: bool
    supported: bool
    reason: str

    def to_dict(self) -> dict:
        return asdict(self)


def discover_linears(model: nn.Module, suffixes: Iterable[str] = DEFAULT_SUFFIXES,
                     include_regex: str | None = None) -> list[LinearSpec]:
    """Every ``nn.Linear`` inside a numbered decoder layer whose last name component is one of
    ``suffixes`` (or whose full name matches ``include_regex``), in module order
    (``adapters.py:57-88``)."""
    wanted = set(suffixes)
    extra = re.compile(include_regex) if include_regex else None
    specs = []
    for name, module in model.named_modules():
        layer = layer_index(name) if isinstance(module, nn.Linear) else None
        if layer is None:
            continue
        op = name.rsplit(".", 1)[-1]
        if op not in wanted and not (extra and extra.search(name)):
            continue
        rows, columns = (int(v) for v in module.weight.shape)
        ok = columns % 16 == 0
        specs.append(LinearSpec(module_name=name, artifact_key=artifact_key(name), layer=layer, op=op, M=rows,
                                K=columns, bias=module.bias is not None, supported=ok,
                                reason="ok" if ok else "K is not divisible by 16"))
    return specs
