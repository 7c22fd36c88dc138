"""Reading a policy from wherever a user keeps it.

``load_policy`` takes a parsed ``OptimizationPolicy`` (returned as is), a
mapping (a document already in memory), or a path to a ``.json``, ``.yaml`` or
``.yml`` file; the reference accepts the same sources
(``optimization/policy_io.py``). YAML is read with the safe loader only. The
factory modes ``"auto"`` and ``"reference"`` are not documents and are
rejected with a message that says so.
"""

from __future__ import annotations

import json
from collections.abc import Callable, Mapping
from os import PathLike
from pathlib import Path

import yaml

from .implementations import ImplementationRegistry
from .policy import OptimizationPolicy, parse_policy

PolicySource = str | PathLike[str] | Mapping[str, object]

# File suffix -> parser of the file's text.
_READERS: Mapping[str, Callable[[str], object]] = {
    ".json": json.loads,
    ".yaml": yaml.safe_load,
    ".yml": yaml.safe_load,
}


def _read_document(path: Path) -> object:
    reader = _READERS.get(path.suffix.lower())
    if reader is None:
        raise ValueError(f"policy file {path.name!r}: the suffix must be .json, .yaml, or .yml")
    return reader(path.read_text(encoding="utf-8"))


def load_policy(
    source: PolicySource | OptimizationPolicy, *, registry: ImplementationRegistry | None = None
) -> OptimizationPolicy:
    if isinstance(source, OptimizationPolicy):
        return source
    if isinstance(source, str) and source in ("auto", "reference"):
        raise ValueError(f"{source!r} is a factory mode, not a policy document")
    document = source if isinstance(source, Mapping) else _read_document(Path(source).expanduser())
    return parse_policy(document, registry=registry)
