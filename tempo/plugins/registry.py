"""Load a plugin by directory name; refuse an unknown contract major without trying to run it.

Reference: tempo/plugins/registry.py:41-88 (load, _validate_rates, by_arch_id).  Same names, same
refusals: ContractError for a missing module, a missing load(), a missing or foreign contract
major, a symbols() that raises, a non-Rate entry, or a MEASURED rate without a clean card.
"""
from __future__ import annotations

import importlib
import pkgutil
from typing import Dict

from . import base
from .base import ContractError

_CACHE: Dict[str, object] = {}


def available() -> list:
    """Sub-packages of tempo.plugins (each is a candidate plugin)."""
    import tempo.plugins as pkg

    return sorted(m.name for m in pkgutil.iter_modules(pkg.__path__) if m.ispkg)


def _major(contract: str) -> str:
    parts = contract.rsplit("/", 1)
    return parts[0] if len(parts) == 2 else contract


def load(arch: str):
    """arch is the plugin's directory name ("gfx950", ...)."""
    if arch in _CACHE:
        return _CACHE[arch]
    try:
        mod = importlib.import_module("tempo.plugins.%s" % arch)
    except ImportError as e:
        raise ContractError("no plugin %r; known: %s" % (arch, ", ".join(available()))) from e
    if not hasattr(mod, "load"):
        raise ContractError("plugin %r declares no load()" % arch)
    p = mod.load()
    contract = getattr(p, "contract", None)
    if contract is None:
        raise ContractError("plugin %r declares no contract" % arch)
    if _major(contract) != base.CONTRACT_MAJOR:
        raise ContractError("plugin %r declares contract %r; this pipeline reads major %r"
                            % (arch, contract, base.CONTRACT_MAJOR))
    _validate_rates(p, arch)
    _CACHE[arch] = p
    return p


def _validate_rates(p, arch: str) -> None:
    try:
        table = p.machine.symbols()
    except Exception as e:
        raise ContractError("plugin %r: symbols() raised: %s" % (arch, e)) from e
    for sym, r in table.items():
        if not isinstance(r, base.Rate):
            raise ContractError("plugin %r: rate %r is not a Rate" % (arch, sym))
        r.check()


def by_arch_id(arch_id: str):
    """Find a plugin by the arch id it declares (not by its directory name)."""
    for name in available():
        try:
            p = load(name)
        except ContractError:
            continue
        if getattr(p, "id", None) == arch_id:
            return p
    raise ContractError("no plugin declares arch id %r" % arch_id)
