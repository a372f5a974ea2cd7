"""Plugin loader: import a plugin package, then hold it to the contract before anyone uses it.

Reference: tempo/plugins/registry.py:41-88.  The refusals are the contract's (every one is a
ContractError, never an AttributeError or ImportError reaching the caller): the package is
missing, it declares no load(), the object load() returns declares no contract or a contract of
another major, its rate table cannot be listed, holds something that is not a Rate, or holds a
MEASURED rate without a clean card state (Rate.check).

Here the gate is a list of checks run in order over the loaded object, each either passing or
raising with the reason; a plugin that passes all of them is cached by directory name.
"""
from __future__ import annotations

import importlib
import pkgutil
from typing import Callable, Dict, List

from . import base
from .base import ContractError

_LOADED: Dict[str, object] = {}


def available() -> list:
    """Directory names under tempo.plugins that are packages (every candidate plugin)."""
    import tempo.plugins as pkg

    return sorted(m.name for m in pkgutil.iter_modules(pkg.__path__) if m.ispkg)


def _contract_major(contract: str) -> str:
    """"tempo/arch/1" -> "tempo/arch": a plugin binds to the major, any minor is accepted."""
    head, sep, _minor = contract.rpartition("/")
    return head if sep else contract


# ---- the gate: (what is checked, check(plugin, name) -> None or raises ContractError) --------
def _declares_contract(plugin, name: str) -> None:
    contract = getattr(plugin, "contract", None)
    if contract is None:
        raise ContractError("plugin %r declares no contract" % name)
    if _contract_major(contract) != base.CONTRACT_MAJOR:
        raise ContractError("plugin %r declares contract %r; this pipeline reads major %r"
                            % (name, contract, base.CONTRACT_MAJOR))


def _rates_are_valid(plugin, name: str) -> None:
    try:
        table = plugin.machine.symbols()
    except Exception as e:  # any failure to list the table is the plugin's contract breach
        raise ContractError("plugin %r: symbols() raised: %s" % (name, e)) from e
    for symbol, r in table.items():
        if not isinstance(r, base.Rate):
            raise ContractError("plugin %r: rate %r is not a Rate" % (name, symbol))
        r.check()  # a MEASURED rate needs a card with no foreign process


GATE: List[Callable[[object, str], None]] = [_declares_contract, _rates_are_valid]


def _import_plugin(name: str):
    try:
        module = importlib.import_module("tempo.plugins.%s" % name)
    except ImportError as e:
        raise ContractError("no plugin %r; known: %s" % (name, ", ".join(available()))) from e
    make = getattr(module, "load", None)
    if make is None:
        raise ContractError("plugin %r declares no load()" % name)
    return make()


def load(name: str):
    """The plugin in directory tempo/plugins/<name>, loaded and gated once per process."""
    if name not in _LOADED:
        plugin = _import_plugin(name)
        for check in GATE:
            check(plugin, name)
        _LOADED[name] = plugin
    return _LOADED[name]


def by_arch_id(arch_id: str):
    """The plugin whose declared id is arch_id (directory names and ids need not agree);
    plugins that fail the gate are skipped."""
    for name in available():
        try:
            plugin = load(name)
        except ContractError:
            continue
        if getattr(plugin, "id", None) == arch_id:
            return plugin
    raise ContractError("no plugin declares arch id %r" % arch_id)
