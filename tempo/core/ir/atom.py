"""Atom helpers (reference tempo/core/ir/atom.py:25-44)."""
from __future__ import annotations

from tempo.plugins.base import Atom, AtomKind, Dep  # noqa: F401

__all__ = ["Atom", "AtomKind", "Dep", "channel_load", "region_of", "summary"]


def channel_load(atoms) -> dict:
    """Total occupancy of each channel by one pass over the atoms."""
    out = {}
    for a in atoms:
        for ch, cyc in a.footprint.items():
            out[ch] = out.get(ch, 0.0) + float(cyc)
    return out


def region_of(atoms, region: str):
    return [a for a in atoms if a.region == region]


def summary(atoms) -> str:
    top = sorted(channel_load(atoms).items(), key=lambda kv: -kv[1])
    return "%d atoms; channels: %s" % (len(atoms), ", ".join("%s=%.1f" % kv for kv in top))
