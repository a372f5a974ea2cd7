"""python3 -m tempo.plugins.gfx950  -- run the plugin self-test."""
from . import load

rep = load().selftest()
print(rep.render())
raise SystemExit(0 if rep.green else 1)
