"""Gates on the architecture-blind core (tempo/core): it names no architecture, carries no
hardware constant in its arithmetic, imports no plugin other than the contract, and starts no
process.  Restated from the reference's gates G1 (lexical) and G5 (imports and processes),
tests/test_gates.py:62-95 and :208-240; the word list here covers both vendors' vocabulary, since
the core must stay blind to the plugin this build adds as much as to the one it started from.

Each gate is falsified on a planted source (the last tests), so a gate that cannot fail is
caught too.
"""
import ast
import io
import os
import re
import tokenize

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CORE = os.path.join(ROOT, "tempo", "core")

# Architecture and toolchain vocabulary (NVIDIA and AMD), matched as whole identifiers in CODE
# (comments and strings are explanations, and are allowed to name things).
ARCH_WORDS = re.compile(
    r"^(sm_?\d\d|volta|ampere|hopper|hmma|imma|ldmatrix|mbarrier|cp_async|cutlass|cublas|nvcc|"
    r"ptxas|ncu|cuobjdump|gfx\d+\w*|cdna\d?|mfma|agprs?|vgprs?|sgprs?|lds_dma|hipcc|hipblaslt|"
    r"rocprof\w*|rocblas|xcds?|wave64|wavefront64|amdgcn|mi\d{3}x?)$", re.IGNORECASE)
# Hardware numbers that must come from the plugin's rate table, never from core arithmetic:
# warp / wavefront widths, CU and SM counts, LDS and register-file sizes, clocks.
HW_LITERALS = {32, 64, 80, 128, 256, 304, 512, 1530, 2400, 65536, 163840, 167936}
ALLOWED_PLUGIN_IMPORT = "tempo.plugins.base"
PROCESS_CALLS = {("os", "system"), ("os", "popen"), ("os", "execv"), ("os", "execve"),
                 ("os", "execvp"), ("os", "spawnl"), ("os", "spawnv"), ("os", "fork")}


def _core_files():
    for dirpath, _, files in os.walk(CORE):
        for f in sorted(files):
            if f.endswith(".py"):
                yield os.path.join(dirpath, f)


def code_identifiers(src: str):
    """(line, name) of every NAME token: comments and string literals are not tokens of this
    kind, so explanations never trip the lexical gate."""
    for tok in tokenize.generate_tokens(io.StringIO(src).readline):
        if tok.type == tokenize.NAME:
            yield tok.start[0], tok.string


def lexical_hits(src: str, rel: str):
    hits = ["%s:%d: names %r" % (rel, ln, name)
            for ln, name in code_identifiers(src) if ARCH_WORDS.match(name)]
    for node in ast.walk(ast.parse(src)):
        if isinstance(node, (ast.BinOp, ast.Compare, ast.AugAssign)):
            for sub in ast.walk(node):
                if (isinstance(sub, ast.Constant) and type(sub.value) is int
                        and sub.value in HW_LITERALS):
                    hits.append("%s:%d: hardware literal %d in arithmetic"
                                % (rel, sub.lineno, sub.value))
    return hits


def import_process_hits(src: str, rel: str):
    hits = []
    for node in ast.walk(ast.parse(src)):
        mods = []
        if isinstance(node, ast.Import):
            mods = [a.name for a in node.names]
        elif isinstance(node, ast.ImportFrom) and node.level == 0 and node.module:
            mods = [node.module]
        for m in mods:
            top = m.split(".")[0]
            if top in ("subprocess", "multiprocessing", "ctypes"):
                hits.append("%s:%d: imports %s" % (rel, node.lineno, m))
            if m.startswith("tempo.plugins") and not (
                    m == ALLOWED_PLUGIN_IMPORT or m.startswith(ALLOWED_PLUGIN_IMPORT + ".")):
                hits.append("%s:%d: imports %s (only %s is allowed)"
                            % (rel, node.lineno, m, ALLOWED_PLUGIN_IMPORT))
        if isinstance(node, ast.Attribute) and isinstance(node.value, ast.Name):
            if (node.value.id, node.attr) in PROCESS_CALLS:
                hits.append("%s:%d: %s.%s" % (rel, node.lineno, node.value.id, node.attr))
        if isinstance(node, ast.Call) and isinstance(node.func, ast.Name) \
                and node.func.id in ("__import__", "exec", "eval"):
            hits.append("%s:%d: %s()" % (rel, node.lineno, node.func.id))
    return hits


def test_g1_core_is_lexically_blind():
    hits = []
    for path in _core_files():
        hits += lexical_hits(open(path, encoding="utf-8").read(), os.path.relpath(path, ROOT))
    assert not hits, "architecture leaks into the core:\n  " + "\n  ".join(hits)


def test_g5_core_imports_only_the_contract_and_spawns_nothing():
    hits = []
    for path in _core_files():
        hits += import_process_hits(open(path, encoding="utf-8").read(),
                                    os.path.relpath(path, ROOT))
    assert not hits, "core imports or processes:\n  " + "\n  ".join(hits)


def test_core_gates_fire_on_planted_sources():
    planted = '''
import subprocess
from tempo.plugins.gfx950 import machine
import os

def lanes(n):
    """mentions gfx950 and 64 in a docstring: allowed"""
    waves = n // 64          # hardware literal in arithmetic
    mfma = waves + 1         # architecture word as an identifier
    os.system("hipcc x")     # process
    return mfma
'''
    lex = lexical_hits(planted, "planted.py")
    imp = import_process_hits(planted, "planted.py")
    assert any("'mfma'" in h for h in lex) and any("literal 64" in h for h in lex)
    # the import line names gfx950 in code; the docstring and the comments name it in text only
    assert [h for h in lex if "gfx950" in h] == ["planted.py:3: names 'gfx950'"]
    assert not any("'hipcc'" in h for h in lex)   # inside a string literal
    assert any("subprocess" in h for h in imp)
    assert any("tempo.plugins.gfx950" in h for h in imp)
    assert any("os.system" in h for h in imp)
