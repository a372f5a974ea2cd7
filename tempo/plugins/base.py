"""The plugin boundary, contract "tempo/arch/1" -- restated for the gfx950 build.

Reference: tempo/plugins/base.py (the contract file of the Tempolator pipeline).  Every public
name, field, enum value and exception below keeps the reference's spelling and meaning, so a
plugin written against this module loads in the reference pipeline and vice versa; only the
prose is new.  Rules the contract carries (reference base.py:12-32):

  * the pipeline core never compares an architecture name with a literal; everything measured on
    a machine lives in that machine's plugin;
  * enum values are ASCII (they are compared in code and written into manifest.json); free text
    (`explain`, `note`, reports) may be anything;
  * a plugin declaring an unknown contract MAJOR is refused at load time.
"""
from __future__ import annotations

from dataclasses import dataclass, field
from enum import Enum
from pathlib import Path
from typing import (Any, Callable, ContextManager, Iterable, Iterator, Literal, Mapping,
                    Optional, Protocol, Sequence, runtime_checkable)

CONTRACT = "tempo/arch/1"
CONTRACT_MAJOR = "tempo/arch"

ArchId = str  # e.g. "gfx950"; the core treats it as an opaque identifier


# ---------------------------------------------------------------------------------------------
# Boundary exceptions (reference base.py:63-85).  The core catches these, never AttributeError.
# ---------------------------------------------------------------------------------------------
class PluginError(Exception):
    """Root of every error that crosses the boundary."""


class PluginCapabilityError(PluginError):
    """The plugin cannot do what was asked: a structural refusal, not a crash."""


class UnknownSymbol(PluginError):
    """A rate outside the plugin's closed Machine.symbols() table was requested.

    A default value would slip past the provenance bookkeeping, so the table refuses instead."""


class ContractError(PluginError):
    """The plugin broke the contract (unknown major, MEASURED without a card, ...)."""


class NotSupported(PluginError):
    """An optional capability is not implemented -- a legal answer, not a defect."""


# ---------------------------------------------------------------------------------------------
# 3.1  Provenance of every number (reference base.py:91-169)
# ---------------------------------------------------------------------------------------------
STATUS = ("MEASURED", "SPEC", "MODEL", "UPPER_BOUND", "NOT_MEASURED")


@dataclass(frozen=True)
class CardState:
    """State of the card when a number was measured; without it the number is not valid."""

    index: int
    clock_mhz: int
    foreign_procs: int
    date: str


@dataclass(frozen=True)
class Provenance:
    tool: str
    counter: Optional[str]
    version: str
    date: str
    who: str
    observability: Literal["clean", "code_edit", "derived"]
    card: Optional[CardState] = None


@dataclass(frozen=True)
class Rate:
    """A number with its unit, its status and where it came from."""

    symbol: str
    value: float
    units: str
    status: Literal["MEASURED", "SPEC", "MODEL", "UPPER_BOUND", "NOT_MEASURED"]
    prov: Optional[Provenance] = None
    note: str = ""

    def __post_init__(self):
        if self.status not in STATUS:
            raise ContractError("status %r is not one of %r" % (self.status, STATUS))

    @property
    def measured(self) -> bool:
        return self.status == "MEASURED"

    def check(self) -> None:
        """Loader rules: MEASURED needs a card, and a card with no foreign process on it."""
        if self.status == "MEASURED":
            if self.prov is None or self.prov.card is None:
                raise ContractError("%s: MEASURED without a card state" % self.symbol)
            if self.prov.card.foreign_procs != 0:
                raise ContractError("%s: measured with %d foreign processes on the card"
                                    % (self.symbol, self.prov.card.foreign_procs))


def spec_forbidden_in_time_bound(r: Rate) -> None:
    """A datasheet (SPEC) rate may not enter a time bound: it overstates what the part does."""
    if r.status == "SPEC":
        raise ContractError("%s: a SPEC rate in a time bound; use MEASURED or UPPER_BOUND"
                            % r.symbol)


# ---------------------------------------------------------------------------------------------
# 3.2  The atom: the only IR of the v1 pipeline (reference base.py:175-213)
# ---------------------------------------------------------------------------------------------
class AtomKind(str, Enum):
    COMPUTE = "COMPUTE"
    MEM_READ = "MEM_READ"
    MEM_WRITE = "MEM_WRITE"
    XFER_ISSUE = "XFER_ISSUE"  # split transaction: the issue ...
    XFER_WAIT = "XFER_WAIT"    # ... and its wait
    BARRIER = "BARRIER"
    BRANCH = "BRANCH"
    SPILL = "SPILL"
    OTHER = "OTHER"


@dataclass(frozen=True)
class Dep:
    src_uid: int
    type: Literal["RAW", "WAR", "WAW", "CTRL", "XFER"]
    distance: int = 0
    min_gap: float = 0.0


@dataclass(frozen=True)
class Atom:
    """A phase of work occupying channels; op_id is opaque to the core."""

    uid: int
    kind: AtomKind
    op_id: str
    footprint: Mapping[str, float]  # channel name -> units (see Channel.scope)
    latency: float = 0.0
    token: Optional[str] = None  # ties an XFER_ISSUE to its XFER_WAIT; None = implicit wait
    deps: tuple = ()
    region: str = "body"


# ---------------------------------------------------------------------------------------------
# 3.3  The eight sections
# ---------------------------------------------------------------------------------------------
# --- 1. Machine (reference base.py:222-259) --------------------------------------------------
@dataclass(frozen=True)
class Channel:
    """Something occupied over an interval; the name is opaque to the core.

    scope "sched": capacity is cycles per instruction and footprints count instructions.
    scope "sm":    capacity is units per cycle for the whole compute unit and footprints count
                   units (bytes, flops ...)."""

    name: str
    scope: Literal["sched", "sm"]
    capacity: Rate


@runtime_checkable
class Machine(Protocol):
    def arch(self) -> ArchId: ...
    def symbols(self) -> Mapping[str, Rate]: ...
    def channels(self) -> Mapping[str, Channel]: ...
    def latency(self, atom_class: str) -> Rate: ...
    def sms(self) -> Rate: ...
    def schedulers_per_sm(self) -> Rate: ...
    def warp_slots_per_sm(self) -> Rate: ...
    def threads_per_warp(self) -> Rate: ...
    def smem_per_sm(self) -> Rate: ...
    def smem_per_cta_max(self) -> Rate: ...
    def regfile_words_per_sm(self) -> Rate: ...
    def clock_mhz(self) -> Rate: ...
    def peak(self, kind: str) -> Rate: ...


# --- 2. Memory (reference base.py:263-296) ----------------------------------------------------
@dataclass(frozen=True)
class WavefrontCost:
    degree: float
    floor: float
    wavefronts: float


@dataclass(frozen=True)
class MemLevel:
    name: str
    bytes_: Rate
    bandwidth: Rate
    latency: Rate


@dataclass(frozen=True)
class Layout:
    """Layout of an array in shared memory (LDS): the input of the bank-conflict law."""

    name: str
    row_words: int
    rows: int
    elem_bytes: int
    swizzle: Optional[str] = None


@runtime_checkable
class Memory(Protocol):
    def levels(self) -> tuple: ...
    def wavefronts(self, lane_words: Sequence, width_bytes: int) -> WavefrontCost: ...
    def alignment_rule(self, width_bytes: int) -> int: ...
    def pad_family(self, layout: Layout) -> Iterable[int]: ...
    def swizzle_family(self, layout: Layout) -> Iterable[str]: ...
    def residency_policy(self) -> str: ...


# --- 3. Tensor unit (reference base.py:300-353) -----------------------------------------------
@dataclass(frozen=True)
class FragmentMap:
    """Lane -> [(row, col, register slot)] for operand A, operand B and the result C."""

    a: Callable[[int], Sequence]
    b: Callable[[int], Sequence]
    c: Callable[[int], Sequence]


@dataclass(frozen=True)
class TensorOp:
    id: str
    m: int
    n: int
    k: int
    in_dtypes: tuple
    acc_dtype: str
    frag: FragmentMap
    cost: Rate
    operand_source: Literal["registers", "smem_direct"]
    loader: Optional[str] = None
    exact_while: Optional[str] = None


@runtime_checkable
class TensorUnit(Protocol):
    def ops(self) -> tuple: ...
    def select(self, in_dtypes: tuple, acc_dtype: str) -> TensorOp: ...


def acc_regs_per_thread(warp_tile: tuple, op: TensorOp) -> int:
    """Accumulator registers per lane for a (M, N) wave tile, derived from the result map."""
    m, n = warp_tile
    return len(op.frag.c(0)) * (m // op.m) * (n // op.n)


def operand_loads_per_mma(warp_tile: tuple, op: TensorOp) -> float:
    """Operand fragment loads per matrix instruction: (MB + NB) / (MB * NB)."""
    mb = warp_tile[0] // op.m
    nb = warp_tile[1] // op.n
    if mb <= 0 or nb <= 0:
        raise ContractError("wave tile %r is smaller than the %s shape" % (warp_tile, op.id))
    return (mb + nb) / float(mb * nb)


# --- 4. Resources and occupancy (reference base.py:357-404) -----------------------------------
RESOURCE_CODES = ("FITS", "SPILL", "WALL_REG", "WALL_SMEM", "NO_BUDGET")


@dataclass(frozen=True)
class Occupancy:
    warps_per_sm: int
    ctas_per_sm: int
    regs_per_thread: int
    limiter: str


@dataclass(frozen=True)
class ResourceVerdict:
    ok: bool
    code: Literal["FITS", "SPILL", "WALL_REG", "WALL_SMEM", "NO_BUDGET"]
    occ: Occupancy
    explain: str  # free text for the report; the core never branches on it

    def __post_init__(self):
        if self.code not in RESOURCE_CODES:
            raise ContractError("verdict code %r is not one of %r" % (self.code, RESOURCE_CODES))


@runtime_checkable
class Resources(Protocol):
    def reg_budget(self, warps_per_sm: int) -> int: ...
    def spill_threshold(self, max_live: int) -> int: ...
    def free_spills(self) -> int: ...
    def spill_cost(self, n: int) -> Rate: ...
    def occupancy(self, regs: int, smem_bytes: int, threads: int) -> Occupancy: ...
    # regs: the optimistic edge of the register estimate (residency, time bound);
    # max_live: the pessimistic edge (the "will it spill" question).
    def verdict(self, regs: int, max_live: int, smem_bytes: int, threads: int,
                min_ctas_per_sm: int = 1, bound_threads: int = 0) -> ResourceVerdict: ...
    def wave_quantum(self, occ: Occupancy) -> int: ...
    def declared_bounds_required(self) -> bool: ...


# --- 5. Synchronisation and transactions (reference base.py:408-436) ---------------------------
@dataclass(frozen=True)
class TransactionKind:
    """How data is fed.  consumes_registers is the falsifier field of gate G8."""

    id: str
    issue_op: str
    wait_op: Optional[str]
    granularity: Literal["instruction", "group", "barrier"]
    in_flight_max: Rate
    occupies: Mapping[str, float]
    consumes_registers: bool
    consumes_smem_staging: bool
    depth_axis: Optional[str] = None


@dataclass(frozen=True)
class BarrierKind:
    id: str
    scope: Literal["warp", "cta"]
    phased: bool
    counted: bool
    cost: Rate


@runtime_checkable
class Sync(Protocol):
    def transactions(self) -> tuple: ...
    def barriers(self) -> tuple: ...
    def rendezvous_cost(self, barrier_id: str, participants: int) -> Rate: ...


# --- 6. ISA classifier (optional) (reference base.py:440-457) ---------------------------------
@dataclass(frozen=True)
class AtomClass:
    channel: str
    cycles: float
    width_bytes: int
    latency_class: str
    predicated: bool


@runtime_checkable
class Classifier(Protocol):
    def classify(self, instr_text: str) -> AtomClass: ...
    def decode(self, binary: Path, kernel_regex: str) -> Any: ...
    def control_fields(self, word: int) -> Any: ...


# --- 7. Skeletons and axes (reference base.py:461-520) ----------------------------------------
@dataclass(frozen=True)
class Hyperform:
    plugin: ArchId
    params: Mapping[str, Any]  # opaque to the core
    key: str                   # injective, stable: names the kernel and the delivery


@dataclass(frozen=True)
class Axis:
    name: str
    affects: frozenset


@dataclass(frozen=True)
class Launch:
    grid_ctas: int
    threads: int
    smem_bytes: int
    entry: str
    # residency the skeleton declares to the compiler (__launch_bounds__ minimum); it sets the
    # register budget, so it crosses the boundary instead of being inferred by the core
    min_ctas_per_sm: int = 1
    # the thread count named in __launch_bounds__ when the launched block can be smaller (a
    # wave count chosen at launch time); 0 = `threads`.  It sets the budget the same way.
    bound_threads: int = 0


@dataclass(frozen=True)
class Rendered:
    source: str
    launch: Launch
    includes: tuple = ()
    notes: str = ""
    # the plugin names the file; a text with an explicit instantiation must be a translation
    # unit, not a header
    filename: str = "kernel.cuh"


@runtime_checkable
class Skeletons(Protocol):
    def ops(self) -> tuple: ...
    def axes(self) -> tuple: ...
    def variants(self, op: "OpSpec") -> Iterator[Hyperform]: ...
    def estimate_atoms(self, op: "OpSpec", h: Hyperform) -> list: ...
    def resources_of(self, op: "OpSpec", h: Hyperform) -> tuple: ...  # regs, max_live, smem
    def launch_of(self, op: "OpSpec", h: Hyperform) -> Launch: ...
    def render(self, op: "OpSpec", h: Hyperform) -> Rendered: ...
    def entry_probe(self, h: Hyperform) -> str: ...
    def capabilities(self) -> frozenset: ...


# --- 8. Toolchain and meters (reference base.py:524-561) --------------------------------------
@dataclass(frozen=True)
class BuildResult:
    ok: bool
    binary: Optional[Path]
    regs: int
    spill_st: int
    spill_ld: int
    stack_frame: int  # separate from spills: a frame can exist with zero reported spills
    smem_static: int
    smem_dynamic: int
    ldl_stl_in_loops: Optional[int]
    log: str


@dataclass(frozen=True)
class EnvReq:
    name: str
    path: Optional[str]
    what: str


@runtime_checkable
class Toolchain(Protocol):
    def arch_flags(self) -> list: ...
    def compile(self, source: Path, out: Path, mode: str, extra: list,
                build_dir: Path) -> BuildResult: ...
    def disasm(self, binary: Path) -> str: ...
    def requirements(self) -> list: ...


@runtime_checkable
class Meters(Protocol):
    def counters(self, kind: str) -> list: ...
    def profile(self, binary: Path, kernel: str, counters: list) -> Mapping[str, float]: ...
    def clock_lock(self, card: int, mhz: int) -> ContextManager: ...


# --- the pipeline side (reference base.py:565-580) --------------------------------------------
@dataclass(frozen=True)
class OpSpec:
    """The DECLARED operation (from the TEMPO-OP block of the naive input)."""

    kind: str
    dtype_a: str
    dtype_b: str
    dtype_c: str
    dtype_acc: str
    layout_a: str
    layout_b: str
    layout_c: str
    shapes: Mapping[str, int]
    scale: Optional[str] = None
    tol_rel_l2: float = 0.0
    coverage: str = "atomic_stamp"


# --- aggregate (reference base.py:584-628) ----------------------------------------------------
@dataclass
class Report:
    """A plugin's self-test report."""

    name: str
    ok: int = 0
    total: int = 0
    lines: list = field(default_factory=list)

    def check(self, label: str, cond: bool, note: str = "") -> bool:
        self.total += 1
        if cond:
            self.ok += 1
        self.lines.append(("ok   " if cond else "FAIL ", label, note))
        return bool(cond)

    @property
    def green(self) -> bool:
        return self.total > 0 and self.ok == self.total

    def render(self) -> str:
        out = ["PLUGIN SELF-TEST %s" % self.name]
        for st, label, note in self.lines:
            out.append("  %-6s %s%s" % (st, label, ("  -- " + note) if note else ""))
        out.append("  TOTAL: %d/%d" % (self.ok, self.total))
        return "\n".join(out)


@runtime_checkable
class Plugin(Protocol):
    id: ArchId
    contract: str
    description: str
    machine: Machine
    memory: Memory
    tensor: TensorUnit
    resources: Resources
    sync: Sync
    classifier: Optional[Classifier]
    skeletons: Skeletons
    toolchain: Toolchain
    meters: Meters

    def declared_stubs(self) -> tuple: ...
    def selftest(self) -> Report: ...


# ---------------------------------------------------------------------------------------------
# Helpers for plugins (not part of the boundary; reference base.py:634-660)
# ---------------------------------------------------------------------------------------------
def rate(symbol, value, units, status, note="", prov=None) -> Rate:
    return Rate(symbol=symbol, value=float(value), units=units, status=status, note=note,
                prov=prov)


def not_measured(symbol, units, note="") -> Rate:
    return Rate(symbol=symbol, value=float("nan"), units=units, status="NOT_MEASURED", note=note)


def closed_table_get(table: Mapping[str, Rate], symbol: str) -> Rate:
    """Closed-table access: a symbol outside the table is refused, never defaulted (gate G4)."""
    try:
        return table[symbol]
    except KeyError:
        raise UnknownSymbol("rate %r is not declared; the closed table has %d symbols"
                            % (symbol, len(table))) from None
