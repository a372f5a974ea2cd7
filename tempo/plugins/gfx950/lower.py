"""gfx950: SKELETONS -- section 7 (reference pattern tempo/plugins/sm70/lower.py).

The product GENERATES a kernel from the declared operation; render() only substitutes: it wraps
the skeleton sources in a namespace and appends the one explicit instantiation named by the
hyperform, so the emitted file compiles to exactly the kernel entry_probe() names.
"""
from __future__ import annotations

import math
import os
from typing import Iterator

from ..base import (Atom, AtomKind, Hyperform, Launch, OpSpec, PluginCapabilityError, Rendered)
from . import space
from .machine import Gfx950Machine
from .resources import Gfx950Resources

HERE = os.path.dirname(os.path.abspath(__file__))
SKEL = os.path.join(HERE, "skeletons")
_M = Gfx950Machine()
_RES = Gfx950Resources()

CAPABILITIES = frozenset({
    "gemm_fp16_ntn",          # C = A . B^T, both operands k-contiguous
    "gemm_w8a16_sym_i8",      # int8 weights, fp16 scale per output channel
    "gemm_w8a16_asym_u8_g128",  # uint8 weights, fp16 scale + uint8 zero per (row, 128 k)
    "lds_dma_pipeline",       # global_load_lds_dwordx4 multi-stage copies
    "xcd_aware_raster",       # block ids remapped so each XCD owns a contiguous tile run
    "decode_lds_ring",        # per-wave LDS-DMA ring for the weight-streaming regime
    "fmha_fwd_causal_gqa",    # attention forward: skeletons/fmha_fwd, op kind 'attention'
})

# kernel symbol, template-parameter order, and argument list, per kind: the emitter's only data
_ENTRY = {
    "ilv": ("k_gemm_ilv", ("BM", "BN", "BK", "WM", "WN", "STAGES", "GROUP", "XCD", "RSP", "SPLIT"),
            "const _Float16*, const _Float16*, _Float16*, int, int, int, int, int, int, float*, int, "
            "int",
            ("common/cdna4.h", "gemm_mfma/kernel.hip", "gemm_mfma/ilv.hip")),
    "ilv8": ("k_gemm_ilv8", ("BM", "BN", "BK", "WM", "WN", "STAGES", "GROUP", "XCD", "RSP", "BFMT",
                             "SPLIT"),
             "const _Float16*, const uint8_t*, const _Float16*, const uint8_t*, _Float16*, int, int, "
             "int, int, int, int, float*, int, int",
             ("common/cdna4.h", "gemm_mfma/kernel.hip", "gemm_mfma/ilv8.hip")),
    "dma": ("k_gemm_dma", ("BM", "BN", "BK", "WM", "WN", "STAGES", "SWZ", "GROUP", "XCD", "XT",
                           "MINB", "MS"),
            "const _Float16*, const _Float16*, _Float16*, int, int, int, int, int, int",
            ("common/cdna4.h", "gemm_mfma/kernel.hip")),
    "reg": ("k_gemm", ("BM", "BN", "BK", "WM", "WN", "MS", "SWZ", "GROUP", "XCD", "BFMT"),
            "const _Float16*, const void*, const _Float16*, const uint8_t*, _Float16*, int, int, "
            "int, int, int, int, int",
            ("common/cdna4.h", "gemm_mfma/kernel.hip")),
    "line": ("k_stream_line", ("MB", "R", "D", "BFMT", "EPI", "SN", "TPB"), "StreamArgs, int",
             ("common/cdna4.h", "gemv_stream/kernel.hip")),
    "ring": ("k_stream_dma", ("MB", "R", "D", "BFMT"), "StreamArgs",
             ("common/cdna4.h", "gemv_stream/kernel.hip")),
    "stream": ("k_stream", ("MB", "R", "U", "BFMT", "ALDS", "EPI"), "StreamArgs",
               ("common/cdna4.h", "gemv_stream/kernel.hip")),
    "shared": ("k_stream_sh", ("MB", "R", "U", "BFMT", "SN", "TPB", "EPI"), "StreamArgs",
               ("common/cdna4.h", "gemv_stream/kernel.hip")),
    "phase": ("k_stream_phase", ("MB", "NS", "D", "BFMT", "EPI", "KSL"), "PhaseArgs",
              ("common/cdna4.h", "gemv_stream/kernel.hip", "gemv_stream/phase.hip")),
}
_ENTRY["fmha"] = ("fmha::k_fmha_fwd", ("D", "CAUSAL"),
                  "const _Float16*, const _Float16*, const _Float16*, _Float16*, float*, int, int, "
                  "int, int, int, float, long, long, long, long, long, long, long, long, long, long, "
                  "long, long",
                  ("common/cdna4.h", "fmha_fwd/kernel.hip"))
_BOOL = {("fmha", "CAUSAL")}  # template parameters of type bool (written true / false)
NAMESPACE = "tempo::gen"
# compiler flags a kind needs beyond the toolchain's own; render() writes them into the source as
# a "// tempo:flags ..." line, which the toolchain (and the library build) read back.  The
# interleaved kernel keeps its accumulator tuples in place only under the register-pressure-
# minimising pre-RA scheduler (the skeleton's header says why).
KIND_FLAGS = {"ilv": ("-mllvm", "-amdgpu-sched-strategy=iterative-minreg"),
              "ilv8": ("-mllvm", "-amdgpu-sched-strategy=iterative-minreg")}
# trailing template parameters with a default in the skeleton: named only when the hyperform
# sets them (EPI = 1 is the fused gate/up epilogue of the decode kernels)
_OPTIONAL = frozenset({"EPI", "SN", "TPB", "SPLIT", "KSL"})
# default of an optional parameter left out in front of one that is named
_DEFAULT = {"EPI": 0, "SN": 1, "TPB": 1024, "SPLIT": 0, "KSL": 0}


def _order(kind: str, p: dict) -> tuple:
    """Template parameters to name: every required one, and the optional (defaulted, trailing)
    ones up to the last the hyperform sets -- an earlier unset one is named with its default."""
    names = _ENTRY[kind][1]
    last = max((i for i, k in enumerate(names) if k in p or k not in _OPTIONAL), default=-1)
    return tuple(names[:last + 1])


def _targ(kind: str, name: str, value) -> str:
    """A template argument as C++ text: bool parameters as true / false, the rest as integers."""
    if (kind, name) in _BOOL or isinstance(value, bool):
        return "true" if value else "false"
    return str(int(value))


def _p(h: Hyperform) -> dict:
    return dict(h.params)


class Gfx950Skeletons:
    _LAYOUT_V1 = ("k", "k", "n")
    _ACC_V1 = "fp32"

    def ops(self):
        return ("gemm", "attention")

    def axes(self):
        return space.axes()

    def capabilities(self):
        return CAPABILITIES

    def _require_form_v1(self, op: OpSpec) -> None:
        if op.kind == "attention":
            # Q, K, V and O rows d-contiguous (any batch / sequence / head strides), fp16 in and
            # out, fp32 scores and accumulation
            if (op.dtype_a, op.dtype_b, op.dtype_c, op.dtype_acc) != ("fp16", "fp16", "fp16",
                                                                       "fp32"):
                raise PluginCapabilityError("gfx950 attention skeleton: fp16 Q/K/V/O, fp32 "
                                            "accumulation; declared %s/%s/%s/%s"
                                            % (op.dtype_a, op.dtype_b, op.dtype_c, op.dtype_acc))
            if (op.layout_a, op.layout_b, op.layout_c) != ("d", "d", "d"):
                raise PluginCapabilityError("gfx950 attention skeleton reads d-contiguous rows; "
                                            "declared layouts %s/%s/%s"
                                            % (op.layout_a, op.layout_b, op.layout_c))
            return
        got = (op.layout_a, op.layout_b, op.layout_c)
        if got != self._LAYOUT_V1:
            raise PluginCapabilityError(
                "gfx950 skeletons compute C = A . B^T with k-contiguous operands (layouts %s); "
                "declared %s.  Refused: another layout is another operation."
                % ("/".join(self._LAYOUT_V1), "/".join(got)))
        if op.dtype_acc != self._ACC_V1:
            raise PluginCapabilityError("gfx950 skeletons accumulate in fp32 (MFMA f32 result); "
                                        "declared %s" % op.dtype_acc)
        if op.dtype_c != "fp16":
            raise PluginCapabilityError("gfx950 skeletons write fp16 C; declared %s" % op.dtype_c)
        space.bfmt(op)

    def variants(self, op: OpSpec) -> Iterator[Hyperform]:
        self._require_form_v1(op)
        return space.variants(op)

    # -- resources without a build ------------------------------------------------------------
    def _split(self, op: OpSpec, p: dict):
        N, K = int(op.shapes["N"]), int(op.shapes["K"])
        kind = p["kind"]
        if kind == "shared":
            return space.shared_split(N, K, p["MB"], p["R"], p["U"], p["SN"], p["TPB"])[:2]
        if kind == "ring":
            per_wave = space.lds_bytes("ring", dict(p, S=1))
            return space.stream_split(N, K, p["R"], 64, p["BFMT"], per_wave)
        return space.stream_split(N, K, p["R"], 64 * p["U"], p["BFMT"])

    def resources_of(self, op: OpSpec, h: Hyperform):
        """(regs, max_live, lds) estimated from the skeleton's structure; the two register numbers
        are the optimistic and pessimistic edges of one estimate."""
        p = _p(h)
        kind = p["kind"]
        if kind == "fmha":
            # O accumulators (D/2), Q fragments (D/4), one block's K and V fragments (D/4 each:
            # the chain's reads run ahead), two score sets (32), two probability sets (16),
            # addresses and the softmax state (~32); pessimistic edge D/8 + 16 more
            D = p["D"]
            regs = D // 2 + 3 * (D // 4) + 32 + 16 + 32
            return regs, regs + D // 8 + 16, space.fmha_lds(D)
        if kind == "stream" and p.get("EPI"):
            p = dict(p, R=2 * p["R"])  # each wave carries the gate and the up row groups
        if kind == "phase":
            # one accumulator per slab and block for the whole chunk (4 NS MBE), one phase's
            # activation fragments (16 MBE), a step's weight bytes and their fp16 expansion (16),
            # fmt 2 zero-points and scales and their LDS addresses per slab (2 NS + 8), copy
            # sources and loop state (48), the gate/up epilogue's up-row copy sources and half
            # selects (8), the k-slice's partial-row addresses and slice offsets (16);
            # pessimistic edge x1.25 (measured: 120-256 registers)
            mbe = max(1, p["MB"])
            regs = (4 * p["NS"] * mbe + 16 * mbe + 16 + (2 * p["NS"] + 8 if p["BFMT"] == 2 else 0)
                    + 48 + (8 if p.get("EPI") else 0) + (16 if p.get("KSL") else 0))
            return regs, int(regs * 1.25), space.phase_lds(int(op.shapes["K"]), p)
        if kind in ("ilv", "ilv8"):
            tm, tn = p["BM"] // p["WM"] // 16, p["BN"] // p["WN"] // 16
            acc = tm * tn * 4
            nw = p["WM"] * p["WN"]
            if kind == "ilv":
                frags = 2 * (tm + tn) * 4
                L = (p["BM"] + p["BN"]) // (1024 // (p["BK"] * 2) * nw)
            else:  # A fragments double-buffered, weight bytes double-buffered, two dequantised
                frags = 2 * tm * 4 + 2 * tn * 2 + 2 * 4 + 4 * tn
                L = p["BM"] // (1024 // (p["BK"] * 2) * nw) + p["BN"] // (16 * nw)
            regs = acc + frags + 2 * L + 16  # + copy offsets, fragment offsets
            # pessimistic edge: the epilogue converts every accumulator (acc held twice when the
            # budget allows it); the split-K epilogue stores fp32 partials straight from the
            # accumulators, at worst with an address pair live per accumulator block
            pess = max(int(regs * 1.2), 2 * acc + 16) + (2 * tm * tn if p.get("SPLIT") else 0)
            return regs, pess, space.lds_bytes(kind, p)
        if kind in ("dma", "reg"):
            ms = p.get("MS", 32)
            nacc = 16 if ms == 32 else 4
            tm, tn = p["BM"] // p["WM"] // ms, p["BN"] // p["WN"] // ms
            acc = tm * tn * nacc
            frags = 2 * (tm + tn) * 4 if kind == "dma" else (tm + tn) * 4
            if kind == "dma":
                # stages of more than four MFMA k-steps (128 k at MS = 16, 256 k at MS = 16 or
                # 32): the compiler runs the fragment reads of a stage further ahead; measured
                # 64 registers at 32 x 64 x 256 where the double-buffer count gives 48
                frags *= max(1, (p["BK"] // (32 if ms == 16 else 16)) // 4)
            nw = p["WM"] * p["WN"]
            if kind == "dma":
                rpb = 1024 // (p["BK"] * 2)
                copies = 2 * ((p["BM"] + p["BN"]) // (rpb * nw))  # 64-bit source addresses
            else:
                per = (p["BM"] + p["BN"]) * p["BK"] // 8 // (nw * 64)
                copies = per * 4 + per * 2  # staged data + addresses
            regs = acc + frags + copies + 16
            # pessimistic edge: the epilogue reads every accumulator out of the AGPRs before the
            # fp16 conversion, so when the budget allows it the compiler holds acc twice
            return regs, max(int(regs * 1.2), 2 * acc + 16), space.lds_bytes(kind, p)
        wb = 2 if p["BFMT"] == 0 else 1
        if kind == "line":
            rr = 2 * p["R"] if p.get("EPI") and not space.line_paired(p) else p["R"]
            mbe = max(1, p["MB"])
            # fragments of one step (2 halves x (2 per row group for fp16, 1 for 8-bit) + the
            # activation fragments), two accumulator chains, the fp16 expansion of 8-bit
            # weights, 64-bit copy sources, scales / zero-points
            regs = (2 * rr * (2 if wb == 2 else 1) * 4 + 2 * mbe * 2 * 4 + 2 * rr * mbe * 4
                    + (8 * rr if p["BFMT"] else 0) + 2 * (2 * rr + (4 * p["MB"] if p["MB"] else 1))
                    + 2 * rr + 16)
            sp = space.line_split(int(op.shapes["N"]), int(op.shapes["K"]), p)
            return regs, int(regs * 1.25), (sp[2] if sp else space.LDS_MAX + 1)
        S, _ = self._split(op, p)
        if kind == "shared":
            # weights double-buffered (U steps x R slabs x 4*wb VGPRs), the activation fragments
            # of U steps (8 per step per MB), accumulators (8 per R x MB), the fp16 expansion of
            # 8-bit weights (4 per step per slab) plus scale/zero for fmt 2, addresses
            U, R, MB, bf = p["U"], p["R"], p["MB"], p["BFMT"]
            regs = (2 * U * R * wb * 4 + 8 * U * MB + 8 * R * MB + (4 * U * R if bf else 0)
                    + (3 * U * R if bf == 2 else 0) + 14)
            lds = space.shared_split(int(op.shapes["N"]), int(op.shapes["K"]), p["MB"], p["R"],
                                     p["U"], p["SN"], p["TPB"])[2]
            return regs, int(regs * 1.25), lds
        if kind == "ring":
            regs = p["R"] * p["MB"] * 4 + (p["R"] * wb + 2 * p["MB"]) * 4 + 2 * (p["R"] + p["MB"]) + 16
        else:
            # activations: register-staged per step (2*MB per step), or read from the LDS copy
            # just before each MFMA (still MB per step in flight)
            act_regs = p["MB"] if p.get("ALDS", 0) else 2 * p["MB"]
            regs = (2 * p["R"] * p["MB"] * 4 + 2 * p["U"] * (p["R"] * wb + act_regs) * 4
                    + 2 * (p["R"] + p["MB"]) + 16)
        lds = space.lds_bytes(kind, dict(p, S=S))
        if kind == "stream" and p.get("ALDS", 0):
            lds += int(op.shapes["M"]) * (2 * int(op.shapes["K"]) + 16)
        return regs, int(regs * 1.25), lds

    def launch_of(self, op: OpSpec, h: Hyperform) -> Launch:
        p = _p(h)
        kind = p["kind"]
        minb, bound = 1, 0
        if kind != "fmha":
            M, N = int(op.shapes["M"]), int(op.shapes["N"])
        if kind == "fmha":  # one workgroup per (128 query rows, head, batch)
            s = op.shapes
            grid = -(-int(s["SQ"]) // p["BQ"]) * int(s["H"]) * int(s["B"])
            _, _, lds = self.resources_of(op, h)
            return Launch(grid_ctas=grid, threads=64 * p["WAVES"], smem_bytes=lds,
                          entry=self.entry_probe(h), min_ctas_per_sm=1,
                          bound_threads=64 * p["WAVES"])
        if kind in ("dma", "reg", "ilv", "ilv8"):
            grid = (-(-M // p["BM"]) * (N // p["BN"])
                    * space.splits_of(kind, p, M, N, int(op.shapes["K"])))
            threads = p["WM"] * p["WN"] * 64
            minb = p.get("MINB", 1) if kind == "dma" else 1
        elif kind == "shared":
            S, _ = self._split(op, p)
            grid = N // (16 * p["R"] * p["SN"])
            threads = 64 * p["SN"] * S
            bound = p["TPB"]  # __launch_bounds__(TPB)
        elif kind == "phase":  # one workgroup of 8 waves per CU
            grid, threads, bound = space.PHASE_CUS, 64 * space.PHASE_WAVES, 512
        elif kind == "line" and p.get("MT"):  # row tiles x slab groups
            sp = space.line_split(N, int(op.shapes["K"]), p)
            grid = -(-M // (16 * p["MB"])) * (N // (16 * p["R"]))
            threads = 64 * (sp[0] if sp else 1)
            bound = p["TPB"]
        elif kind == "line":
            sp = space.line_split(N, int(op.shapes["K"]), p)
            grid = (N // (16 * p["R"] * (p["SN"] // 2 if space.line_paired(p) else p.get("SN", 1)))
                    * (sp[3] if sp else 1))
            threads = 64 * p.get("SN", 1) * (sp[0] if sp else 1)
            bound = p.get("TPB", 1024)  # k_stream_line: __launch_bounds__(TPB)
        else:
            S, _ = self._split(op, p)
            grid = N // (16 * p["R"])
            threads = 64 * S
            bound = 512  # k_stream / k_stream_dma: __launch_bounds__(512)
        _, _, lds = self.resources_of(op, h)
        return Launch(grid_ctas=grid, threads=threads, smem_bytes=lds, entry=self.entry_probe(h),
                      min_ctas_per_sm=minb, bound_threads=bound)

    def estimate_atoms(self, op: OpSpec, h: Hyperform) -> list:
        """Per-wave load of the whole operation on the channels MFMA (flop), LDS and VMEM (bytes),
        as one compute unit sees it: one k-tile (or k-step) footprint times the number of times a
        CU replays it (k-tiles x rounds of resident workgroups)."""
        p = _p(h)
        kind = p["kind"]
        if kind != "fmha":
            M, N, K = int(op.shapes["M"]), int(op.shapes["N"]), int(op.shapes["K"])
        regs, _, lds = self.resources_of(op, h)
        lau = self.launch_of(op, h)
        occ = _RES.occupancy(min(regs, _RES.declared_budget(lau.threads, lau.min_ctas_per_sm,
                                                            lau.bound_threads)), lds, lau.threads)
        per_cu = max(1, occ.ctas_per_sm)
        rounds = -(-lau.grid_ctas // (int(_M.rate("GEOM.SMS").value) * per_cu))
        # a grid smaller than one residency round leaves slots empty: a CU then holds only
        # ceil(grid / CUs) workgroups, and its per-wave load counts that many times, not per_cu
        fill = min(per_cu, -(-lau.grid_ctas // int(_M.rate("GEOM.SMS").value))) / per_cu
        atoms = []
        if kind == "fmha":
            return self._fmha_atoms(op, p, lau, occ, rounds, fill)
        if kind in ("dma", "reg", "ilv", "ilv8"):
            ms = p.get("MS", 32) if kind not in ("ilv", "ilv8") else 16
            tm, tn = p["BM"] // p["WM"] // ms, p["BN"] // p["WN"] // ms
            ks = p["BK"] // (16 if ms == 32 else 32)
            nw = p["WM"] * p["WN"]
            sp = space.splits_of(kind, p, M, N, K)
            reps = -(-(K // p["BK"]) // sp) * rounds  # k-tiles of one split
            flops = tm * tn * ks * space.MFMA_FLOPS[ms]
            lds_rd = (tm + tn) * ks * 1024 if kind != "ilv8" else (tm * 1024 + tn * 512) * ks
            vmem = (p["BM"] + p["BN"]) * p["BK"] * 2 // nw
            if p.get("BFMT", 0):
                vmem = p["BM"] * p["BK"] * 2 // nw + p["BN"] * p["BK"] // nw
        elif kind == "phase":
            # a wave's step: 16 rows x 128 k of weights (two 1 KiB copies, two 16-byte reads a
            # lane) against 4 MBE MFMAs; a phase's activations (4 MBE KiB, or 256 B at M = 1)
            # copied and read once per NS steps
            mbe = max(1, p["MB"])
            act = 4 * p["MB"] * 1024 if p["MB"] else 256
            reps = p["NS"] * -(-K // (128 * p.get("KS", 1) * space.PHASE_WAVES)) * rounds
            flops = 4 * mbe * space.MFMA_FLOPS[16]
            vmem = 2048 + act // p["NS"]
            lds_rd = 2048 + act // p["NS"]
        elif kind == "line":
            wb = 2 if p["BFMT"] == 0 else 1
            sp = space.line_split(N, K, p)
            reps = (sp[1] if sp else K // 128) * rounds
            flops = 4 * p["R"] * max(1, p["MB"]) * space.MFMA_FLOPS[16]
            copies, wslot, aslot = space.line_geometry(p)
            vmem = wslot + aslot // p.get("SN", 1)
            lds_rd = wslot + aslot
        else:
            wb = 2 if p["BFMT"] == 0 else 1
            S, chunk = self._split(op, p)
            reps = (chunk // 64) * rounds
            flops = 2 * p["R"] * p["MB"] * space.MFMA_FLOPS[16]
            vmem = (p["R"] * wb + 2 * p["MB"]) * 1024
            lds_rd = vmem if kind == "ring" else 0
        reps *= fill
        atoms.append(Atom(uid=0, kind=AtomKind.COMPUTE, op_id="v_mfma x%d" % (flops // 16384),
                          footprint={"MFMA": float(flops * reps)},
                          latency=_M.rate("LATENCY.MFMA32").value))
        if lds_rd:
            atoms.append(Atom(uid=1, kind=AtomKind.MEM_READ, op_id="ds_read_b128",
                              footprint={"LDS": float(lds_rd * reps)},
                              latency=_M.rate("LATENCY.LDS").value))
        atoms.append(Atom(uid=2, kind=AtomKind.XFER_ISSUE,
                          op_id=("buffer_load_dwordx4 lds" if kind in ("ilv", "ilv8") else
                                 "global_load_lds_dwordx4" if kind in ("dma", "ring", "line", "phase")
                                 else "global_load_dwordx4"),
                          footprint={"VMEM": float(vmem * reps)},
                          latency=_M.rate("LATENCY.VMEM").value, token="copy"))
        atoms.append(Atom(uid=3, kind=AtomKind.XFER_WAIT, op_id="s_waitcnt vmcnt", footprint={},
                          token="copy"))
        atoms.append(Atom(uid=4, kind=AtomKind.BARRIER, op_id="s_barrier", footprint={}))
        # device-wide HBM floor: the operation's HBM bytes (weights and their metadata once,
        # activations, output, and the fp32 partial sums a split writes and reads back), each CU
        # carrying 1/CUS of them, per resident wave
        bf = p.get("BFMT", 0)
        hbm = (N * K * (2 if bf == 0 else 1) + (2 * N if bf == 1 else 3 * N * K // 128 if bf == 2 else 0)
               + 2 * M * K + 2 * M * N)
        if kind in ("ilv", "ilv8"):
            hbm += 2 * 4 * M * N * space.splits_of(kind, p, M, N, K) if p.get("SW") else 0
        elif kind == "line":
            sp = space.line_split(N, K, p)
            hbm += 2 * 4 * M * N * sp[3] if sp and sp[3] > 1 else 0
        elif kind == "phase" and p.get("KS", 1) > 1:
            hbm += 2 * 4 * M * N * p["KS"]
        cus = int(_M.rate("GEOM.SMS").value)
        atoms.append(Atom(uid=5, kind=AtomKind.MEM_READ, op_id="HBM (device share)",
                          footprint={"HBM": float(hbm) / (cus * max(1, occ.warps_per_sm))},
                          latency=_M.rate("LATENCY.VMEM").value))
        return atoms

    def _fmha_atoms(self, op: OpSpec, p: dict, lau, occ, rounds, fill):
        """Per-wave load of the attention skeleton: per 32-key block a wave runs the scores
        (32 x 32 x D) and P.V (32 x D x 32) on the matrix cores, reads that block's K and V from
        LDS (32 x D x 2 bytes each), and issues a quarter of the block's K and V copies; a
        workgroup walks the key blocks its 128 query rows see (with the causal mask, about the
        mean visible keys of a row plus the half block of its diagonal)."""
        from tempo.core.op.spec import visible_pairs

        s = op.shapes
        D, BKV = p["D"], p["BKV"]
        sq, sk = int(s["SQ"]), int(s["SK"])
        mean_keys = visible_pairs(sq, sk, int(s["CAUSAL"])) / sq
        blocks = min(-(-sk // BKV), -(-int(mean_keys + p["BQ"] / 2) // BKV))
        reps = blocks * rounds * fill
        flops = 4 * BKV * 32 * D  # scores + P.V of one block for the wave's 32 query rows
        lds_rd = 2 * BKV * D * 2
        vmem = 2 * BKV * D * 2 // p["WAVES"]
        hbm = (2 * int(s["B"]) * sq * int(s["H"]) * D * 2
               + 2 * int(s["B"]) * sk * int(s["HKV"]) * D * 2)
        cus = int(_M.rate("GEOM.SMS").value)
        return [
            Atom(uid=0, kind=AtomKind.COMPUTE, op_id="v_mfma x%d" % (flops // 32768),
                 footprint={"MFMA": float(flops * reps)}, latency=_M.rate("LATENCY.MFMA32").value),
            Atom(uid=1, kind=AtomKind.MEM_READ, op_id="ds_read_b128 / ds_read_b64_tr_b16",
                 footprint={"LDS": float(lds_rd * reps)}, latency=_M.rate("LATENCY.LDS").value),
            Atom(uid=2, kind=AtomKind.XFER_ISSUE, op_id="buffer_load_dwordx4 lds",
                 footprint={"VMEM": float(vmem * reps)}, latency=_M.rate("LATENCY.VMEM").value,
                 token="copy"),
            Atom(uid=3, kind=AtomKind.XFER_WAIT, op_id="s_waitcnt vmcnt", footprint={},
                 token="copy"),
            Atom(uid=4, kind=AtomKind.BARRIER, op_id="s_barrier", footprint={}),
            Atom(uid=5, kind=AtomKind.MEM_READ, op_id="HBM (device share)",
                 footprint={"HBM": float(hbm) / (cus * max(1, occ.warps_per_sm))},
                 latency=_M.rate("LATENCY.VMEM").value),
        ]

    # -- emission ------------------------------------------------------------------------------
    def render(self, op: OpSpec, h: Hyperform) -> Rendered:
        self._require_form_v1(op)
        p = _p(h)
        kind = p["kind"]
        if kind not in _ENTRY:
            raise PluginCapabilityError("no entry declared for skeleton kind %r" % kind)
        sym, _, args, files = _ENTRY[kind]
        order = _order(kind, p)
        body = []
        for f in files:
            with open(os.path.join(SKEL, f), encoding="utf-8") as fh:
                body.append("// ===== %s =====\n%s\n" % (f, fh.read()))
        head = ("// GENERATED by tempo: plugin gfx950, hyperform %s, operation %s %s.\n"
                % (h.key, op.kind, " ".join("%s=%s" % kv for kv in sorted(op.shapes.items()))))
        if kind in KIND_FLAGS:
            head += "// tempo:flags %s\n" % " ".join(KIND_FLAGS[kind])
        head += ("#include <hip/hip_runtime.h>\n#include <stdint.h>\n\nnamespace tempo {\n"
                 "namespace gen {\n\n")
        inst = ("\n// explicit instantiation: the one kernel this file exists to contain\n"
                "template __global__ void %s<%s>(%s);\n"
                % (sym, ", ".join(_targ(kind, k, p.get(k, _DEFAULT.get(k, 0))) for k in order),
                   args))
        src = head + "".join(body) + inst + "\n}  // namespace gen\n}  // namespace tempo\n"
        return Rendered(source=src, launch=self.launch_of(op, h), includes=(),
                        notes="namespace wrap + one explicit instantiation; logic lives in the skeleton",
                        filename="kernel_%s.hip" % h.key)

    def entry_probe(self, h: Hyperform) -> str:
        """The kernel's name as the profiler prints it (demangled template id)."""
        p = _p(h)
        sym = _ENTRY[p["kind"]][0]
        order = _order(p["kind"], p)
        vals = [_targ(p["kind"], k, p.get(k, _DEFAULT.get(k, 0))) for k in order]
        return "%s::%s<%s>" % (NAMESPACE, sym, ", ".join(vals))
