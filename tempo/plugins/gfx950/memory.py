"""gfx950: MEMORY -- section 2 (reference pattern tempo/plugins/sm70/memory.py).

LDS bank law used by the model: 64 banks of 4 bytes; a wide access (ds_read_b64/b128) is served
in passes of 256 bytes, 16 lanes of a b128 per pass.  The conflict degree of one pass is the
largest number of distinct 4-byte words that land in one bank; the cost of an access is
max(degree, width/64B floor) passes per quarter-wave.  The skeletons' XOR swizzles are chosen so
16 consecutive rows of one 16-byte chunk land in 16 distinct bank groups (SWZ 2); SWZ 1 targets a
32-bank, 8-lane-per-pass reading of the same law.  Which one the hardware rewards is measured
(SQ_LDS_BANK_CONFLICT) -- the law here is a model, not a datasheet."""
from __future__ import annotations

from ..base import Layout, MemLevel, WavefrontCost, rate, not_measured
from .machine import Gfx950Machine

_M = Gfx950Machine()
BANKS = 64
BANK_BYTES = 4


class Gfx950Memory:
    def levels(self) -> tuple:
        return (
            MemLevel("LDS", _M.rate("GEOM.SMEM_PER_SM"), _M.rate("CAP.LDS"), _M.rate("LATENCY.LDS")),
            MemLevel("L2", _M.rate("PEAK.L2_BYTES_PER_XCD"), _M.rate("CAP.VMEM_L2"),
                     not_measured("LATENCY.L2", "clk")),
            MemLevel("MALL", _M.rate("PEAK.MALL_BYTES"), not_measured("BW.MALL", "GB/s"),
                     not_measured("LATENCY.MALL", "clk")),
            MemLevel("HBM", _M.rate("PEAK.HBM_BYTES"), _M.rate("PEAK.HBM"), _M.rate("LATENCY.VMEM")),
        )

    def wavefronts(self, lane_words, width_bytes: int) -> WavefrontCost:
        """lane_words: starting 4-byte word address of each lane's access (one wave)."""
        words_per_lane = max(1, width_bytes // BANK_BYTES)
        lanes_per_pass = max(1, (BANKS * BANK_BYTES) // max(BANK_BYTES, width_bytes))
        worst = 1
        passes = 0
        lw = list(lane_words)
        for p0 in range(0, len(lw), lanes_per_pass):
            banks = {}
            for w0 in lw[p0:p0 + lanes_per_pass]:
                for j in range(words_per_lane):
                    w = int(w0) + j
                    banks.setdefault(w % BANKS, set()).add(w)
            deg = max(len(v) for v in banks.values()) if banks else 1
            worst = max(worst, deg)
            passes += deg
        floor = max(1.0, width_bytes / 64.0)
        return WavefrontCost(degree=float(worst), floor=floor, wavefronts=float(max(passes, 1)))

    def alignment_rule(self, width_bytes: int) -> int:
        return max(4, width_bytes)

    def pad_family(self, layout: Layout):
        return (0,)  # the skeletons swizzle instead of padding (padding would cost LDS capacity)

    def swizzle_family(self, layout: Layout):
        return ("none", "xor_row128", "xor_row256")

    def residency_policy(self) -> str:
        return "l2_per_xcd+mall_shared"
