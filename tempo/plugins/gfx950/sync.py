"""gfx950: SYNC AND TRANSACTIONS -- section 5 (reference pattern tempo/plugins/sm70/sync.py).

Two ways to feed LDS from global memory, and the contract's falsifier field tells them apart:
  gmem->vgpr->lds   global_load_dwordx4 into registers, then ds_write_b128: the staging
                    registers cost occupancy (consumes_registers=True); used where the data is
                    transformed on the way (W8A16 dequantisation while staging).
  gmem->lds:dma     global_load_lds_dwordx4 (gfx950 LDS DMA): 1 KiB per wave instruction straight
                    into LDS, counted by vmcnt, no registers (consumes_registers=False).
Barrier: s_barrier, workgroup scope, not phased, not counted."""
from __future__ import annotations

from ..base import BarrierKind, Rate, TransactionKind, rate
from .machine import Gfx950Machine

_M = Gfx950Machine()


class Gfx950Sync:
    def transactions(self) -> tuple:
        return (
            TransactionKind(id="gmem->vgpr->lds", issue_op="global_load_dwordx4+ds_write_b128",
                            wait_op="s_waitcnt vmcnt", granularity="instruction",
                            in_flight_max=rate("VMCNT.MAX", 63, "instr", "SPEC"),
                            occupies={"VMEM": 1.0, "LDS": 1.0}, consumes_registers=True,
                            consumes_smem_staging=True, depth_axis="stages"),
            TransactionKind(id="gmem->lds:dma", issue_op="global_load_lds_dwordx4",
                            wait_op="s_waitcnt vmcnt + s_barrier", granularity="barrier",
                            in_flight_max=rate("VMCNT.MAX", 63, "instr", "SPEC"),
                            occupies={"VMEM": 1.0}, consumes_registers=False,
                            consumes_smem_staging=True, depth_axis="stages"),
        )

    def barriers(self) -> tuple:
        return (BarrierKind(id="s_barrier", scope="cta", phased=False, counted=False,
                            cost=rate("BARRIER.COST", 16, "clk", "MODEL")),)

    def rendezvous_cost(self, barrier_id: str, participants: int) -> Rate:
        if barrier_id != "s_barrier":
            from ..base import UnknownSymbol

            raise UnknownSymbol("barrier %r is not declared" % barrier_id)
        return rate("BARRIER.COST", 16 + 2 * max(0, participants - 1), "clk", "MODEL")
