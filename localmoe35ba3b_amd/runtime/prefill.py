"""Host-planned routed MoE (drop-in for routed_moe of qwen35_deploy/runtime/prefill.py).

The reference reads the routing ids to the host, plans the routes there and
uploads the plan (prefill.py:52-68).  Here the ids are read once into host
memory and the whole plan - sorted rows, tile table, combine order - comes
from one native call (routing.tile_plan, a stable counting sort in the
library); the grouped GEMMs and the combine then run exactly as in the
device-planned gpu_routes.routed_moe.  The reference's PrefillPipeline
(pinned host bank, slab double buffer, prefill.py:88-164) has no
counterpart: the bank is HBM-resident.
"""
import torch

from ..operators import routing
from . import gpu_routes


def routed_moe(x, weights, ids, banks, large_tile=False, stats=None, ready_event=None):
    """Same result as gpu_routes.routed_moe with a host-computed plan.

    stats, if given, receives the routing statistics the reference reports
    (active_experts, total_experts, routed_tokens, tokens)."""
    gpu_routes.check_banks(x, banks)
    x = x.contiguous()
    bm = gpu_routes.BM_LARGE if large_tile else gpu_routes.BM_DEFAULT
    experts = banks[0].shape[0]
    host_ids = ids.detach().to('cpu', torch.int64)
    pos, table, ordered, slots, active = routing.tile_plan(host_ids, experts, bm)
    if stats is not None:
        stats.update(active_experts=active, total_experts=experts,
                     routed_tokens=host_ids.numel(), tokens=x.shape[0])
    dev = x.device
    plan = [t.to(dev, non_blocking=False) for t in (pos, table, ordered, slots)]
    return gpu_routes.run_plan(x, weights, banks, *plan, bm, ready_event)
