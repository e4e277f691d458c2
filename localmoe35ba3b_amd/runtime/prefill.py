"""Host-planned routed MoE (drop-in for routed_moe of qwen35_deploy/runtime/prefill.py).

The route plan is computed on the host by the native plan_routes
(routing.py:5-20 semantics) and uploaded; the grouped GEMMs and the combine
run on the GPU kernels.  The reference's PrefillPipeline (pinned host bank,
slab double buffer, prefill.py:88-164) has no counterpart: the bank is
HBM-resident.
"""
import torch

from .. import _lib
from ..operators.routing import plan_routes
from . import gpu_routes


def routed_moe(x, weights, ids, banks, large_tile=False, stats=None, ready_event=None):
    """Same result as gpu_routes.routed_moe with a host-computed plan (prefill.py:52-85)."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError('W8A16 requires CUDA FP16/BF16 activations')
    x = x.contiguous()
    bm = gpu_routes.BM_LARGE if large_tile else gpu_routes.BM_DEFAULT
    cpu = ids.cpu()
    qg, sg, qd, sd = banks
    positions, segments = plan_routes(cpu, qg.shape[0])
    if stats is not None:
        stats.update(active_experts=len(segments), total_experts=qg.shape[0],
                     routed_tokens=cpu.numel(), tokens=x.shape[0])
    tiles = [(e, start, stop) for e, begin, stop in segments for start in range(begin, stop, bm)]
    table = torch.tensor(tiles, dtype=torch.int64).reshape(-1, 3).to(x.device)
    pos = positions[0].to(x.device)
    routes = cpu.numel()
    top = cpu.shape[1]
    slots = cpu.argsort(dim=1, stable=True)
    original = positions[0] * top + positions[1]
    inverse = torch.empty_like(original)
    inverse[original] = torch.arange(routes)
    ordered = inverse[torch.arange(cpu.shape[0])[:, None] * top + slots]
    ordered, slots = ordered.to(x.device), slots.to(x.device)
    if ready_event is not None:
        torch.cuda.current_stream().wait_event(ready_event)
    st = _lib.stream(x.device)
    hidden = torch.empty((routes, qg.shape[1] // 2), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gate_up_swiglu', x.data_ptr(), qg.data_ptr(), sg.data_ptr(),
              pos.data_ptr(), table.data_ptr(), table.shape[0], bm, hidden.data_ptr(),
              qg.shape[1], qg.shape[2], qg.stride(0), sg.stride(0), st)
    down = torch.empty((routes, qd.shape[1]), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gemm_w8a16', hidden.data_ptr(), qd.data_ptr(), sd.data_ptr(),
              pos.data_ptr(), table.data_ptr(), table.shape[0], bm, down.data_ptr(), qd.shape[1],
              qd.shape[2], 0, qd.stride(0), sd.stride(0), st)
    return gpu_routes.routed_reduce(down, ordered, slots, weights, x.shape[0], x.shape[1])
