"""Device route plan and routed MoE (drop-in for qwen35_deploy/runtime/gpu_routes.py).

plan        one-block HIP kernel: stable counting sort of the flat routing
            ids, tile table, ordered/slots (gpu_routes.py:17-63) - no host
            synchronisation, no torch sort.
routed_moe  plan -> grouped gate_up GEMM with the SwiGLU glue fused into the
            MFMA epilogue -> grouped down GEMM -> ordered combine
            (gpu_routes.py:66-82).  The expert bank is HBM-resident, so the
            ready_event hook of the reference's PCIe double buffer is only
            honoured for API compatibility.
"""
import torch

from .. import _lib

# Tile heights of the MFMA grouped GEMM.  96 rows cover a typical expert
# (64 +- 8 routes per 2048-token chunk) in one tile, so its weights stream
# once through the pipelined kernel; the reference's large_tile switch
# (gpu_routes.py:67) selects 128-row tiles (register-prefetch kernel).
BM_DEFAULT = 96
BM_LARGE = 128


def _check_ids(ids):
    if ids.device.type != 'cuda' or ids.ndim != 2 or not ids.is_contiguous():
        raise ValueError('Expected contiguous CUDA [tokens,top_k] routing IDs')
    if ids.dtype != torch.int64:
        raise ValueError('Expected contiguous CUDA [tokens,top_k] routing IDs')


def plan(ids, experts, bm):
    """Returns (pos [R], table [cdiv(R, bm) + experts, 3], ordered [T, k], slots [T, k]).

    pos[p] is the token of the p-th route in stable expert order; table rows
    are (expert, start, stop) per bm-row tile, surplus rows (0, 0, 0);
    ordered[t, i] is the sorted position of token t's i-th smallest-id route
    and slots = argsort(ids, dim=1, stable).  ids must lie in [0, experts).
    """
    _check_ids(ids)
    tokens, top = ids.shape
    routes = tokens * top
    max_tiles = (routes + bm - 1) // bm + experts
    dev = ids.device
    pos = torch.empty(routes, dtype=torch.int64, device=dev)
    table = torch.empty((max_tiles, 3), dtype=torch.int64, device=dev)
    ordered = torch.empty((tokens, top), dtype=torch.int64, device=dev)
    slots = torch.empty((tokens, top), dtype=torch.int64, device=dev)
    _lib.call('lm_route_plan', ids.data_ptr(), tokens, top, int(experts), int(bm), pos.data_ptr(),
              table.data_ptr(), max_tiles, ordered.data_ptr(), slots.data_ptr(),
              _lib.stream(dev))
    return pos, table, ordered, slots


def _check_bank(q, s):
    if q.dtype != torch.int8 or s.dtype != torch.float32 or q.ndim != 3 or s.ndim != 3:
        raise ValueError('Invalid INT8 group geometry')
    e, n, k = q.shape
    if k % 128 or tuple(s.shape) != (e, n, k // 128):
        raise ValueError('Invalid INT8 group geometry')
    if q.stride(2) != 1 or q.stride(1) != k or s.stride(2) != 1 or s.stride(1) != k // 128:
        raise ValueError('Invalid INT8 group geometry')


def routed_gemm(x, q, s, pos, table, bm, gather):
    """Routed grouped W8A16 GEMM (prefill._routed / _nonempty) -> bf16 [R, N]."""
    _check_bank(q, s)
    routes = pos.numel()
    out = torch.empty((routes, q.shape[1]), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gemm_w8a16', x.data_ptr(), q.data_ptr(), s.data_ptr(), pos.data_ptr(),
              table.data_ptr(), table.shape[0], int(bm), out.data_ptr(), q.shape[1], q.shape[2],
              int(bool(gather)), q.stride(0), s.stride(0), _lib.stream(x.device))
    return out


def routed_reduce(values, ordered, slots, weights, tokens, n):
    """Prefill combine (prefill._reduce): ascending-expert bf16 accumulation per token."""
    out = torch.empty((tokens, n), device=values.device, dtype=values.dtype)
    weights = weights.contiguous()
    _lib.call('lm_routed_reduce', values.data_ptr(), ordered.data_ptr(), slots.data_ptr(),
              weights.data_ptr(), _lib.dtype_code(weights.dtype), out.data_ptr(), tokens, n,
              ordered.shape[1], _lib.stream(values.device))
    return out


def routed_moe(x, weights, ids, banks, large_tile=False, ready_event=None):
    """Routed experts of one MoE layer for a prefill chunk -> bf16 [T, H]."""
    if not x.is_cuda or x.dtype != torch.bfloat16 or x.ndim != 2:
        raise ValueError('W8A16 requires CUDA FP16/BF16 activations')
    x = x.contiguous()
    bm = BM_LARGE if large_tile else BM_DEFAULT
    qg, sg, qd, sd = banks
    _check_bank(qg, sg)
    _check_bank(qd, sd)
    if qg.shape[2] != x.shape[1] or qd.shape[2] * 2 != qg.shape[1] or qd.shape[1] != x.shape[1]:
        raise ValueError('Invalid INT8 group geometry')
    pos, table, ordered, slots = plan(ids, qg.shape[0], bm)
    routes = ids.numel()
    if ready_event is not None:
        torch.cuda.current_stream().wait_event(ready_event)
    hidden = torch.empty((routes, qg.shape[1] // 2), device=x.device, dtype=x.dtype)
    st = _lib.stream(x.device)
    _lib.call('lm_routed_gate_up_swiglu', x.data_ptr(), qg.data_ptr(), sg.data_ptr(),
              pos.data_ptr(), table.data_ptr(), table.shape[0], bm, hidden.data_ptr(),
              qg.shape[1], qg.shape[2], qg.stride(0), sg.stride(0), st)
    down = torch.empty((routes, qd.shape[1]), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gemm_w8a16', hidden.data_ptr(), qd.data_ptr(), sd.data_ptr(),
              pos.data_ptr(), table.data_ptr(), table.shape[0], bm, down.data_ptr(), qd.shape[1],
              qd.shape[2], 0, qd.stride(0), sd.stride(0), st)
    return routed_reduce(down, ordered, slots, weights, x.shape[0], x.shape[1])
