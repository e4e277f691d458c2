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


def _check_activation(x):
    if not x.is_cuda or x.dtype not in (torch.bfloat16, torch.float16) or x.ndim != 2:
        raise ValueError('W8A16 requires CUDA FP16/BF16 activations')


def routed_gemm(x, q, s, pos, table, bm, gather):
    """Routed grouped W8A16 GEMM (prefill._routed / _nonempty) -> [R, N] in x.dtype.

    R = pos.numel(): the rows of the plan; gather reads x[pos[r]], otherwise
    x[r] (then x needs at least R rows)."""
    _check_bank(q, s)
    _check_activation(x)
    x = x.contiguous()
    routes = pos.numel()
    out = torch.empty((routes, q.shape[1]), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gemm_w8a16', x.data_ptr(), x.shape[0], q.data_ptr(), s.data_ptr(),
              q.shape[0], q.stride(0), s.stride(0), pos.data_ptr(), table.data_ptr(),
              table.shape[0], int(bm), out.data_ptr(), routes, q.shape[1], q.shape[2],
              int(bool(gather)), _lib.dtype_code(x.dtype), _lib.stream(x.device))
    return out


def routed_reduce(values, ordered, slots, weights, tokens, n):
    """Prefill combine (prefill._reduce): ascending-expert accumulation per
    token, rounded to the values' dtype at every step."""
    out = torch.empty((tokens, n), device=values.device, dtype=values.dtype)
    weights = weights.contiguous()
    _lib.call('lm_routed_reduce', values.data_ptr(), ordered.data_ptr(), slots.data_ptr(),
              weights.data_ptr(), _lib.dtype_code(weights.dtype), out.data_ptr(), tokens, n,
              ordered.shape[1], _lib.dtype_code(values.dtype), _lib.stream(values.device))
    return out


def run_plan(x, weights, banks, pos, table, ordered, slots, bm, ready_event=None):
    """The device half of routed_moe for a plan already on the device:
    grouped gate_up with the SwiGLU glue fused into its epilogue, grouped
    down, ordered combine (prefill.py:69-85, gpu_routes.py:69-82)."""
    qg, sg, qd, sd = banks
    routes = pos.numel()
    if ready_event is not None:
        torch.cuda.current_stream().wait_event(ready_event)
    st = _lib.stream(x.device)
    code = _lib.dtype_code(x.dtype)
    hidden = torch.empty((routes, qg.shape[1] // 2), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gate_up_swiglu', x.data_ptr(), x.shape[0], qg.data_ptr(), sg.data_ptr(),
              qg.shape[0], qg.stride(0), sg.stride(0), pos.data_ptr(), table.data_ptr(),
              table.shape[0], bm, hidden.data_ptr(), routes, qg.shape[1], qg.shape[2], code, st)
    down = torch.empty((routes, qd.shape[1]), device=x.device, dtype=x.dtype)
    _lib.call('lm_routed_gemm_w8a16', hidden.data_ptr(), routes, qd.data_ptr(), sd.data_ptr(),
              qd.shape[0], qd.stride(0), sd.stride(0), pos.data_ptr(), table.data_ptr(),
              table.shape[0], bm, down.data_ptr(), routes, qd.shape[1], qd.shape[2], 0, code, st)
    return routed_reduce(down, ordered, slots, weights, x.shape[0], x.shape[1])


def check_banks(x, banks):
    """Validates x against the routed banks [qg, sg, qd, sd] (reference format)."""
    _check_activation(x)
    qg, sg, qd, sd = banks
    _check_bank(qg, sg)
    _check_bank(qd, sd)
    if qg.shape[2] != x.shape[1] or qd.shape[2] * 2 != qg.shape[1] or qd.shape[1] != x.shape[1]:
        raise ValueError('Invalid INT8 group geometry')
    if qd.shape[0] != qg.shape[0]:
        raise ValueError('Invalid INT8 group geometry')


def routed_moe(x, weights, ids, banks, large_tile=False, ready_event=None):
    """Routed experts of one MoE layer for a prefill chunk -> [T, H] in x.dtype."""
    check_banks(x, banks)
    x = x.contiguous()
    bm = BM_LARGE if large_tile else BM_DEFAULT
    pos, table, ordered, slots = plan(ids, banks[0].shape[0], bm)
    return run_plan(x, weights, banks, pos, table, ordered, slots, bm, ready_event)
