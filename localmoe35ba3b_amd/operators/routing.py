"""Stable host routing plan (drop-in for qwen35_deploy/operators/routing.py).

plan_routes runs in the native library (lm_plan_routes_host, a stable
counting sort) on CPU tensors, exactly like the reference's CPU function.
"""
import torch

from .. import _lib


def plan_routes(ids, experts):
    """Returns (positions int64 [2, R], segments [(expert, start, stop), ...]).

    positions[0] is the token and positions[1] the top-k slot of each route in
    stable expert order; segments lists the non-empty experts (routing.py:5-20).
    """
    if ids.device.type != 'cpu' or ids.ndim != 2 or ids.numel() == 0:
        raise ValueError('Expected nonempty CPU [tokens,top_k] IDs')
    flat = ids.to(torch.int64).contiguous()
    routes = flat.numel()
    positions = torch.empty((2, routes), dtype=torch.int64)
    seg = torch.empty((3, max(int(experts), 1)), dtype=torch.int64)
    count = torch.zeros(1, dtype=torch.int64)
    _lib.call('lm_plan_routes_host', flat.data_ptr(), ids.shape[0], ids.shape[1], int(experts),
              positions.data_ptr(), seg[0].data_ptr(), seg[1].data_ptr(), seg[2].data_ptr(),
              count.data_ptr())
    n = int(count.item())
    segments = [tuple(int(v) for v in seg[:, i]) for i in range(n)]
    return positions, segments


def tile_plan(ids, experts, bm):
    """Host route plan in the device plan's format, for CPU routing ids.

    Returns (pos [R], table [n_tiles, 3], ordered [T, k], slots [T, k],
    active) as int64 CPU tensors: the plan gpu_routes.plan computes on the
    device, except that the table holds only the bm-row tiles of the
    non-empty experts (what the reference's host-planned prefill launches,
    prefill.py:52-68) and `active` counts those experts.  Computed by
    lm_route_plan_host, one stable counting sort.
    """
    if ids.device.type != 'cpu' or ids.ndim != 2 or ids.numel() == 0:
        raise ValueError('Expected nonempty CPU [tokens,top_k] IDs')
    flat = ids.to(torch.int64).contiguous()
    tokens, top = ids.shape
    routes = flat.numel()
    capacity = (routes + bm - 1) // bm + int(experts)
    pos = torch.empty(routes, dtype=torch.int64)
    table = torch.empty((capacity, 3), dtype=torch.int64)
    ordered = torch.empty((tokens, top), dtype=torch.int64)
    slots = torch.empty((tokens, top), dtype=torch.int64)
    counts = torch.zeros(2, dtype=torch.int64)
    _lib.call('lm_route_plan_host', flat.data_ptr(), tokens, top, int(experts), int(bm),
              pos.data_ptr(), table.data_ptr(), capacity, ordered.data_ptr(), slots.data_ptr(),
              counts[0:1].data_ptr(), counts[1:2].data_ptr())
    n_tiles, active = (int(v) for v in counts)
    return pos, table[:n_tiles], ordered, slots, active
