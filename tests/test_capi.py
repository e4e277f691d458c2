"""CPU checks of the C ABI: the library loads, exports every declared symbol,
validates arguments before any launch, and the host route planner matches the
oracle.  No kernel is launched here (there may be no GPU)."""
import ctypes
import pathlib
import re

import numpy as np
import pytest
import torch

from localmoe35ba3b_amd import _lib
from localmoe35ba3b_amd.operators import int8, routing, w8a8
from localmoe35ba3b_amd.runtime import gpu_routes
from oracle import moe_oracle as O

HEADER = pathlib.Path(__file__).resolve().parents[1] / 'include' / 'localmoe35ba3b.h'


def declared_functions():
    text = re.sub(r'/\*.*?\*/', '', HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r'\b(lm_[a-z0-9_]+)\s*\(', text)))


def test_header_declares_what_python_binds():
    names = declared_functions()
    assert len(names) >= 20
    assert sorted(_lib.SIGNATURES) == names


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert b'gfx950' in lib.lm_version()


def test_invalid_geometry_rejected_before_launch():
    lib = _lib.lib()
    rc = lib.lm_w8a16_linear(None, None, None, None, 4, 64, 100, 0, 0, None)
    assert rc == _lib.LM_EINVAL
    assert b'Invalid INT8 group geometry' in lib.lm_last_error()
    assert lib.lm_w8a16_linear(None, None, None, None, 4, 64, 128, 7, 0, None) == _lib.LM_EINVAL
    assert b'FP16/BF16' in lib.lm_last_error()
    assert lib.lm_act_quant_g128(None, 0, None, None, 2, 130, None) == _lib.LM_EINVAL
    assert b'K divisible by 128' in lib.lm_last_error()
    assert lib.lm_route_plan(None, 4, 8, 300, 16, None, None, 0, None, None, None) == _lib.LM_EINVAL
    assert lib.lm_route_plan(None, 4, 8, 256, 16, None, None, 5, None, None, None) == _lib.LM_EINVAL
    # tile height beyond 128, then an fp32 activation type
    assert lib.lm_routed_gemm_w8a16(None, 1, None, None, 256, 0, 0, None, None, 1, 200, None, 16,
                                    64, 128, 1, 0, None) == _lib.LM_EINVAL
    assert lib.lm_routed_gemm_w8a16(None, 1, None, None, 256, 0, 0, None, None, 1, 96, None, 16,
                                    64, 128, 1, 2, None) == _lib.LM_EINVAL
    assert b'FP16/BF16' in lib.lm_last_error()
    # contiguous rows need at least as many activation rows as output rows
    fake = ctypes.c_void_p(256)
    assert lib.lm_routed_gemm_w8a16(fake, 8, fake, fake, 256, 0, 0, None, fake, 1, 96, fake, 16,
                                    64, 128, 0, 0, None) == _lib.LM_EINVAL
    assert b'more output rows' in lib.lm_last_error()
    assert lib.lm_routed_gate_up_swiglu(fake, 8, fake, fake, 256, 0, 0, None, fake, 1, 96, fake,
                                        16, 64, 128, 0, None) == _lib.LM_EINVAL
    assert b'gather needs pos' in lib.lm_last_error()
    assert lib.lm_router_topk(None, None, None, None, None, None, 1, 512, 2048, 8,
                              None) == _lib.LM_EINVAL
    assert lib.lm_w8a8_linear(None, None, None, None, 9, 64, 128, 0, 0, None) == _lib.LM_EINVAL
    assert lib.lm_w8a8_linear(None, None, None, None, 1, 64, 128, 0, 2, None) == _lib.LM_EINVAL
    assert lib.lm_w8a8_gemm(None, None, None, None, None, 9, 64, 100, 0, 0, None) == _lib.LM_EINVAL
    assert b'Invalid INT8 group geometry' in lib.lm_last_error()
    assert lib.lm_w8a8_gemm(None, None, None, None, None, 9, 63, 128, 1, 0, None) == _lib.LM_EINVAL
    assert lib.lm_w8a8_gemm(None, None, None, None, None, 9, 64, 128, 0, 0, None) == _lib.LM_EINVAL
    assert b'null pointer' in lib.lm_last_error()
    assert lib.lm_w8a8_gemm(None, None, None, None, None, 9, 64, 128, 0, 2, None) == _lib.LM_EINVAL
    assert b'bf16 or fp16' in lib.lm_last_error()
    assert lib.lm_w8a8_gemm(None, None, None, None, None, 0, 64, 128, 0, 0, None) == _lib.LM_OK
    # a grid beyond one launch is refused before anything is launched (the
    # non-null placeholder pointers are never dereferenced)
    assert lib.lm_w8a8_gemm(fake, fake, fake, fake, fake, 1 << 24, 1 << 24, 128, 0, 0,
                            None) == _lib.LM_EINVAL
    assert b'too large' in lib.lm_last_error()
    assert lib.lm_swiglu(fake, fake, 4, 64, 2, None) == _lib.LM_EINVAL
    assert lib.lm_ordered_reduce(fake, fake, fake, 0, fake, 64, 8, 2, None) == _lib.LM_EINVAL
    assert lib.lm_routed_reduce(fake, fake, fake, fake, 3, fake, 4, 64, 8, 0,
                                None) == _lib.LM_EINVAL
    assert lib.lm_moe_workspace_init(fake, 258, None) == _lib.LM_EINVAL


def test_moe_layer_bounds_rejected_before_launch():
    """The fused layer accepts 1..65536 tokens of the 2048/512/256/top-8
    geometry, with a workspace sized for the token count; every refusal
    happens before a launch (the placeholder pointers are never used)."""
    lib = _lib.lib()
    fake = 256
    layer = _lib.MoeLayer(*([fake] * 8), 0, 0, 0, 0)
    ws = lib.lm_moe_workspace_bytes(65536, 2048, 512, 256, 8)
    assert ws > lib.lm_moe_workspace_bytes(2048, 2048, 512, 256, 8) > 0
    assert lib.lm_moe_workspace_bytes(0, 2048, 512, 256, 8) == -1
    assert lib.lm_moe_workspace_bytes(16, 4096, 512, 256, 8) == -1

    def fwd(tokens, ws_bytes, hidden=2048, lay=layer):
        return lib.lm_moe_layer_forward(ctypes.byref(lay), fake, tokens, hidden, 512, 256, 8,
                                        1e-6, fake, ws_bytes, None, None, None, None)

    assert fwd(0, ws) == _lib.LM_EINVAL
    assert b'invalid token count' in lib.lm_last_error()
    assert fwd(65537, 1 << 62) == _lib.LM_EINVAL
    assert fwd(16, ws, hidden=4096) == _lib.LM_EINVAL
    assert b'hidden 2048' in lib.lm_last_error()
    assert fwd(65536, ws - 1) == _lib.LM_ENOMEM
    assert fwd(2, lib.lm_moe_workspace_bytes(1, 2048, 512, 256, 8)) == _lib.LM_ENOMEM
    hole = _lib.MoeLayer(*([fake] * 5), None, fake, fake, 0, 0, 0, 0)
    assert fwd(16, ws, lay=hole) == _lib.LM_EINVAL
    assert b'null layer weight' in lib.lm_last_error()
    # a caller compiled against another layout of the struct is refused
    assert layer.struct_size == ctypes.sizeof(_lib.MoeLayer) == 16 * 8  # the ENOMEM above: C agrees
    older = _lib.MoeLayer(*([fake] * 8), 0, 0, 0, 0)
    older.struct_size = ctypes.sizeof(_lib.MoeLayer) - 8
    assert fwd(16, ws, lay=older) == _lib.LM_EINVAL
    assert b'struct_size' in lib.lm_last_error()
    bad_fmt = _lib.MoeLayer(*([fake] * 8), 0, 0, 0, 0, None, None, 7)
    assert fwd(16, ws, lay=bad_fmt) == _lib.LM_EINVAL
    assert b'gu_q_tiles_format' in lib.lm_last_error()


def test_chained_input_normed_refused_without_chain():
    """lm_moe_layer_forward_chain refuses input_normed = 1 unless the previous
    call on the same workspace chained into this layer (same tokens and eps),
    before any launch."""
    lib = _lib.lib()
    fake = 512
    layer = _lib.MoeLayer(*([fake] * 8), 0, 0, 0, 0)
    ws = lib.lm_moe_workspace_bytes(64, 2048, 512, 256, 8)
    rc = lib.lm_moe_layer_forward_chain(ctypes.byref(layer), None, 1, fake, 16, 2048, 512, 256, 8,
                                        1e-6, fake + 4096, ws, None, None, None, None)
    assert rc == _lib.LM_EINVAL
    assert b'input_normed' in lib.lm_last_error()


def test_workspace_regions():
    """Every region lies inside the workspace of its token count; the
    decode-only regions (W8A8 intermediates of the one-token path) and the
    prefill-only ones (route rows, approximate router logits and their
    norms) are refused for the other kind of call."""
    lib = _lib.lib()
    off, nb = ctypes.c_int64(), ctypes.c_int64()
    for tokens in (1, 2, 37, 2048):
        total = lib.lm_moe_workspace_bytes(tokens, 2048, 512, 256, 8)
        spans = []
        for name, code in _lib.WS_REGIONS.items():
            rc = lib.lm_moe_workspace_region(tokens, code, ctypes.byref(off), ctypes.byref(nb))
            decode_only = 7 <= code <= 12
            prefill_only = name == 'route_rows' or code >= 13
            if (tokens == 1 and prefill_only) or (tokens > 1 and decode_only):
                assert rc == _lib.LM_EINVAL, (tokens, name)
                continue
            assert rc == _lib.LM_OK, (tokens, name)
            assert off.value % 256 == 0 and off.value + nb.value <= total, (tokens, name)
            spans.append((off.value, off.value + nb.value))
        spans.sort()
        assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:])), tokens  # disjoint
    sizes = {}
    for name in ('hidden', 'down', 'act_q', 'act_scales', 'slot_ids', 'slot_weights',
                 'gate_up_acc', 'down_acc'):
        assert lib.lm_moe_workspace_region(1, _lib.WS_REGIONS[name], ctypes.byref(off),
                                           ctypes.byref(nb)) == _lib.LM_OK
        sizes[name] = nb.value
    assert sizes == {'hidden': 9 * 512 * 2, 'down': 9 * 2048 * 2, 'act_q': 2048,
                     'act_scales': 16 * 4, 'slot_ids': 32, 'slot_weights': 32,
                     'gate_up_acc': 8 * 1024 * 4, 'down_acc': 8 * 2048 * 4}
    for name, size in (('router_approx', 37 * 256 * 4), ('row_norms', 37 * 4),
                       ('router_norms', 256 * 4)):
        assert lib.lm_moe_workspace_region(37, _lib.WS_REGIONS[name], ctypes.byref(off),
                                           ctypes.byref(nb)) == _lib.LM_OK
        assert nb.value == size, name
    assert lib.lm_moe_workspace_region(2, 16, ctypes.byref(off), ctypes.byref(nb)) == _lib.LM_EINVAL


def test_status_maps_to_reference_exceptions():
    with pytest.raises(ValueError, match='Invalid INT8 group geometry'):
        _lib.call('lm_w8a16_linear', None, None, None, None, 1, 8, 100, 0, 0, None)


def test_python_wrappers_validate_like_reference():
    x = torch.zeros(2, 256, dtype=torch.bfloat16)
    q = torch.zeros(64, 256, dtype=torch.int8)
    s = torch.zeros(64, 2)
    with pytest.raises(ValueError, match='W8A16 requires CUDA FP16/BF16 activations'):
        int8.linear(x, q, s)
    with pytest.raises(ValueError, match='Expected CUDA rows with K divisible by 128'):
        w8a8.quantize(x)
    with pytest.raises(ValueError, match='Expected CUDA int8 rows and weights'):
        w8a8.gemm(q[:2], s[:2], q, s)
    with pytest.raises(ValueError, match='Expected contiguous CUDA'):
        gpu_routes.plan(torch.zeros(2, 8, dtype=torch.int64), 256, 16)
    with pytest.raises(ValueError, match='Expected nonempty CPU'):
        routing.plan_routes(torch.zeros(0, 8, dtype=torch.int64), 256)
    with pytest.raises(ValueError, match='Out-of-range expert ID'):
        routing.plan_routes(torch.tensor([[0, 256]]), 256)
    with pytest.raises(ValueError, match='Out-of-range expert ID'):
        routing.plan_routes(torch.tensor([[-1, 3]]), 256)


@pytest.mark.parametrize('t,k,e', [(1, 8, 256), (13, 8, 256), (2048, 8, 256), (5, 3, 7)])
def test_host_plan_routes_matches_oracle(t, k, e):
    rng = np.random.default_rng(t + e)
    ids = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int64)
    positions, segments = routing.plan_routes(torch.from_numpy(ids), e)
    ref_pos, ref_seg = O.plan_routes(ids, e)
    assert np.array_equal(positions.numpy(), ref_pos)
    assert segments == ref_seg


@pytest.mark.parametrize('t,k,e,bm', [(1, 8, 256, 96), (13, 8, 256, 16), (2048, 8, 256, 96),
                                      (5, 3, 7, 2), (300, 8, 256, 128)])
def test_host_tile_plan_matches_oracle(t, k, e, bm):
    """The native host planner (lm_route_plan_host) behind runtime/prefill.py
    gives the oracle's pos / ordered / slots bit for bit and its tile table
    without the surplus rows."""
    rng = np.random.default_rng(7 * t + e)
    ids = np.stack([rng.choice(e, size=k, replace=False) for _ in range(t)]).astype(np.int64)
    if t == 300:  # skewed: most routes on a few experts, most experts empty
        ids = np.stack([rng.choice(12, size=k, replace=False) * 3 for _ in range(t)])
    pos, table, ordered, slots, active = routing.tile_plan(torch.from_numpy(ids), e, bm)
    rpos, rtable, rordered, rslots = O.plan(ids, e, bm)
    assert np.array_equal(pos.numpy(), rpos)
    assert np.array_equal(ordered.numpy(), rordered)
    assert np.array_equal(slots.numpy(), rslots)
    n = table.shape[0]
    assert np.array_equal(table.numpy(), rtable[:n])
    assert not rtable[n:].any()  # the oracle's remaining rows are surplus (0, 0, 0)
    assert active == len(np.unique(ids))


def test_host_tile_plan_duplicate_ids_and_errors():
    ids = torch.tensor([[3, 3, 1], [0, 3, 3]])  # duplicates inside a token: stable order
    pos, table, ordered, slots, _ = routing.tile_plan(ids, 4, 2)
    rpos, rtable, rordered, rslots = O.plan(ids.numpy(), 4, 2)
    assert np.array_equal(slots.numpy(), rslots) and np.array_equal(ordered.numpy(), rordered)
    assert np.array_equal(pos.numpy(), rpos)
    with pytest.raises(ValueError, match='Out-of-range expert ID'):
        routing.tile_plan(torch.tensor([[0, 4]]), 4, 2)
    with pytest.raises(ValueError, match='Expected nonempty CPU'):
        routing.tile_plan(torch.zeros(0, 2, dtype=torch.int64), 4, 2)
