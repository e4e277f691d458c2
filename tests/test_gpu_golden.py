"""The HIP path against the committed golden fixtures (oracle outputs on
seeded inputs, tests/golden/golden_small.npz), through the public operators.

Bit-exact: quantizers, int32 partials, W8A8 outputs, combine, RMSNorm, router
ids and logits, route plans.  Within the bf16 tolerance of tests/conftest.py:
the fp32-accumulated W8A16 GEMM, SwiGLU; router weights within 2^-8.
"""
import pathlib

import numpy as np
import pytest
import torch

from localmoe35ba3b_amd import convert, router
from localmoe35ba3b_amd.operators import int8, routing, w8a8
from localmoe35ba3b_amd.runtime import gpu_routes
from tests.conftest import BF16_TOL, assert_close

pytestmark = pytest.mark.gpu

FIXTURES = pathlib.Path(__file__).resolve().parent / 'golden' / 'golden_small.npz'


@pytest.fixture(scope='module')
def gold():
    return np.load(FIXTURES, allow_pickle=False)


def bf16_dev(bits, dev):
    """uint16 bf16 bit patterns -> CUDA bf16 tensor."""
    return torch.from_numpy(np.asarray(bits, np.uint16).view(np.int16).copy()).view(
        torch.bfloat16).to(dev)


def bits(t):
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def f32(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def test_quantizer(gold, dev):
    for w, q, s in (('kat_w', 'kat_q', 'kat_s'), ('quant_w', 'quant_q', 'quant_s')):
        gq, gs = convert.quantize_g128(torch.from_numpy(gold[w]).to(dev))
        assert np.array_equal(gq.cpu().numpy(), gold[q]), w
        assert np.array_equal(gs.cpu().numpy().reshape(gold[s].shape), gold[s]), w


def test_act_quant(gold, dev):
    q, s = w8a8.quantize(bf16_dev(gold['act_x'], dev))
    assert np.array_equal(q.cpu().numpy(), gold['act_q'])
    assert np.array_equal(s.cpu().numpy(), gold['act_s'])


def test_w8a8_partials_and_linear(gold, dev):
    x = bf16_dev(gold['w8a8_x'], dev)
    q = torch.from_numpy(gold['w8a8_q']).to(dev)
    s = torch.from_numpy(gold['w8a8_s']).to(dev)
    xq, _ = w8a8.quantize(x)
    assert np.array_equal(w8a8.group_partials(xq, q).cpu().numpy(), gold['w8a8_p'])
    assert np.array_equal(bits(w8a8.linear(x, q, s)), gold['w8a8_y'])


def test_w8a16_linear(gold, dev):
    y = int8.linear(bf16_dev(gold['w8a16_x'], dev), torch.from_numpy(gold['w8a16_q']).to(dev),
                    torch.from_numpy(gold['w8a16_s']).to(dev))
    assert_close(f32(bits(y)), f32(gold['w8a16_y']), BF16_TOL, 'w8a16 linear')


def test_swiglu(gold, dev):
    h = int8.swiglu(bf16_dev(gold['swiglu_gu'], dev))
    assert_close(f32(bits(h)), f32(gold['swiglu_h']), BF16_TOL, 'swiglu')
    assert (bits(h) == gold['swiglu_h']).mean() > 0.99


def test_ordered_combine(gold, dev):
    table = torch.zeros(8, 5, dtype=torch.int64)
    table[:, 4] = torch.arange(8)
    w = bf16_dev(gold['combine_w'], dev).reshape(1, 8)
    y = int8.ordered_reduce(bf16_dev(gold['combine_v'], dev), table.to(dev), w)
    assert np.array_equal(bits(y)[0], gold['combine_y'])


def test_router(gold, dev):
    lg, wts, ids = router.router_topk(bf16_dev(gold['router_x'], dev),
                                      bf16_dev(gold['router_w'], dev), 8,
                                      torch.from_numpy(gold['router_bias']))
    assert np.array_equal(ids.cpu().numpy(), gold['router_ids'])
    assert np.array_equal(lg.cpu().numpy(), gold['router_logits'])
    assert np.abs(f32(bits(wts)) - f32(gold['router_weights'])).max() <= 2.0 ** -8


def test_route_plan(gold, dev):
    ids = torch.from_numpy(gold['plan_ids'])
    pos, table, ordered, slots = gpu_routes.plan(ids.to(dev), 40, 16)
    assert np.array_equal(pos.cpu().numpy(), gold['plan_pos'])
    assert np.array_equal(table.cpu().numpy(), gold['plan_table'])
    assert np.array_equal(ordered.cpu().numpy(), gold['plan_ordered'])
    assert np.array_equal(slots.cpu().numpy(), gold['plan_slots'])
    positions, segments = routing.plan_routes(ids, 40)
    assert np.array_equal(np.asarray(positions), gold['plan_routes_positions'])
    assert np.array_equal(np.asarray(segments, np.int64), gold['plan_routes_segments'])


def test_rmsnorm(gold, dev):
    y = router.rmsnorm(bf16_dev(gold['rms_x'], dev), torch.from_numpy(gold['rms_w']))
    assert np.array_equal(bits(y), gold['rms_y'])
