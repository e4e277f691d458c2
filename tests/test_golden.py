"""The committed golden fixtures (tests/golden/golden_small.npz) against the
CPU oracle and the reference's own known-answer test.

The fixtures are the oracle's outputs on seeded inputs, written by
tests/golden/make_golden.py; the GPU tests compare the HIP path with them.
Here, on the CPU: the quantizer fixture equals the reference's closed-form
known answer (tests/test_release.py:20-26), and the oracle still reproduces
every stored output bit for bit (the float GEMM output, computed by torch's
CPU matmul, within the bf16 tolerance).
"""
import pathlib

import numpy as np
import torch

from tests.conftest import BF16_TOL, assert_close
from tests.golden import make_golden

FIXTURES = pathlib.Path(__file__).resolve().parent / 'golden' / 'golden_small.npz'


def load():
    return np.load(FIXTURES, allow_pickle=False)


def test_fixture_matches_reference_known_answer():
    d = load()
    weight = torch.linspace(-1, 1, 256).reshape(2, 128).bfloat16()
    ref_scale = weight.float().abs().amax(-1, keepdim=True) / 127
    ref = (weight.float() / ref_scale).round().clamp(-127, 127).to(torch.int8)
    assert np.array_equal(d['kat_q'], ref.numpy())
    assert np.array_equal(d['kat_s'], ref_scale.numpy())


def test_oracle_reproduces_fixtures():
    d = load()
    fresh = make_golden.build()
    assert sorted(fresh) == sorted(d.files)
    for name in d.files:
        if name == 'w8a16_y':
            assert_close(make_golden.from_bits(fresh[name]), make_golden.from_bits(d[name]),
                         BF16_TOL, name)
        else:
            assert fresh[name].dtype == d[name].dtype, name
            assert np.array_equal(fresh[name], d[name]), name


def test_fixture_invariants():
    """Properties the fixtures must have whatever produced them."""
    d = load()
    # quantizer: |q| <= 127 and q * s reconstructs w to half a step
    q, s, w = d['quant_q'], d['quant_s'], d['quant_w']
    assert np.abs(q.astype(np.int32)).max() <= 127
    rec = q.reshape(64, 4, 128).astype(np.float64) * s[..., None]
    assert np.all(np.abs(rec - w.reshape(64, 4, 128)) <= 0.5 * s[..., None] * (1 + 1e-6))
    assert np.all(q[3, 128:256] == 0)
    # partials are exact integer dots
    xq, _ = make_golden.O.act_quant(make_golden.from_bits(d['w8a8_x']))
    p = np.einsum('mgk,ngk->mng', xq.reshape(4, 4, 128).astype(np.int64),
                  d['w8a8_q'].reshape(96, 4, 128).astype(np.int64))
    assert np.array_equal(p, d['w8a8_p'])
    # router: ties resolved to the lower id, ids distinct per token
    ids = d['router_ids']
    for row in ids.tolist():  # experts 3 and 17 tie: both chosen, the lower id first
        assert 3 in row and row.index(17) == row.index(3) + 1
    assert all(len(set(r)) == 8 for r in ids)
    # plan: pos lists each token top_k times, expert 11 is empty
    assert np.array_equal(np.bincount(d['plan_pos'], minlength=37), np.full(37, 8))
    assert 11 not in d['plan_routes_segments'][:, 0]


def test_host_plan_routes_matches_fixture():
    """The library's host plan (routing.plan_routes) against the fixture."""
    from localmoe35ba3b_amd.operators import routing
    d = load()
    positions, segments = routing.plan_routes(torch.from_numpy(d['plan_ids']), 40)
    assert np.array_equal(positions.numpy(), d['plan_routes_positions'])
    assert np.array_equal(np.asarray(segments, np.int64), d['plan_routes_segments'])
