"""Writes tests/golden/golden_small.npz: seeded inputs and the CPU oracle's
outputs for every operator of the quantized MoE-FFN path, at sizes small
enough to commit (~0.5 MB).

    python tests/golden/make_golden.py

bf16 tensors are stored as their uint16 bit patterns, so every value is
kept exactly.  The reference ships only one known-answer test for this path
(tests/test_release.py:20-26, the weight quantizer); it is stored here as
`kat_*` next to the oracle-generated vectors.  tests/test_golden.py checks
that the oracle still reproduces this file; tests/test_gpu_golden.py checks
the HIP path against it.
"""
import pathlib
import sys

import numpy as np
import torch

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

from oracle import moe_oracle as O  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / 'golden_small.npz'


def bf16_bits(a):
    """float32 array holding bf16 values -> uint16 bit patterns."""
    a = np.ascontiguousarray(O.bf16(a), dtype=np.float32)
    return (a.view(np.uint32) >> 16).astype(np.uint16)


def from_bits(b):
    return (np.asarray(b, np.uint32) << 16).view(np.float32)


def randn(gen, shape, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).numpy().astype(np.float32)


def build():
    g = torch.Generator()
    f = {}
    # a1 quantizer: the reference's known answer, then a random bank with a
    # zero group and a large-magnitude group.
    kat = torch.linspace(-1, 1, 256).reshape(2, 128).bfloat16().float().numpy()
    f['kat_w'] = kat
    f['kat_q'], f['kat_s'] = O.quantize_weight(kat)
    g.manual_seed(0)
    w = randn(g, (64, 512), 0.02)
    w[3, 128:256] = 0.0
    w[5, :128] *= 1e4
    f['quant_w'] = w
    f['quant_q'], f['quant_s'] = O.quantize_weight(w)
    # a4 activation quantization (one all-zero group)
    g.manual_seed(1)
    x = O.bf16(randn(g, (4, 512)))
    x[1, 128:256] = 0.0
    f['act_x'] = bf16_bits(x)
    f['act_q'], f['act_s'] = O.act_quant(x)
    # a5 W8A8 linear: int32 partials and the fp32 epilogue, bf16 out
    g.manual_seed(2)
    x = O.bf16(randn(g, (4, 512)))
    wq, ws = O.quantize_weight(randn(g, (96, 512), 0.02))
    xq, xs = O.act_quant(x)
    f['w8a8_x'], f['w8a8_q'], f['w8a8_s'] = bf16_bits(x), wq, ws
    f['w8a8_p'] = O.w8a8_partials(xq, wq)
    f['w8a8_y'] = bf16_bits(O.w8a8_linear(x, wq, ws))
    # a2 W8A16 linear (fp32 accumulation, bf16 out)
    g.manual_seed(3)
    x = O.bf16(randn(g, (4, 512)))
    q, s = O.quantize_weight(randn(g, (128, 512), 0.02))
    f['w8a16_x'], f['w8a16_q'], f['w8a16_s'] = bf16_bits(x), q, s
    f['w8a16_y'] = bf16_bits(O.w8a16_linear(x, q, s))
    # a11 SwiGLU
    g.manual_seed(4)
    gu = O.bf16(randn(g, (6, 1024), 3.0))
    f['swiglu_gu'] = bf16_bits(gu)
    f['swiglu_h'] = bf16_bits(O.swiglu(gu))
    # a6 ordered combine: 8 expert rows in ascending expert order
    g.manual_seed(5)
    v = O.bf16(randn(g, (8, 2048)))
    wts = O.bf16(torch.rand(8, generator=g).numpy().astype(np.float32))
    f['combine_v'], f['combine_w'] = bf16_bits(v), bf16_bits(wts)
    f['combine_y'] = bf16_bits(O.ordered_combine(v, wts))
    # a8 router: 24 tokens, 256 experts, hidden 256, with a tie pair
    g.manual_seed(6)
    x = O.bf16(randn(g, (24, 256)))
    rw = O.bf16(randn(g, (256, 256), 0.02))
    rw[17] = rw[3]  # experts 3 and 17 tie for every token: the lower id comes first
    bias = np.zeros(256, np.float32)
    bias[200:] = np.float32(0.5)
    bias[[3, 17]] = np.float32(2.0)  # ... and both are always selected
    lg, rwts, ids = O.router(x, rw, 8, bias)
    f['router_x'], f['router_w'], f['router_bias'] = bf16_bits(x), bf16_bits(rw), bias
    f['router_logits'], f['router_weights'], f['router_ids'] = lg, bf16_bits(rwts), ids
    # a9 route plan: ragged ids with empty experts, bm = 16
    rng = np.random.default_rng(7)
    live = np.array([e for e in range(40) if e != 11])  # expert 11 stays empty
    pids = np.stack([rng.choice(live, 8, replace=False) for _ in range(37)]).astype(np.int64)
    f['plan_ids'] = pids
    f['plan_pos'], f['plan_table'], f['plan_ordered'], f['plan_slots'] = O.plan(pids, 40, 16)
    f['plan_routes_positions'], segs = O.plan_routes(pids, 40)
    f['plan_routes_segments'] = np.asarray(segs, np.int64)
    # a14 RMSNorm with a weight vector (the fixed reduction tree)
    g.manual_seed(8)
    x = O.bf16(randn(g, (5, 2048)))
    nw = randn(g, (2048,), 0.1)
    f['rms_x'], f['rms_w'] = bf16_bits(x), nw
    f['rms_y'] = bf16_bits(O.rmsnorm(x, nw))
    return f


if __name__ == '__main__':
    fixtures = build()
    np.savez_compressed(OUT, **fixtures)
    print(f'wrote {OUT} ({OUT.stat().st_size} bytes, {len(fixtures)} arrays)')
