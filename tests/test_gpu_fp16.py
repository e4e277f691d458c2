"""GPU parity of the fp16-activation paths against the oracle's fp16 variants.

The reference allocates every output in x.dtype, so an fp16 model runs the
same operators with fp16 rounding in place of bf16: the routed grouped GEMMs
and their combine (prefill.py:70-84, gpu_routes.py:70-81), the W8A8 decode
GEMV (w8a8.py:46) and the grouped W8A16 decode with its combine
(int8.py:228-250).  W8A8 outputs are compared bit for bit (exact int32
partials and the restated epilogue); everything through an fp32-accumulated
GEMM within the tolerance of tests/conftest.py.
"""
import numpy as np
import pytest
import torch

from localmoe35ba3b_amd.operators import int8, w8a8
from localmoe35ba3b_amd.runtime import gpu_routes, prefill
from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close, seeded
from tests.test_gpu_ops import _bank, _ids, _table

pytestmark = pytest.mark.gpu


def f16_rand(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.float16)


def npf(t):
    return t.detach().float().cpu().numpy()


@pytest.mark.parametrize('large', [False, True])
def test_routed_moe_fp16(dev, large):
    gen = seeded(70)
    e, t, k = 24, 96, 8
    gq, gs = _bank(gen, e, 1024, 2048)
    dq, ds = _bank(gen, e, 2048, 512)
    banks = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    x = f16_rand((t, 2048), gen)
    ids = _ids(seeded(71), t, e, k, True)
    wts = torch.softmax(torch.randn(t, k, generator=gen), -1).to(torch.float16)
    out = gpu_routes.routed_moe(x.to(dev), wts.to(dev), ids.to(dev), banks, large)
    assert out.dtype == torch.float16
    xn, idn, wn = npf(x), ids.numpy(), npf(wts)
    ref = np.zeros_like(xn)
    for ex in np.unique(idn):
        token, slot = np.nonzero(idn == ex)
        y = O.expert_w8a16(xn[token], gq[ex], gs[ex], dq[ex], ds[ex], O.fp16)
        ref[token] = O.fp16(ref[token] + O.fp16(y * wn[token, slot][:, None]))
    assert_close(npf(out), ref, BF16_TOL, 'routed_moe fp16')
    stats = {}
    out_host = prefill.routed_moe(x.to(dev), wts.to(dev), ids.to(dev), banks, large, stats=stats)
    assert torch.equal(out_host, out)
    assert stats == dict(active_experts=len(np.unique(idn)), total_experts=e,
                         routed_tokens=t * k, tokens=t)


def test_w8a8_fp16_bit_exact(dev):
    gen = seeded(72)
    gq, gs = _bank(gen, 12, 1024, 2048)
    dq, ds = _bank(gen, 12, 2048, 512)
    tg = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    ids = [9, 2, 11, 0, 5, 7, 3, 10]
    table, order = _table(dev, *tg, ids)
    x = f16_rand((1, 2048), gen)
    gu = w8a8.grouped_linear(x.to(dev), table, 8, 1024, 0, True)
    assert gu.dtype == torch.float16
    ref = np.stack([O.w8a8_linear(npf(x), gq[e], gs[e], O.fp16)[0] for e in order])
    assert np.array_equal(npf(gu), ref)
    h = f16_rand((8, 512), gen, 0.5)
    dn = w8a8.grouped_linear(h.to(dev), table, 8, 2048, 2, False)
    ref_dn = np.stack([O.w8a8_linear(npf(h)[i:i + 1], dq[e], ds[e], O.fp16)[0]
                       for i, e in enumerate(order)])
    assert np.array_equal(npf(dn), ref_dn)
    for m in (1, 4, 8, 37):  # dense rows: fused GEMV up to 8 rows, int8 MFMA GEMM beyond
        xm = f16_rand((m, 2048), gen)
        y = w8a8.linear(xm.to(dev), tg[0][3], tg[1][3])
        assert y.dtype == torch.float16
        full = O.w8a8_linear(npf(xm), gq[3], gs[3], O.fp16)
        assert np.array_equal(npf(y), full)  # epilogue restated exactly
        h = w8a8.linear(xm.to(dev), tg[0][3], tg[1][3], swiglu=True)
        href = O.swiglu(full, O.fp16)
        assert_close(npf(h), href, BF16_TOL, f'w8a8 fp16 swiglu m={m}')
        assert (npf(h) == href).mean() > 0.99  # silu's exp may differ by an ulp


def test_int8_experts_decode_fp16(dev):
    gen = seeded(73)
    gq, gs = _bank(gen, 10, 1024, 2048)
    dq, ds = _bank(gen, 10, 2048, 512)
    tg = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    ids = [4, 9, 1, 0, 7, 2, 8, 3]
    _, order = _table(dev, *tg, ids)
    x = f16_rand((1, 2048), gen)
    experts = int8.Int8Experts(0, {'q': tg[0], 'scale': tg[1]}, {'q': tg[2], 'scale': tg[3]})
    wts = torch.rand(1, 8, generator=gen).to(torch.float16)
    top = torch.tensor([ids], dtype=torch.int64)
    out = experts(x.to(dev), top.to(dev), wts.to(dev))
    assert out.dtype == torch.float16
    vals = np.stack([O.expert_w8a16(npf(x), gq[e], gs[e], dq[e], ds[e], O.fp16)[0]
                     for e in order])
    wsorted = [npf(wts)[0, ids.index(e)] for e in order]
    assert_close(npf(out)[0], O.ordered_combine(vals, wsorted, O.fp16), BF16_TOL,
                 'Int8Experts fp16')
    v = f16_rand((8, 2048), gen)
    table = torch.zeros(8, 5, dtype=torch.int64)
    table[:, 4] = torch.tensor([3, 0, 7, 1, 6, 2, 5, 4])
    y = int8.ordered_reduce(v.to(dev), table.to(dev), wts.to(dev))
    ref = O.ordered_combine(npf(v), [npf(wts)[0, s] for s in table[:, 4].tolist()], O.fp16)
    assert np.array_equal(npf(y)[0], ref)
    gu = f16_rand((37, 1024), gen, 3.0)
    hs = int8.swiglu(gu.to(dev))
    assert hs.dtype == torch.float16
    assert_close(npf(hs), O.swiglu(npf(gu), O.fp16), BF16_TOL, 'swiglu fp16')
