"""GPU parity of every operator against the CPU oracle on identical seeded inputs.

Bit-exact: weight quantizer, activation quantizer, W8A8 int32 partials and
W8A8 outputs (the fp32 epilogue is restated exactly), dequantized weights
(checked through exactly-representable GEMMs), combines, route plans, router
ids and logits.  Tolerance (tests/conftest.py): bf16 outputs of fp32-accumulated
GEMMs and anything downstream of exp (SwiGLU, softmax weights).
"""
import numpy as np
import pytest
import torch

from localmoe35ba3b_amd import convert, router
from localmoe35ba3b_amd.operators import int8, routing, w8a8
from localmoe35ba3b_amd.runtime import gpu_routes, prefill
from localmoe35ba3b_amd.runtime.stack import zipf_bias
from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close, seeded

pytestmark = pytest.mark.gpu


def bf16_rand(shape, gen, scale=1.0):
    return (torch.randn(shape, generator=gen) * scale).to(torch.bfloat16)


def npf(t):
    return t.detach().float().cpu().numpy()


# ------------------------------------------------------------- a1 quantizer
def test_quantizer_reference_known_answer(dev):
    weight = torch.linspace(-1, 1, 256).reshape(2, 128).bfloat16()
    q, s = convert.quantize_g128(weight.to(dev))
    ref_scale = weight.float().abs().amax(-1, keepdim=True) / 127
    ref = (weight.float() / ref_scale).round().clamp(-127, 127).to(torch.int8)
    assert torch.equal(q.cpu(), ref)
    assert torch.equal(s.cpu(), ref_scale)
    qc, sc, err, energy = convert.quantize(weight.to(dev))
    assert torch.equal(qc, ref) and err >= 0 and energy > 0


def test_quantizer_random_bit_exact(dev):
    w = torch.randn(300, 1024, generator=seeded(0)) * 0.02
    w[5, 128:256] = 0.0
    w[7, :128] *= 1e4
    q, s = convert.quantize_g128(w.to(dev))
    rq, rs = O.quantize_weight(w.numpy())
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


# ------------------------------------------------------------- a4 act quant
def test_act_quant_bit_exact(dev):
    x = bf16_rand((9, 2048), seeded(1))
    x[2, :128] = 0
    x[3, 128:256] *= 1000
    x[4, 256:384] = torch.tensor(np.linspace(-3, 3, 128), dtype=torch.bfloat16)
    q, s = w8a8.quantize(x.to(dev))
    rq, rs = O.act_quant(npf(x))
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(s.cpu().numpy(), rs)


# ------------------------------------------------------------- a5 W8A8
@pytest.mark.parametrize('m', [1, 4, 5, 8])
@pytest.mark.parametrize('n,k', [(1024, 2048), (1000, 384), (2048, 512), (1000, 2048)])
def test_w8a8_partials_bit_exact(dev, m, n, k):
    g = np.random.default_rng(m * 7 + n + k)
    xq = g.integers(-127, 128, size=(m, k)).astype(np.int8)
    wq = g.integers(-127, 128, size=(n, k)).astype(np.int8)
    xq[0, :128] = -127
    wq[0, :128] = -127  # extreme group: 128 * 127^2
    p = w8a8.group_partials(torch.from_numpy(xq).to(dev), torch.from_numpy(wq).to(dev))
    assert np.array_equal(p.cpu().numpy(), O.w8a8_partials(xq, wq))


@pytest.mark.parametrize('m', [1, 4, 5, 8])
def test_w8a8_linear_gate_up(dev, m):
    """The W8A8 decode linear: x bf16 [M, 2048], fused gate_up [1024, 2048]."""
    gen = seeded(2)
    x = bf16_rand((m, 2048), gen)
    wq, ws = O.quantize_weight((torch.randn(1024, 2048, generator=gen) * 0.02).numpy())
    xd, qd, sd = x.to(dev), torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev)
    y = w8a8.linear(xd, qd, sd)
    ref = O.w8a8_linear(npf(x), wq, ws)
    assert np.array_equal(npf(y), ref)  # epilogue restated exactly -> bit-exact bf16
    h = w8a8.linear(xd, qd, sd, swiglu=True)
    href = O.swiglu(ref)
    assert_close(npf(h), href, BF16_TOL, 'w8a8 swiglu')
    assert (npf(h) == href).mean() > 0.99


@pytest.mark.parametrize('m,n,rows', [(9, 1024, None), (130, 1024, None), (300, 200, None),
                                      (2048, 4096, 40)])
def test_w8a8_gemm_bit_exact(dev, m, n, rows):
    """The int8 MFMA W8A8 GEMM (more than 8 rows, through w8a8.linear): every
    row equals the oracle's w8a8._linear restatement bit for bit, with ragged
    row tiles (9, 130, 300 rows), ragged column tiles (200 columns) and the
    fused SwiGLU.  At 2048 x 4096 a seeded sample of `rows` rows is checked
    (rows are computed independently)."""
    gen = seeded(31)
    x = bf16_rand((m, 2048), gen)
    wq, ws = O.quantize_weight((torch.randn(n, 2048, generator=gen) * 0.02).numpy())
    xd, qd, sd = x.to(dev), torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev)
    sel = np.arange(m) if rows is None else np.sort(
        np.random.default_rng(5).choice(m, rows, replace=False))
    y = w8a8.linear(xd, qd, sd)
    ref = O.w8a8_linear(npf(x)[sel], wq, ws)
    assert np.array_equal(npf(y)[sel], ref)
    h = w8a8.linear(xd, qd, sd, swiglu=True)
    href = O.swiglu(ref)
    assert_close(npf(h)[sel], href, BF16_TOL, 'w8a8 gemm swiglu')
    assert (npf(h)[sel] == href).mean() > 0.99
    # the GEMM on rows quantized by quantize() is the same call without the wrapper
    xq, xs = w8a8.quantize(xd)
    assert torch.equal(w8a8.gemm(xq, xs, qd, sd), y)


def _bank(gen, e, n, k, scale=0.02):
    w = torch.randn(e, n, k, generator=gen) * scale
    q, s = O.quantize_weight(w.numpy())
    return q, s


def _table(dev, qg, sg, qd, sd, ids):
    order = sorted((int(e), slot) for slot, e in enumerate(ids))
    rows = []
    for e, slot in order:
        rows.append([qg[e].data_ptr(), sg[e].data_ptr(), qd[e].data_ptr(), sd[e].data_ptr(), slot])
    return torch.tensor(rows, dtype=torch.int64, device=dev), [e for e, _ in order]


def test_w8a8_grouped_decode_bit_exact(dev):
    gen = seeded(3)
    gq, gs = _bank(gen, 12, 1024, 2048)
    dq, ds = _bank(gen, 12, 2048, 512)
    tg = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    ids = [9, 2, 11, 0, 5, 7, 3, 10]
    table, order = _table(dev, *tg, ids)
    x = bf16_rand((1, 2048), gen)
    gu = w8a8.grouped_linear(x.to(dev), table, 8, 1024, 0, True)
    ref_gu = np.stack([O.w8a8_linear(npf(x), gq[e], gs[e])[0] for e in order])
    assert np.array_equal(npf(gu), ref_gu)
    h = bf16_rand((8, 512), gen)
    dn = w8a8.grouped_linear(h.to(dev), table, 8, 2048, 2, False)
    ref_dn = np.stack([O.w8a8_linear(npf(h)[i:i + 1], dq[e], ds[e])[0] for i, e in enumerate(order)])
    assert np.array_equal(npf(dn), ref_dn)
    q, s = w8a8.quantize(h.to(dev))
    dn2 = w8a8.grouped_gemv(q, s, table, 8, 2048, 2, False)
    assert torch.equal(dn2, dn)


# ------------------------------------------------------------- a2 W8A16
@pytest.mark.parametrize('m,n,k', [(1, 4096, 2048), (2048, 4096, 2048), (3, 1000, 384),
                                   (37, 1000, 384), (8, 512, 2048), (130, 2048, 512),
                                   (1057, 4096, 2048), (1100, 1000, 512), (3000, 3000, 2048),
                                   (4096, 2048, 512)])
def test_w8a16_linear(dev, m, n, k):
    """Every GEMM path of int8.linear against the oracle: the GEMV (m <= 8),
    96-row tiles, 128-row tiles from m = 1024 (1057 and 1100 end in partial
    tiles of 33 and 76 rows), the wide 8-wave 256-column tiles where they give
    every CU a tile (2048 x 4096, 3000 x 3000 with a partial row tile of 56
    rows and a partial column tile of 184 columns, and K = 512), the generic
    kernel at K = 384."""
    gen = seeded(m + n)
    x = bf16_rand((m, k), gen)
    wq, ws = O.quantize_weight((torch.randn(n, k, generator=gen) * 0.02).numpy())
    y = int8.linear(x.to(dev), torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev))
    assert_close(npf(y), O.w8a16_linear(npf(x), wq, ws), BF16_TOL, f'w8a16 {m}x{n}x{k}')


@pytest.mark.parametrize('m,n', [(1, 384), (5, 384), (300, 384), (1030, 384), (4000, 2048)])
def test_w8a16_linear_exact(dev, m, n):
    """Integer activations and power-of-two scales make every product and sum
    exact in fp32, so any MFMA/GEMV layout or dequant error shows bit for bit
    (4000 x 2048 runs the wide 8-wave tiles, ending in a 32-row tile)."""
    g = np.random.default_rng(m)
    x = g.integers(-8, 9, size=(m, 512)).astype(np.float32)
    q = g.integers(-127, 128, size=(n, 512)).astype(np.int8)
    s = np.full((n, 4), 2.0 ** -6, np.float32)
    s[::3] = 2.0 ** -5
    y = int8.linear(torch.from_numpy(x).to(torch.bfloat16).to(dev), torch.from_numpy(q).to(dev),
                    torch.from_numpy(s).to(dev))
    exact = x.astype(np.float64) @ O.dequant(q, s, lambda a: a).astype(np.float64).T
    assert np.array_equal(npf(y), O.bf16(exact.astype(np.float32)))


@pytest.mark.parametrize('m', [64, 1030])
def test_w8a16_linear_fp16(dev, m):
    gen = seeded(5)
    x = (torch.randn(m, 512, generator=gen)).to(torch.float16)
    wq, ws = O.quantize_weight((torch.randn(256, 512, generator=gen) * 0.02).numpy())
    y = int8.linear(x.to(dev), torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev))
    wd = O.dequant(wq, ws, lambda a: a.astype(np.float16).astype(np.float32))
    ref = x.float().numpy().astype(np.float64) @ wd.astype(np.float64).T
    assert_close(y.float().cpu().numpy(), ref, BF16_TOL, 'w8a16 fp16')
    y1 = int8.linear(x[:1].to(dev), torch.from_numpy(wq).to(dev), torch.from_numpy(ws).to(dev))
    assert_close(y1.float().cpu().numpy(), ref[:1], BF16_TOL, 'w8a16 fp16 gemv')


def test_w8a16_grouped_and_experts_decode(dev):
    gen = seeded(6)
    gq, gs = _bank(gen, 10, 1024, 2048)
    dq, ds = _bank(gen, 10, 2048, 512)
    tg = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    ids = [4, 9, 1, 0, 7, 2, 8, 3]
    table, order = _table(dev, *tg, ids)
    x = bf16_rand((1, 2048), gen)
    gu = int8.grouped_linear(x.to(dev), table, 8, 1024, 0, True)
    ref = np.stack([O.w8a16_linear(npf(x), gq[e], gs[e])[0] for e in order])
    assert_close(npf(gu), ref, BF16_TOL, 'grouped w8a16')
    # full Int8Experts decode, W8A16 and (after the module swap) W8A8
    experts = int8.Int8Experts(0, {'q': tg[0], 'scale': tg[1]}, {'q': tg[2], 'scale': tg[3]})
    wts = torch.rand(1, 8, generator=gen).to(torch.bfloat16)
    top = torch.tensor([ids], dtype=torch.int64)
    out = experts(x.to(dev), top.to(dev), wts.to(dev))
    vals = np.stack([O.expert_w8a16(npf(x), gq[e], gs[e], dq[e], ds[e])[0] for e in order])
    wsorted = [npf(wts)[0, ids.index(e)] for e in order]
    assert_close(npf(out)[0], O.ordered_combine(vals, wsorted), BF16_TOL, 'Int8Experts w8a16')
    saved = int8.grouped_linear
    try:
        int8.grouped_linear = w8a8.grouped_linear
        out8 = experts(x.to(dev), top.to(dev), wts.to(dev))
    finally:
        int8.grouped_linear = saved
    vals8 = np.stack([O.expert_w8a8(npf(x), gq[e], gs[e], dq[e], ds[e])[0] for e in order])
    assert_close(npf(out8)[0], O.ordered_combine(vals8, wsorted), BF16_TOL, 'Int8Experts w8a8')


# ------------------------------------------------------------- a6/a11/a12 glue
def test_ordered_reduce_bit_exact(dev):
    gen = seeded(7)
    v = bf16_rand((8, 2048), gen)
    w = torch.rand(1, 8, generator=gen).to(torch.bfloat16)
    slots = [3, 0, 7, 1, 6, 2, 5, 4]
    table = torch.zeros(8, 5, dtype=torch.int64)
    table[:, 4] = torch.tensor(slots)
    y = int8.ordered_reduce(v.to(dev), table.to(dev), w.to(dev))
    ref = O.ordered_combine(npf(v), [npf(w)[0, s] for s in slots])
    assert np.array_equal(npf(y)[0], ref)
    y32 = int8.ordered_reduce(v.to(dev), table.to(dev), w.float().to(dev))
    assert torch.equal(y32, y)


def test_swiglu_glue(dev):
    gu = bf16_rand((37, 1024), seeded(8), 3.0)
    h = int8.swiglu(gu.to(dev))
    ref = O.swiglu(npf(gu))
    assert_close(npf(h), ref, BF16_TOL, 'swiglu')
    assert (npf(h) == ref).mean() > 0.99


# ------------------------------------------------------------- a8 router / norm
@pytest.mark.parametrize('tokens', [1, 5, 2048])
@pytest.mark.parametrize('skew', [False, True])
def test_router_bit_exact_ids(dev, tokens, skew):
    gen = seeded(9 + tokens)
    x = bf16_rand((tokens, 2048), gen)
    w = bf16_rand((256, 2048), gen, 0.02)
    bias = zipf_bias() if skew else None
    lg, wts, ids = router.router_topk(x.to(dev), w.to(dev), 8,
                                      None if bias is None else torch.from_numpy(bias))
    rl, rw, ri = O.router(npf(x), npf(w), 8, bias)
    assert np.array_equal(lg.cpu().numpy(), rl)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8


def test_router_ties_lowest_id(dev):
    gen = seeded(10)
    w = bf16_rand((256, 2048), gen, 0.02)
    w[200] = w[3]
    w[100] = w[3]
    w[50:60] = 0
    x = bf16_rand((64, 2048), gen)
    _, _, ids = router.router_topk(x.to(dev), w.to(dev), 8)
    _, _, ri = O.router(npf(x), npf(w), 8)
    assert np.array_equal(ids.cpu().numpy(), ri)
    zx = torch.zeros(1, 2048, dtype=torch.bfloat16)
    _, wz, iz = router.router_topk(zx.to(dev), w.to(dev), 8)
    assert iz.cpu().tolist() == [list(range(8))]
    assert np.all(npf(wz) == O.bf16(np.float32(0.125)))


@pytest.mark.parametrize('bias_kind', ['none', 'zero', 'tiny'])
def test_router_key_widths(dev, bias_kind):
    # Logits that are all bf16 values select on 32-bit keys, any other fp32
    # logits on 64-bit keys.  A zero bias keeps every logit a bf16 value; a
    # bias of 2^-20 multiples does not.  All logits are <= 0 (signed-key
    # order, -0 against +0) and rows of w repeat (exact ties).
    gen = seeded(12)
    x = bf16_rand((37, 2048), gen).abs()
    w = -bf16_rand((256, 2048), gen, 0.02).abs()
    w[9] = w[130]
    w[240] = w[130]
    w[17:40] = 0
    x[5] = 0
    bias = {'none': None, 'zero': np.zeros(256, np.float32),
            'tiny': (np.arange(256) % 7).astype(np.float32) * np.float32(2.0 ** -20)}[bias_kind]
    lg, wts, ids = router.router_topk(x.to(dev), w.to(dev), 8,
                                      None if bias is None else torch.from_numpy(bias))
    rl, rw, ri = O.router(npf(x), npf(w), 8, bias)
    assert np.array_equal(lg.cpu().numpy(), rl)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8
    assert ids[5].cpu().tolist() == ri[5].tolist()


def test_rmsnorm_bit_exact(dev):
    gen = seeded(11)
    x = bf16_rand((5, 2048), gen, 3.0)
    w = torch.randn(2048, generator=gen) * 0.1
    assert np.array_equal(npf(router.rmsnorm(x.to(dev), w.to(dev))), O.rmsnorm(npf(x), w.numpy()))
    x2 = bf16_rand((3, 1000), gen)
    assert np.array_equal(npf(router.rmsnorm(x2.to(dev))), O.rmsnorm(npf(x2)))


# ------------------------------------------------------------- a9 route plans
def _ids(gen, t, e, k, skew):
    logits = torch.randn(t, e, generator=gen)
    if skew:
        logits = logits + 3 * torch.from_numpy(zipf_bias(e))
    return logits.topk(k, dim=1).indices


@pytest.mark.parametrize('t,bm,skew', [(1, 16, False), (7, 64, True), (2048, 64, False),
                                       (2048, 16, True), (2048, 128, True), (5000, 64, True)])
def test_route_plan_bit_exact(dev, t, bm, skew):
    ids = _ids(seeded(t + bm), t, 256, 8, skew)
    got = gpu_routes.plan(ids.to(dev), 256, bm)
    ref = O.plan(ids.numpy(), 256, bm)
    for g, r, name in zip(got, ref, ('pos', 'table', 'ordered', 'slots')):
        assert np.array_equal(g.cpu().numpy(), r), name


# ------------------------------------------------------------- a10/a13 routed GEMM
@pytest.mark.parametrize('large', [False, True])
def test_routed_gemm_exact_layout(dev, large):
    """Exactly representable grouped GEMM over uneven groups and empty experts:
    checks gather, tile table, MFMA layout and dequant bit for bit."""
    g = np.random.default_rng(12)
    e, t, k = 20, 150, 2
    ids = _ids(seeded(13), t, e, k, True)
    x = g.integers(-4, 5, size=(t, 256)).astype(np.float32)
    q = g.integers(-127, 128, size=(e, 384, 256)).astype(np.int8)
    s = np.full((e, 384, 2), 2.0 ** -7, np.float32)
    bm = gpu_routes.BM_LARGE if large else gpu_routes.BM_DEFAULT
    pos, table, _, _ = gpu_routes.plan(ids.to(dev), e, bm)
    y = gpu_routes.routed_gemm(torch.from_numpy(x).to(torch.bfloat16).to(dev),
                               torch.from_numpy(q).to(dev), torch.from_numpy(s).to(dev), pos, table,
                               bm, True)
    rpos, _, _, _ = O.plan(ids.numpy(), e, bm)
    flat = np.sort(ids.numpy().reshape(-1), kind='stable')
    ref = np.stack([x[rpos[i]].astype(np.float64) @ (q[flat[i]].astype(np.float64) * 2.0 ** -7).T
                    for i in range(t * k)])
    assert np.array_equal(npf(y), O.bf16(ref.astype(np.float32)))


@pytest.mark.parametrize('large', [False, True])
def test_routed_moe_vs_oracle(dev, large):
    gen = seeded(14)
    e, t, k = 24, 96, 8
    gq, gs = _bank(gen, e, 1024, 2048)
    dq, ds = _bank(gen, e, 2048, 512)
    banks = [torch.from_numpy(a).to(dev) for a in (gq, gs, dq, ds)]
    x = bf16_rand((t, 2048), gen)
    ids = _ids(seeded(15), t, e, k, True)
    wts = torch.softmax(torch.randn(t, k, generator=gen), -1).to(torch.bfloat16)
    out = gpu_routes.routed_moe(x.to(dev), wts.to(dev), ids.to(dev), banks, large)
    xn, idn, wn = npf(x), ids.numpy(), npf(wts)
    ref = np.zeros_like(xn)
    for ex in np.unique(idn):
        token, slot = np.nonzero(idn == ex)
        y = O.expert_w8a16(xn[token], gq[ex], gs[ex], dq[ex], ds[ex])
        ref[token] = O.bf16(ref[token] + O.bf16(y * wn[token, slot][:, None]))
    assert_close(npf(out), ref, BF16_TOL, 'routed_moe')
    out_host = prefill.routed_moe(x.to(dev), wts.to(dev), ids.to(dev), banks, large)
    assert torch.equal(out_host, out)
    # routing weights in fp32 give the same combine inputs after bf16 casts
    assert torch.equal(gpu_routes.routed_moe(x.to(dev), wts.float().to(dev), ids.to(dev), banks,
                                             large), out)


def test_plan_routes_host_matches_device(dev):
    ids = _ids(seeded(16), 300, 256, 8, True)
    positions, segments = routing.plan_routes(ids, 256)
    pos, table, _, _ = gpu_routes.plan(ids.to(dev), 256, 16)
    assert torch.equal(positions[0], pos.cpu())
    tiles = [(e, s0, stop) for e, b, stop in segments for s0 in range(b, stop, 16)]
    assert [tuple(r) for r in table[:len(tiles)].cpu().tolist()] == tiles


# ------------------------------------------------------------- a12 bit-exact, f4 lm_head
@pytest.mark.parametrize('dtype', [torch.bfloat16, torch.float16])
def test_routed_reduce_bit_exact(dev, dtype):
    """Prefill combine (prefill._reduce, prefill.py:37-49) on identical inputs:
    per token, its routes in ascending expert id, acc = T(acc + T(v * w)),
    bit for bit against the oracle's ordered_combine, including a token whose
    weights arrive in fp32."""
    rnd = O.bf16 if dtype == torch.bfloat16 else O.fp16
    t, k, e, n = 300, 8, 256, 2048
    ids = _ids(seeded(50), t, e, k, True)
    pos, table, ordered, slots = gpu_routes.plan(ids.to(dev), e, 96)
    gen = seeded(51)
    v = (torch.randn(t * k, n, generator=gen) * 2).to(dtype)
    w = torch.softmax(torch.randn(t, k, generator=gen), -1).to(dtype)
    y = gpu_routes.routed_reduce(v.to(dev), ordered, slots, w.to(dev), t, n)
    vn, wn, idn = v.float().numpy(), w.float().numpy(), ids.numpy()
    rpos, _, rordered, rslots = O.plan(idn, e, 96)
    for tok in range(t):
        rows = vn[rordered[tok]]                     # its routes' rows, ascending expert
        wts = wn[tok, rslots[tok]]
        assert np.array_equal(y[tok].float().cpu().numpy(), O.ordered_combine(rows, wts, rnd))
    y32 = gpu_routes.routed_reduce(v.to(dev), ordered, slots, w.float().to(dev), t, n)
    assert torch.equal(y32, y)


LM_HEAD_N = 248320  # vocabulary of the 35B-A3B configuration


@pytest.mark.parametrize('m', [1, 2])
def test_lm_head_vocab_shape(dev, m):
    """int8.linear at the lm_head shape, [m, 2048] x [248320, 2048] (the
    reference quantizes lm_head with the same rule, convert.py:80-81, and runs
    it through int8.linear, int8.py:26-37): a sample of output rows spread over
    the whole vocabulary, always including the first and last rows, against
    the oracle; every row is finite and rows of the sample's neighbours
    agree with an integer-exact reconstruction."""
    gen = torch.Generator(device=dev)
    gen.manual_seed(60)
    w = torch.randn((LM_HEAD_N, 2048), generator=gen, device=dev) * 0.02
    q, s = convert.quantize_g128(w)
    del w
    x = torch.randn((m, 2048), generator=gen, device=dev).to(torch.bfloat16)
    y = int8.linear(x, q, s)
    torch.cuda.synchronize()
    assert y.shape == (m, LM_HEAD_N) and torch.isfinite(y.float()).all()
    rows = np.unique(np.concatenate([
        np.random.default_rng(61).choice(LM_HEAD_N, 250, replace=False),
        np.arange(16), np.arange(LM_HEAD_N - 16, LM_HEAD_N)]))
    idx = torch.from_numpy(rows).to(dev)
    qs, ss = q[idx].cpu().numpy(), s[idx].cpu().numpy()
    ref = O.w8a16_linear(npf(x), qs, ss)
    assert_close(npf(y)[:, rows], ref, BF16_TOL, f'lm_head m={m}')
