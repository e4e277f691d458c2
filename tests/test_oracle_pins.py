"""Pins every oracle function against something other than its own formula.

Sources of truth, per function:
  quantize_weight  the reference's own known-answer test (tests/test_release.py:20-26),
                   exact-rational brute force, invariants
  dequant / bf16   exact-rational products, torch's independent bf16 cast, ties
  act_quant        exact-rational brute force; multiply-by-reciprocal vs divide
  w8a8_partials    pure-Python loops, linearity
  w8a8_accumulate  exact-rational step-by-step evaluation; order sensitivity
  w8a16_linear     float64 matmul; exactly representable integer cases
  swiglu           float64 formula; gate/up half order
  ordered_combine  scalar loop with torch's bf16 cast; order sensitivity
  router           exact-rational logits; brute-force top-k; ties; fp64 softmax
  plan/plan_routes pure-Python definitions on ragged inputs with empty experts
  rmsnorm          float64 formula
  moe_block        float64 dense formulation of the whole block
  fp16 variants    exact-rational fp16 rounding with ties; torch's independent fp16
                   cast; the fp16 GEMM/SwiGLU/combine against float64 and scalar loops
"""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close, seeded


# ------------------------------------------------------------- exact helpers
def round_f32(fr):
    """Round a Fraction to the nearest float32 (ties to even), exactly."""
    fr = Fraction(fr)
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormal spacing
    scale = Fraction(2) ** (e - 23)
    m = a / scale
    fl = math.floor(m)
    rem = m - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * float(fl * scale)


def f32(v):
    return Fraction(float(np.float32(v)))


def torch_bf16(v):
    return float(torch.tensor(float(v), dtype=torch.float32).to(torch.bfloat16).float())


# ------------------------------------------------------------- quantizer (a1)
def test_quantizer_reference_known_answer():
    # tests/test_release.py:20-26 of the reference, restated.
    weight = torch.linspace(-1, 1, 256).reshape(2, 128).bfloat16()
    q, s = O.quantize_weight(weight.float().numpy())
    ref_scale = weight.float().abs().amax(-1, keepdim=True) / 127
    ref = (weight.float() / ref_scale).round().clamp(-127, 127).to(torch.int8)
    assert np.array_equal(q, ref.numpy())
    assert np.array_equal(s[:, 0], ref_scale[:, 0].numpy())


def test_quantizer_exact_rational():
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((3, 256)) * 0.02).astype(np.float32)
    w[1, :128] = 0.0  # all-zero group -> clamp_min(1e-30)
    q, s = O.quantize_weight(w)
    for r in range(3):
        for g in range(2):
            grp = w[r, g * 128:(g + 1) * 128]
            amax = max(abs(Fraction(float(v))) for v in grp)
            se = max(round_f32(amax / 127), float(np.float32(1e-30)))
            assert s[r, g] == np.float32(se)
            for j, v in enumerate(grp):
                qq = round_f32(Fraction(float(v)) / Fraction(se))
                qq = max(-127, min(127, round(qq)))  # round(): ties to even
                assert q[r, g * 128 + j] == qq
    nz = q.reshape(3, 2, 128)
    assert np.abs(nz).max() <= 127
    assert (np.abs(nz[0]).max(-1) == 127).all()
    assert (nz[1, 0] == 0).all()


# ------------------------------------------------------------- bf16 / dequant
def test_bf16_rounding_matches_torch_and_ties():
    rng = np.random.default_rng(2)
    v = rng.standard_normal(4096).astype(np.float32) * 10
    # exact ties: bf16 value + half an ulp
    base = O.bf16(v)
    ulp = np.abs(base) * 2.0 ** -7
    ties = (base + ulp / 2).astype(np.float32)
    for arr in (v, ties, np.array([1 + 2 ** -8, 1 + 3 * 2 ** -8, -0.0, 65504.0], np.float32)):
        ref = torch.from_numpy(arr).to(torch.bfloat16).float().numpy()
        assert np.array_equal(O.bf16(arr).view(np.uint32), ref.view(np.uint32))
    assert O.bf16(np.float32(1 + 2 ** -8)) == 1.0            # tie -> even
    assert O.bf16(np.float32(1 + 3 * 2 ** -8)) == 1 + 2 ** -6  # tie -> even (up)


def test_dequant_is_rounded_exact_product():
    rng = np.random.default_rng(3)
    q = rng.integers(-127, 128, size=(4, 256)).astype(np.int8)
    s = (rng.random((4, 2)) * 1e-3 + 1e-5).astype(np.float32)
    w = O.dequant(q, s)
    for r in range(4):
        for k in range(0, 256, 7):
            exact = Fraction(int(q[r, k])) * Fraction(float(s[r, k // 128]))
            assert w[r, k] == np.float32(torch_bf16(round_f32(exact)))


# ------------------------------------------------------------- act quant (a4)
def test_act_quant_exact_rational_and_reciprocal():
    rng = np.random.default_rng(4)
    x = O.bf16(rng.standard_normal((2, 256)).astype(np.float32))
    x[1, 128:] = 0.0
    q, s = O.act_quant(x)
    inv = f32(1.0 / 127.0)
    for r in range(2):
        for g in range(2):
            grp = x[r, g * 128:(g + 1) * 128]
            amax = max(max(abs(Fraction(float(v))) for v in grp), f32(1e-10))
            se = round_f32(amax * inv)
            assert s[r, g] == np.float32(se)
            for j, v in enumerate(grp):
                assert q[r, g * 128 + j] == round(round_f32(Fraction(float(v)) / Fraction(se)))
    assert (q[1, 128:] == 0).all()
    # a value where amax * fl(1/127) != fl(amax / 127): the oracle must multiply
    found = None
    for cand in rng.standard_normal(20000).astype(np.float32):
        a = float(abs(O.bf16(np.array([cand]))[0]))
        if a and np.float32(a * np.float32(1 / 127)) != np.float32(a / np.float32(127)):
            found = a
            break
    assert found is not None
    xs = np.zeros((1, 128), np.float32)
    xs[0, 0] = found
    _, sc = O.act_quant(xs)
    assert sc[0, 0] == np.float32(found * np.float32(1 / 127))
    assert sc[0, 0] != np.float32(found / np.float32(127))


# ------------------------------------------------------------- W8A8 (a5)
def test_w8a8_partials_brute_force_and_linearity():
    rng = np.random.default_rng(5)
    xq = rng.integers(-127, 128, size=(2, 256)).astype(np.int8)
    wq = rng.integers(-127, 128, size=(3, 256)).astype(np.int8)
    p = O.w8a8_partials(xq, wq)
    for m in range(2):
        for n in range(3):
            for g in range(2):
                ref = sum(int(xq[m, k]) * int(wq[n, k]) for k in range(g * 128, g * 128 + 128))
                assert p[m, n, g] == ref
    x2 = rng.integers(-60, 60, size=(2, 256)).astype(np.int8)
    x1 = rng.integers(-60, 60, size=(2, 256)).astype(np.int8)
    assert np.array_equal(O.w8a8_partials(x1 + x2, wq),
                          O.w8a8_partials(x1, wq) + O.w8a8_partials(x2, wq))
    extreme = np.full((1, 128), -127, np.int8)
    assert O.w8a8_partials(extreme, extreme)[0, 0, 0] == 128 * 127 * 127


def test_w8a8_accumulate_exact_sequence_and_order():
    rng = np.random.default_rng(6)
    p = rng.integers(-2_000_000, 2_000_000, size=(1, 2, 16)).astype(np.int32)
    xs = (rng.random((1, 16)) * 0.03).astype(np.float32)
    ws = (rng.random((2, 16)) * 3e-4).astype(np.float32)
    acc = O.w8a8_accumulate(p, xs, ws)
    for n in range(2):
        a = Fraction(0)
        for g in range(16):
            t = Fraction(round_f32(Fraction(int(p[0, n, g])) * f32(xs[0, g])))
            t = Fraction(round_f32(t * f32(ws[n, g])))
            a = Fraction(round_f32(a + t))
        assert acc[0, n] == np.float32(float(a))
    # reversed group order gives a different fp32 value for some input: the
    # oracle is order-faithful, not merely close
    diffs = 0
    for seed in range(40):
        r = np.random.default_rng(100 + seed)
        pp = r.integers(-2_000_000, 2_000_000, size=(1, 1, 16)).astype(np.int32)
        xx = (r.random((1, 16)) * 0.03).astype(np.float32)
        ww = (r.random((1, 16)) * 3e-4).astype(np.float32)
        fwd = O.w8a8_accumulate(pp, xx, ww)[0, 0]
        rev = O.w8a8_accumulate(pp[:, :, ::-1], xx[:, ::-1], ww[:, ::-1])[0, 0]
        diffs += fwd != rev
    assert diffs > 0


# ------------------------------------------------------------- W8A16 (a2)
def test_w8a16_linear_vs_float64_and_exact_case():
    g = seeded(7)
    x = O.bf16(torch.randn(5, 256, generator=g).numpy())
    w = (torch.randn(64, 256, generator=g) * 0.02).numpy()
    q, s = O.quantize_weight(w)
    y = O.w8a16_linear(x, q, s)
    ref = x.astype(np.float64) @ O.dequant(q, s).astype(np.float64).T
    assert_close(y, ref, BF16_TOL, 'w8a16 vs f64')
    # exactly representable: small integers times power-of-two scales
    xi = np.random.default_rng(8).integers(-8, 9, size=(3, 256)).astype(np.float32)
    qi = np.random.default_rng(9).integers(-127, 128, size=(16, 256)).astype(np.int8)
    si = np.full((16, 2), 2.0 ** -6, np.float32)
    exact = xi.astype(np.float64) @ (qi.astype(np.float64) * 2.0 ** -6).T
    assert np.array_equal(O.w8a16_linear(xi, qi, si), O.bf16(exact.astype(np.float32)))


# ------------------------------------------------------------- SwiGLU (a11)
def test_swiglu_formula_and_half_order():
    rng = np.random.default_rng(10)
    gu = O.bf16(rng.standard_normal((4, 64)).astype(np.float32) * 3)
    h = O.swiglu(gu)
    g, u = gu[:, :32].astype(np.float64), gu[:, 32:].astype(np.float64)
    assert_close(h, g / (1 + np.exp(-g)) * u, BF16_TOL, 'swiglu')
    swapped = O.swiglu(np.concatenate([gu[:, 32:], gu[:, :32]], 1))
    assert not np.array_equal(h, swapped)


# ------------------------------------------------------------- combine (a6/a12)
def test_ordered_combine_scalar_and_order():
    rng = np.random.default_rng(11)
    v = O.bf16(rng.standard_normal((8, 64)).astype(np.float32))
    w = O.bf16(rng.random(8).astype(np.float32))
    out = O.ordered_combine(v, w)
    for n in range(0, 64, 5):
        acc = 0.0
        for e in range(8):
            acc = torch_bf16(acc + torch_bf16(float(v[e, n]) * float(w[e])))
        assert out[n] == np.float32(acc)
    big = np.array([[1.0], [2.0 ** -8], [2.0 ** -8]], np.float32)
    ones = np.ones(3, np.float32)
    assert O.ordered_combine(big, ones)[0] == 1.0          # each tiny term rounds away
    assert O.ordered_combine(big[::-1], ones)[0] != 1.0    # summed first, it survives


# ------------------------------------------------------------- router (a8)
def test_router_logits_exact_rational():
    g = seeded(12)
    x = O.bf16(torch.randn(3, 256, generator=g).numpy())
    w = O.bf16((torch.randn(8, 256, generator=g) * 0.02).numpy())
    lg = O.router_logits(x, w)
    for t in range(3):
        for e in range(8):
            exact = sum(Fraction(float(a)) * Fraction(float(b)) for a, b in zip(x[t], w[e]))
            assert lg[t, e] == np.float32(torch_bf16(round_f32(exact)))


def test_topk_brute_force_and_ties():
    rng = np.random.default_rng(13)
    lg = O.bf16(rng.standard_normal((50, 32)).astype(np.float32))
    lg[:, 5] = lg[:, 20]          # forced exact ties
    lg[:, 7] = lg[:, 3]
    lg[0, :] = 0.0                 # a fully tied row
    lg[1, 2], lg[1, 9] = -0.0, 0.0
    ids = O.topk_select(lg, 8)
    for t in range(50):
        ref = sorted(range(32), key=lambda e: (-float(lg[t, e]), e))[:8]
        assert list(ids[t]) == ref
    assert list(ids[0]) == list(range(8))


def test_router_weights_vs_float64():
    g = seeded(14)
    x = O.bf16(torch.randn(16, 256, generator=g).numpy())
    w = O.bf16((torch.randn(32, 256, generator=g) * 0.05).numpy())
    bias = (np.arange(32) * 0.01).astype(np.float32)
    lg, wts, ids = O.router(x, w, 8, bias)
    l64 = lg.astype(np.float64)
    p = np.exp(l64 - l64.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    top = np.take_along_axis(p, ids, -1)
    assert_close(wts, top / top.sum(-1, keepdims=True), BF16_TOL, 'router weights')
    assert np.all(np.diff(np.take_along_axis(lg, ids, -1), axis=1) <= 0)


# ------------------------------------------------------------- route plans (a9)
def _ragged_ids(rng, t, k, e, empty):
    ids = np.empty((t, k), np.int64)
    pool = np.array([i for i in range(e) if i not in empty])
    for r in range(t):
        ids[r] = rng.choice(pool, size=k, replace=False)
    return ids


@pytest.mark.parametrize('t,k,e,bm', [(1, 8, 256, 64), (7, 4, 16, 3), (33, 8, 40, 16)])
def test_plan_brute_force(t, k, e, bm):
    rng = np.random.default_rng(t)
    ids = _ragged_ids(rng, t, k, e, empty={0, e // 2})
    pos, table, ordered, slots = O.plan(ids, e, bm)
    flat = [(int(ids[i // k, i % k]), i) for i in range(t * k)]
    srt = sorted(flat)  # stable by expert: ties by flat index
    assert list(pos) == [i // k for _, i in srt]
    tiles = []
    start = 0
    for ex in range(e):
        cnt = sum(1 for v, _ in flat if v == ex)
        for s0 in range(start, start + cnt, bm):
            tiles.append((ex, s0, start + cnt))
        start += cnt
    assert table.shape == ((t * k + bm - 1) // bm + e, 3)
    assert [tuple(r) for r in table[:len(tiles)]] == tiles
    assert (table[len(tiles):] == 0).all()
    where = {i: p for p, (_, i) in enumerate(srt)}
    for r in range(t):
        order = sorted(range(k), key=lambda j: (int(ids[r, j]), j))
        assert list(slots[r]) == order
        assert list(ordered[r]) == [where[r * k + j] for j in order]


def test_plan_routes_brute_force():
    rng = np.random.default_rng(15)
    ids = _ragged_ids(rng, 9, 4, 12, empty={3})
    positions, segments = O.plan_routes(ids, 12)
    flat = sorted((int(ids[i // 4, i % 4]), i) for i in range(36))
    assert [(int(a), int(b)) for a, b in positions.T] == [(i // 4, i % 4) for _, i in flat]
    counts = [sum(1 for v, _ in flat if v == ex) for ex in range(12)]
    exp, s0 = [], 0
    for ex, c in enumerate(counts):
        if c:
            exp.append((ex, s0, s0 + c))
            s0 += c
    assert segments == exp
    with pytest.raises(ValueError):
        O.plan_routes(np.array([[12]]), 12)


# ------------------------------------------------------------- RMSNorm / block
def test_rmsnorm_vs_float64():
    rng = np.random.default_rng(16)
    x = O.bf16(rng.standard_normal((4, 2048)).astype(np.float32) * 3)
    w = (rng.standard_normal(2048) * 0.1).astype(np.float32)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * (1 + w)
    assert_close(O.rmsnorm(x, w), ref, BF16_TOL, 'rmsnorm')


def _tiny_layer(rng, e=8, h=256, inter=128):
    def qz(shape):
        return O.quantize_weight((rng.standard_normal(shape) * 0.05).astype(np.float32))
    gq, gs = qz((e + 1, 2 * inter, h))
    dq, ds = qz((e + 1, h, inter))
    return dict(router_w=O.bf16((rng.standard_normal((e, h)) * 0.05).astype(np.float32)),
                router_bias=None,
                shared_gate_w=O.bf16((rng.standard_normal(h) * 0.05).astype(np.float32)),
                gu_q=gq, gu_s=gs, dn_q=dq, dn_s=ds)


@pytest.mark.parametrize('tokens', [1, 6])
def test_moe_block_vs_float64_dense(tokens):
    rng = np.random.default_rng(17 + tokens)
    layer = _tiny_layer(rng)
    x = O.bf16(rng.standard_normal((tokens, 256)).astype(np.float32))
    out, (_, wts, ids) = O.moe_block(x, layer, k=4)
    x64 = x.astype(np.float64)

    def mlp(e):
        gu = x64 @ O.dequant(layer['gu_q'][e], layer['gu_s'][e], lambda a: a).astype(np.float64).T
        g, u = gu[:, :128], gu[:, 128:]
        hdn = g / (1 + np.exp(-g)) * u
        return hdn @ O.dequant(layer['dn_q'][e], layer['dn_s'][e], lambda a: a).astype(np.float64).T

    ref = np.zeros_like(x64)
    for t in range(tokens):
        for j in range(4):
            ref[t] += wts[t, j] * mlp(ids[t, j])[t]
    gate = x64 @ layer['shared_gate_w'].astype(np.float64)
    ref += (1 / (1 + np.exp(-gate)))[:, None] * mlp(8)
    # W8A8 decode (tokens == 1) adds activation-quantization error on top of
    # the bf16 rounding chain; 5e-2 norm-wise covers both
    rel = np.linalg.norm(out - ref) / np.linalg.norm(ref)
    assert rel < 5e-2


# ------------------------------------------------------------- fp16 activations
def round_f16(fr):
    """Round a Fraction to the nearest fp16 value (ties to even), exactly;
    normal range only."""
    fr = Fraction(fr)
    if fr == 0:
        return 0.0
    sign = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 10)
    m = a / ulp
    lo = math.floor(m)
    rem = m - lo
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and lo % 2 == 1):
        lo += 1
    return sign * float(lo * ulp)


def test_fp16_rounding_exact_rational_and_torch():
    rng = np.random.default_rng(40)
    v = (rng.standard_normal(2000) * 30).astype(np.float32)
    ties = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(2 + 2.0 ** -10)], np.float32)
    v = np.concatenate([v, ties])
    got = O.fp16(v)
    for i in list(range(0, 2000, 37)) + [2000, 2001, 2002]:
        assert got[i] == np.float32(round_f16(Fraction(float(v[i])))), v[i]
    assert np.array_equal(got, torch.from_numpy(v).half().float().numpy())
    assert got[2000] == 1.0 and got[2001] == np.float32(1 + 2.0 ** -9)  # ties to even


def test_fp16_paths_vs_float64_and_scalar_loops():
    rng = np.random.default_rng(41)
    x = O.fp16(rng.standard_normal((5, 256)).astype(np.float32))
    q, s = O.quantize_weight((rng.standard_normal((64, 256)) * 0.02).astype(np.float32))
    y = O.w8a16_linear(x, q, s, O.fp16)
    ref = x.astype(np.float64) @ (q.astype(np.float64).reshape(64, 2, 128)
                                  * s[..., None]).reshape(64, 256).T
    assert_close(y, ref, 1e-2, 'w8a16 fp16 vs f64')
    assert np.array_equal(y, O.fp16(y))  # outputs are fp16 values
    gu = O.fp16(rng.standard_normal((4, 64)).astype(np.float32) * 3)
    h = O.swiglu(gu, O.fp16)
    g, u = gu[:, :32].astype(np.float64), gu[:, 32:].astype(np.float64)
    assert_close(h, g / (1 + np.exp(-g)) * u, 1e-2, 'swiglu fp16')
    v = O.fp16(rng.standard_normal((8, 16)).astype(np.float32))
    w = O.fp16(rng.random(8).astype(np.float32))
    out = O.ordered_combine(v, w, O.fp16)
    for n in range(16):
        acc = torch.tensor(0.0, dtype=torch.float16)
        for e in range(8):
            term = (torch.tensor(float(v[e, n])) * torch.tensor(float(w[e]))).half()
            acc = (acc.float() + term.float()).half()
        assert out[n] == np.float32(acc.item())
