"""GPU parity of the fused MoE-FFN layer (synthetic stack) against the oracle.

Routing ids are compared bit for bit (the RMSNorm feeding the router is
reproducible bit for bit and the router logits are order-independent);
layer outputs within the bf16 tolerance of tests/conftest.py.  Large-size
checks use size-independent properties: token independence across chunks,
HIP-graph replay equality, and a sampled per-token oracle at T = 2048.
"""
import numpy as np
import pytest
import torch

from localmoe35ba3b_amd import router
from localmoe35ba3b_amd.runtime.stack import EPS, SyntheticMoEStack, zipf_bias
from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def stack(dev):
    return SyntheticMoEStack(layers=2, seed=11, device=dev, max_tokens=2048)


def npf(t):
    return t.detach().float().cpu().numpy()


def inputs(tokens, seed, dev):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(tokens, 2048, generator=g).to(torch.bfloat16).to(dev)


def run_layer(stack, h, l=0):
    t = h.shape[0]
    ids = torch.empty((t, 8), dtype=torch.int32, device=h.device)
    wts = torch.empty((t, 8), dtype=torch.bfloat16, device=h.device)
    out = h.clone()
    stack.layer_forward(out, l, ids, wts)
    return out, ids, wts


def oracle_layer(stack, h_np, l, ids_gpu):
    layer = stack.layer_host(l, experts=np.unique(ids_gpu))
    return O.moe_layer(h_np, layer, k=8, eps=EPS)


@pytest.mark.parametrize('seed', [0, 1, 2])
def test_decode_layer(stack, dev, seed):
    h = inputs(1, seed, dev)
    out, ids, wts = run_layer(stack, h, seed % 2)
    ref, (lg, rw, ri) = oracle_layer(stack, npf(h), seed % 2, ids.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8
    assert_close(npf(out), ref, BF16_TOL, 'decode layer')


@pytest.mark.parametrize('tokens', [2, 67, 96, 97, 192])
def test_prefill_layer(stack, dev, tokens):
    """One prefill layer against the oracle; 96, 97 and 192 tokens put the
    shared expert's rows on and just past whole 96-row tiles of the
    tile-major gather map."""
    h = inputs(tokens, 100 + tokens, dev)
    out, ids, wts = run_layer(stack, h)
    ref, (lg, rw, ri) = oracle_layer(stack, npf(h), 0, ids.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8
    assert_close(npf(out), ref, BF16_TOL, 'prefill layer')


def test_prefill_chunk_2048_sampled(stack, dev):
    h = inputs(2048, 7, dev)
    out, ids, _ = run_layer(stack, h, 1)
    # routing of every token, bit for bit, from the oracle router on the same
    # normalized rows
    layer = stack.layer_host(1, experts=[])
    xn = O.rmsnorm(npf(h), None, EPS)
    _, _, ri = O.router(xn, layer['router_w'], 8)
    assert np.array_equal(ids.cpu().numpy(), ri)
    # full layer output for a sample of tokens
    sample = np.random.default_rng(0).choice(2048, 12, replace=False)
    sub_ids = ids.cpu().numpy()[sample]
    ref, _ = oracle_layer(stack, npf(h)[sample], 1, sub_ids)
    assert_close(npf(out)[sample], ref, BF16_TOL, 'prefill 2048 sample')


def test_token_independence(stack, dev):
    """The MoE-FFN is per token: one 96-token call equals three 32-token calls."""
    h = inputs(96, 8, dev)
    whole, _, _ = run_layer(stack, h)
    parts = torch.cat([run_layer(stack, h[i:i + 32].contiguous())[0] for i in range(0, 96, 32)])
    assert torch.equal(whole, parts)


def test_prefill_max_tokens(dev):
    """The largest token count one call accepts (65536 tokens, 524288 routes,
    about 2048 rows per expert): one call equals 32 calls of 2048 tokens bit
    for bit, and a sample of tokens matches the oracle (routing exact,
    outputs within the bf16 tolerance)."""
    st = SyntheticMoEStack(layers=1, seed=41, device=dev, max_tokens=65536)
    h = inputs(65536, 40, dev)
    whole, ids, _ = run_layer(st, h)
    parts = torch.cat([run_layer(st, h[i:i + 2048].contiguous())[0]
                       for i in range(0, 65536, 2048)])
    assert torch.equal(whole, parts)
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=256)
    assert counts.sum() == 65536 * 8 and counts.max() > 2048
    sample = np.random.default_rng(3).choice(65536, 12, replace=False)
    sample[0] = 65535
    sub_ids = ids.cpu().numpy()[sample]
    ref, (_, _, ri) = oracle_layer(st, npf(h[sample]), 0, sub_ids)
    assert np.array_equal(sub_ids, ri)
    assert_close(npf(whole[sample]), ref, BF16_TOL, 'prefill 65536 sample')


def test_decode_graph_replay(stack, dev):
    h0 = inputs(1, 9, dev)
    eager = h0.clone()
    stack.forward(eager)
    static = h0.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        stack.forward(static.clone())  # warm up on the capture stream
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.forward(static)
    for _ in range(3):
        static.copy_(h0)
        graph.replay()
        torch.cuda.synchronize()
        other = inputs(1, 10, dev)
        stack.forward(other)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static, eager)


def test_prefill_graph_replay(stack, dev):
    """The prefill path (96 tokens, both layers) captured as a HIP graph gives
    the eager result on every replay, with eager prefill work in between."""
    h0 = inputs(96, 14, dev)
    eager = h0.clone()
    stack.forward(eager)
    static = h0.clone()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        stack.forward(static.clone())
    torch.cuda.current_stream().wait_stream(stream)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.forward(static)
    for i in range(3):
        static.copy_(h0)
        graph.replay()
        torch.cuda.synchronize()
        other = inputs(67, 15 + i, dev)
        stack.forward(other)
        torch.cuda.synchronize()
        assert torch.equal(static, eager)


@pytest.mark.parametrize('tokens,chunk', [(250, 96), (4096, 2048)])
def test_overlapped_prefill(stack, dev, tokens, chunk):
    """Chunks overlapped on two streams (chunk c enters layer l once chunk
    c-1 has left layer l-1) equal chunks run one after the other, eagerly
    and as a HIP graph replayed with eager work in between; 250 tokens in
    chunks of 96 give three chunks, the last one ragged."""
    h0 = inputs(tokens, 21, dev)
    serial = stack.prefill(h0, chunk=chunk, overlap=False)
    assert torch.equal(stack.prefill(h0, chunk=chunk), serial)
    static = h0.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack.prefill_(static, chunk)
    for i in range(3):
        static.copy_(h0)
        graph.replay()
        torch.cuda.synchronize()
        other = inputs(67, 30 + i, dev)
        stack.forward(other)
        torch.cuda.synchronize()
        assert torch.equal(static, serial), f'replay {i}'


def test_prefill_rejects_oversized_chunk(stack, dev):
    """A chunk larger than the workspace is refused before any work is queued
    (the hidden states stay untouched)."""
    h = inputs(4096, 22, dev)
    before = h.clone()
    with pytest.raises(MemoryError):
        stack.prefill_(h, chunk=4096)
    with pytest.raises(ValueError):
        stack.prefill_(h.float(), chunk=2048)
    torch.cuda.synchronize()
    assert torch.equal(h, before)
    assert stack.prefill(h[:0]).shape == (0, 2048)  # an empty prompt queues nothing


def test_skewed_router_bias(dev):
    st = SyntheticMoEStack(layers=1, seed=12, device=dev, max_tokens=256,
                           router_bias=zipf_bias())
    h = inputs(256, 13, dev)
    out, ids, _ = run_layer(st, h)
    counts = np.bincount(ids.cpu().numpy().reshape(-1), minlength=256)
    assert (counts == 0).sum() > 20  # skew leaves many experts empty
    layer = st.layer_host(0, experts=np.unique(ids.cpu().numpy()))
    ref, (_, _, ri) = O.moe_layer(npf(h), layer, k=8, eps=EPS)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert_close(npf(out), ref, BF16_TOL, 'skewed prefill layer')
    for seed in (30, 31):  # the decode path adds the same bias
        h1 = inputs(1, seed, dev)
        out1, ids1, wts1 = run_layer(st, h1)
        layer1 = st.layer_host(0, experts=np.unique(ids1.cpu().numpy()))
        ref1, (_, rw1, ri1) = O.moe_layer(npf(h1), layer1, k=8, eps=EPS)
        assert np.array_equal(ids1.cpu().numpy(), ri1)
        assert np.abs(npf(wts1) - rw1).max() <= 2.0 ** -8
        assert_close(npf(out1), ref1, BF16_TOL, 'skewed decode layer')


def test_zipf_chunk_2048(dev):
    """One layer on the survey's skewed prefill workload at its stated size:
    a 2048-token chunk (x ~ N(0, 1) from the device generator, seed 3) with
    the Zipf(1.1) router bias, so the hottest expert takes about 2,000 rows
    (21+ tiles of 96) while about 150 experts get none.  Routing ids equal
    the oracle router's on the same normalized rows bit for bit; the layer
    output matches the oracle on a sample of tokens that includes every
    token routed into the hot expert's last tile, tokens from its other
    tiles and random tokens; a HIP-graph replay equals the eager run."""
    st = SyntheticMoEStack(layers=1, seed=3, device=dev, max_tokens=2048,
                           router_bias=zipf_bias())
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    x = torch.randn((2048, 2048), generator=gen, device=dev).to(torch.bfloat16)
    out, ids, _ = run_layer(st, x)
    torch.cuda.synchronize()
    idn = ids.cpu().numpy()
    xn = st.workspace_view('normed', 2048).clone()
    rows = st.workspace_view('route_rows', 2048).cpu().numpy()
    assert np.array_equal(npf(xn), O.rmsnorm(npf(x), None, EPS))
    _, _, ri = O.router(npf(xn), st.layer_host(0, experts=[])['router_w'], 8,
                        st.router_bias.cpu().numpy())
    assert np.array_equal(idn, ri)
    counts = np.bincount(idn.reshape(-1), minlength=256)
    hot = int(counts.argmax())
    assert counts[hot] > 20 * 96 and (counts == 0).sum() > 120
    # the hot expert's rows are [off, off + count) of the expert-sorted order
    off = int(counts[:hot].sum())
    tok_hot, slot_hot = np.nonzero(idn == hot)
    r_hot = rows[tok_hot, slot_hot]
    assert np.array_equal(np.sort(r_hot), np.arange(off, off + counts[hot]))
    last_tile = off + 96 * ((counts[hot] - 1) // 96)
    in_last = tok_hot[r_hot >= last_tile]
    rng = np.random.default_rng(4)
    sample = np.unique(np.concatenate([
        in_last, rng.choice(tok_hot[r_hot < last_tile], 8, replace=False),
        rng.choice(2048, 8, replace=False)]))
    ref, (_, _, rs) = oracle_layer(st, npf(x)[sample], 0, idn[sample])
    assert np.array_equal(rs, idn[sample])
    assert_close(npf(out)[sample], ref, BF16_TOL, 'Zipf chunk sample')
    # graph replay of the same chunk, with eager work between replays
    static = x.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st.layer_forward(static, 0)
    for i in range(2):
        static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        run_layer(st, inputs(300, 60 + i, dev))
        torch.cuda.synchronize()
        assert torch.equal(static, out), f'replay {i}'


def f16_expert(x, gu_q, gu_s, dn_q, dn_s, round_to=O.bf16):
    """O.expert_w8a16 with the gate_up of the fused layer's fp16 path
    (f16_gate_up_model: unrounded q * s) and the reference's down."""
    return O.w8a16_linear(O.swiglu(f16_gate_up_model(x, gu_q, gu_s)), dn_q, dn_s, round_to)


@pytest.mark.parametrize('fmt', [0, 1])
def test_prefill_extreme_inputs(dev, fmt, monkeypatch):
    """The prefill path on inputs at the edges of its number formats, with
    both gate_up tile formats: RMSNorm weights that put normalized values
    far beyond fp16's range (the fp16 row copy is scaled by a power of two
    from the row norm), a token row 10^6 times smaller than the others, a
    routed expert with all-zero weight groups (scale 1e-30, the quantizer's
    floor) and groups with scales of 1e-3 and 1e3 times their neighbours'.
    Routing is exact and the layer output stays within the bf16 tolerance
    of the oracle (norm-wise for the fp16 path, whose skipped bf16 rounding
    of q * s exceeds the elementwise bound on a few hundred of the large,
    cancelling outputs here; elementwise against a model of its own
    arithmetic)."""
    st = SyntheticMoEStack(layers=1, seed=91, device=dev, max_tokens=256, norm=True,
                           gate_up_format=fmt)
    g = torch.Generator(device=dev)
    g.manual_seed(92)
    w = torch.randn(2048, generator=g, device=dev) * 0.5
    w[::97] = 3000.0  # (1 + w) up to 3001: |xn| up to ~1.4e5 on those channels
    st.norm_w[0].copy_(w)
    h = inputs(256, 93, dev)
    h[7] *= 1e-6
    # pick an expert that the routing uses, then damage its weights
    _, ids, _ = run_layer(st, h)
    e = int(ids[0, 0])
    st.gu_q[0, e, :, :128] = 0
    st.gu_s[0, e, :, 0] = 1e-30
    st.gu_s[0, e, :512, 3] *= 1e-3
    st.gu_s[0, e, 512:, 5] *= 1e3
    st.dn_q[0, e, :, 128:256] = 0
    st.dn_s[0, e, :, 1] = 1e-30
    st.build_prefill_tiles(fmt)
    out, ids, wts = run_layer(st, h)
    torch.cuda.synchronize()
    ref, (_, rw, ri) = oracle_layer(st, npf(h), 0, ids.cpu().numpy())
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8
    assert np.isfinite(npf(out)).all()
    if fmt == 0:
        assert_close(npf(out), ref, BF16_TOL, 'extreme inputs, exact gate_up')
        return
    rel = np.linalg.norm(npf(out) - ref) / np.linalg.norm(ref)
    assert rel <= BF16_TOL, rel
    monkeypatch.setattr(O, 'expert_w8a16', f16_expert)
    model, _ = oracle_layer(st, npf(h), 0, ids.cpu().numpy())
    assert_close(npf(out), model, BF16_TOL, 'extreme inputs, fp16 gate_up vs its model')


@pytest.mark.parametrize('fmt', [0, 1])
@pytest.mark.parametrize('tokens', [1, 100, 300])
def test_chained_layers_bit_identical(dev, fmt, tokens):
    """Chained layer calls (lm_moe_layer_forward_chain: each combine does the
    next layer's norm work, the next call skips its norm kernel) give the
    unchained calls' results bit for bit: random RMSNorm weights, both gate_up
    tile formats (the fp16 row copy is made for the next layer), fewer tokens
    than experts (workgroups past the tokens only take router-row norms) and a
    decode call, which ignores the chain.  The overlapped prefill chains its
    two chunks' layers too."""
    st = SyntheticMoEStack(layers=3, seed=31, device=dev, max_tokens=512, norm=True,
                           gate_up_format=fmt)
    g = torch.Generator(device=dev)
    g.manual_seed(32)
    st.norm_w.copy_(torch.randn(st.norm_w.shape, generator=g, device=dev) * 0.3)
    h = inputs(tokens, 33, dev)
    plain = st.forward(h.clone(), chain=False)
    chained = st.forward(h.clone(), chain=True)
    assert torch.equal(plain, chained)
    if tokens > 1:  # input_normed only right after a call that chained into the layer
        with pytest.raises(Exception, match='input_normed'):
            st.layer_forward(h.clone(), 1, input_normed=True)  # the last call did not chain
        st.layer_forward(h.clone(), 0, next_layer=1)
        with pytest.raises(Exception, match='input_normed'):
            st.layer_forward(h.clone(), 2, input_normed=True)  # it chained into layer 1
        with pytest.raises(Exception, match='input_normed'):
            st.layer_forward(h[:-1].clone(), 1, input_normed=True)  # other token count
    if tokens > 1:
        two = st.prefill(h, chunk=(tokens + 1) // 2, overlap=True)  # two chained chunks
        assert torch.equal(two, plain)


def test_tile_copy_stale_weights_refused(dev):
    """Writing gu_q or dn_q in place after build_prefill_tiles leaves the
    prefill tile copies stale: the stack refuses to run until they are
    rebuilt, then runs the new weights in both prefill and decode."""
    st = SyntheticMoEStack(layers=1, seed=17, device=dev, max_tokens=64)
    h = inputs(16, 18, dev)
    before, _, _ = run_layer(st, h)
    st.dn_q[0, :, :, :8].neg_()
    with pytest.raises(RuntimeError, match='build_prefill_tiles'):
        run_layer(st, h)
    with pytest.raises(RuntimeError, match='build_prefill_tiles'):
        st.layer_forward_static(h.clone(), 0)
    st.build_prefill_tiles()
    after, ids, _ = run_layer(st, h)
    assert not torch.equal(after, before)
    ref, _ = oracle_layer(st, npf(h), 0, ids.cpu().numpy())
    assert_close(npf(after), ref, BF16_TOL, 'rebuilt tiles')


def _bf16_up(v):
    """The next bf16 value above each element of the bf16 tensor v (finite, nonzero)."""
    bits = v.view(torch.int16).to(torch.int32)
    step = torch.where(v > 0, 1, -1).to(torch.int32)
    return (bits + step).to(torch.int16).view(torch.bfloat16)


@pytest.mark.parametrize('mode', ['near_ties', 'all_equal'])
def test_prefill_router_boundary(dev, mode):
    """Prefill routing stays exact where approximate router logits cannot
    separate experts: 32 router rows that differ from a dominant row by one
    bf16 step in one element (exact logits equal or one bf16 step apart, so
    the 8 winners among them are decided by the exact logits and the id
    order), and all 256 rows equal (every expert is a candidate)."""
    st = SyntheticMoEStack(layers=1, seed=21, device=dev, max_tokens=128)
    w = st.router_w[0].clone()
    if mode == 'near_ties':
        base = (w[5].float() * 3.0).to(torch.bfloat16)
        for i, e in enumerate(range(0, 256, 8)):
            row = base.clone()
            if i:
                k = (i * 37) % 2048
                row[k] = _bf16_up(row[k:k + 1])[0]
            w[e] = row
    else:
        w[:] = w[3]
    st.router_w[0].copy_(w)
    h = inputs(128, 22, dev)
    _, ids, wts = run_layer(st, h)
    xn = O.rmsnorm(npf(h), None, EPS)
    _, rw, ri = O.router(xn, st.layer_host(0, experts=[])['router_w'], 8)
    assert np.array_equal(ids.cpu().numpy(), ri)
    assert np.abs(npf(wts) - rw).max() <= 2.0 ** -8
    if mode == 'all_equal':
        assert (ids.cpu().numpy() == np.arange(8)).all()


def test_fused_prefill_combine_bit_exact(dev):
    """The fused prefill combine (prefill_combine_kernel) on the exact bf16
    inputs it consumed: the down rows, routing weights and route rows the
    call left in its workspace.  Per token, routes in ascending expert id,
    acc = bf16(acc + bf16(v * w)) (prefill.py:37-49), then the gated shared
    expert and the residual, bit for bit.  The shared gate weight is zero, so
    its sigmoid is exactly 0.5 and no transcendental enters the check."""
    st = SyntheticMoEStack(layers=1, seed=51, device=dev, max_tokens=2048)
    st.gate_w.zero_()
    h = inputs(2048, 52, dev)
    out, ids, wts = run_layer(st, h)
    T, R = 2048, 2048 * 8
    v = npf(st.workspace_view('down', T))
    rows = st.workspace_view('route_rows', T).cpu().numpy()
    gate = st.workspace_view('gate', T).cpu().numpy()
    assert (gate == 0).all()
    assert torch.equal(st.workspace_view('ids', T).to(torch.int32), ids)
    assert torch.equal(st.workspace_view('weights', T), wts)
    idn, wn, hn = ids.cpu().numpy(), npf(wts), npf(h)
    # every route has its own row; the routed rows are a permutation of [0, R)
    assert np.array_equal(np.sort(rows.reshape(-1)), np.arange(R))
    for tok in range(T):
        order = np.argsort(idn[tok], kind='stable')
        routed = O.ordered_combine(v[rows[tok, order]], wn[tok, order])
        block = O.bf16(routed + O.bf16(np.float32(0.5) * v[R + tok]))
        assert np.array_equal(npf(out[tok]), O.bf16(hn[tok] + block)), tok


def test_prefill_weights_vs_exact_router(dev, capsys):
    """The fused prefill router selects with exact logits only for the
    experts its error bound leaves open; the softmax denominator sees the
    rounded approximate logits of the others.  On the same normalized rows,
    its ids equal the all-exact router's (lm_router_topk) bit for bit and its
    weights differ by at most one bf16 step; the mismatch rate is reported."""
    st = SyntheticMoEStack(layers=2, seed=53, device=dev, max_tokens=2048)
    total = mismatched = 0
    for l, seed in ((0, 54), (1, 55), (0, 56)):
        h = inputs(2048, seed, dev)
        _, ids, wts = run_layer(st, h, l)
        xn = st.workspace_view('normed', 2048).clone()
        assert torch.equal(xn, router.rmsnorm(h, None, EPS))
        _, ewts, eids = router.router_topk(xn, st.router_w[l], 8)
        assert torch.equal(ids.to(torch.int64), eids)
        a = wts.view(torch.int16).to(torch.int32)
        b = ewts.view(torch.int16).to(torch.int32)
        assert (a - b).abs().max().item() <= 1  # same sign: one bit step = one bf16 ulp
        total += a.numel()
        mismatched += int((a != b).sum())
    rate = mismatched / total
    with capsys.disabled():
        print(f'\n[prefill router] weights differing from the all-exact router: '
              f'{mismatched} of {total} ({rate:.2e})')
    assert rate < 1e-2


@pytest.mark.parametrize('mode', ['random', 'wide_range', 'aligned'])
def test_router_approx_error_bound(dev, capsys, mode):
    """The prefill selection rests on the error of the approximate router
    logits A: each bf16 MFMA sums its 32 exact products from zero and the
    results are added in fp32, so a product passes through at most 49
    roundings and |A - S| <= 49 2^-23 sum_k |x_k w_ek| <= 2^-17 |x| |w_e|.
    Checked on every (token, expert) pair against float64 dot products of
    the same bf16 rows, for random rows, rows whose elements span 2^-40 ..
    2^20 (products of every magnitude inside one MFMA) and rows along one
    router row each (logits near |x| |w_e|, sums of same-sign products).
    The norms the bound uses are checked against float64 norms."""
    T = 512
    st = SyntheticMoEStack(layers=1, seed=61, device=dev, max_tokens=T)
    g = torch.Generator()
    g.manual_seed(62)
    if mode == 'random':
        h = torch.randn(T, 2048, generator=g)
    elif mode == 'wide_range':
        h = torch.randn(T, 2048, generator=g) * torch.exp2(
            torch.randint(-40, 21, (T, 2048), generator=g).float())
    else:
        pick = torch.randint(0, 256, (T,), generator=g)
        sign = torch.where(torch.rand(T, 1, generator=g) < 0.5, -1.0, 1.0)
        h = st.router_w[0].float().cpu()[pick] * sign * 50 + \
            torch.randn(T, 2048, generator=g) * 0.01
    h = h.to(torch.bfloat16).to(dev)
    run_layer(st, h)
    A = st.workspace_view('router_approx', T).double().cpu().numpy()
    nx = st.workspace_view('row_norms', T).double().cpu().numpy()
    nw = st.workspace_view('router_norms', T).double().cpu().numpy()
    xn = st.workspace_view('normed', T).double().cpu().numpy()
    W = st.router_w[0].double().cpu().numpy()
    S = xn @ W.T  # exact products; float64 sums err by < 2^-40 of sum |x w|
    P = np.abs(xn) @ np.abs(W).T
    err = np.abs(A - S)
    model = 49 * 2.0 ** -23 * P * (1 + 2.0 ** -30) + 1e-30
    assert np.isfinite(A).all()
    assert (err <= model).all(), float((err / model).max())
    assert (err <= 2.0 ** -17 * np.outer(nx, nw)).all()
    assert np.allclose(nx, np.sqrt((xn * xn).sum(1)), rtol=1e-6, atol=0)
    assert np.allclose(nw, np.sqrt((W * W).sum(1)), rtol=1e-6, atol=0)
    with capsys.disabled():
        print(f'\n[router bound, {mode}] max |A - S| / (49 2^-23 sum|x w|) = '
              f'{float((err / model).max()):.3e}')


@pytest.mark.parametrize('fmt', [0, 1])
def test_tile_rows_layout(dev, fmt):
    """lm_w8_tile_rows against the index formula of its declaration, on a
    bank whose experts sit further apart than n * k (the stride is kept);
    the fp16 format (1) also biases every byte by 128 and stores the bytes
    of each 4-byte word in the order k = 0, 2, 1, 3."""
    from localmoe35ba3b_amd import _lib
    g = np.random.default_rng(7)
    E, n, k, es = 3, 48, 192, 48 * 192 + 1024
    flat = g.integers(-127, 128, size=E * es).astype(np.int8)
    q = torch.from_numpy(flat).to(dev)
    tiles = torch.zeros_like(q)
    _lib.call('lm_w8_tile_rows', q.data_ptr(), E, n, k, es, tiles.data_ptr(), fmt,
              _lib.stream(dev))
    got = tiles.cpu().numpy()
    ref = np.zeros_like(flat)
    for e in range(E):
        w = flat[e * es:e * es + n * k].reshape(n // 16, 16, k // 64, 4, 16)  # b, r, s, p, j
        t = w.transpose(0, 2, 3, 1, 4).reshape(-1)  # b, s, p, r, j
        if fmt == 1:
            t = (t.view(np.uint8) ^ 0x80).reshape(-1, 4)[:, [0, 2, 1, 3]].reshape(-1).view(np.int8)
        ref[e * es:e * es + n * k] = t
    assert np.array_equal(got, ref)


def f16_gate_up_model(xn, q, s):
    """The fused layer's fp16 gate_up GEMM restated (not a reference
    function): fp16 copies of the rows are exact and the MFMAs multiply them
    by exact q, each group's scale acts on the fp32 sums, so up to fp32
    summation the result is the float64 product with the unrounded weights
    q * s (no bf16 rounding of q * s, unlike int8.py:21), rounded to bf16."""
    w = q.astype(np.float64) * np.repeat(s.astype(np.float64), 128, axis=1)
    return O.bf16((np.asarray(xn, np.float64) @ w.T).astype(np.float32))


def test_prefill_tiles(dev, capsys):
    """The prefill GEMMs on the tile-layout copies.  Plain copies give the
    standard layout's result bit for bit.  The fp16 gate_up GEMM
    (LM_TILES_F16) matches its own arithmetic restated in numpy (unrounded
    q * s) to within a bf16 step or two on a few values, and the reference's
    bf16(q * s) dequantization within the bf16 tolerance; routing is
    unchanged."""
    st = SyntheticMoEStack(layers=1, seed=71, device=dev, max_tokens=2048, prefill_tiles=False)
    h = inputs(2048, 71, dev)
    plain, ids0, w0 = run_layer(st, h)
    plain_h = st.workspace_view('hidden', 2048).clone()
    plain_rows = st.workspace_view('route_rows', 2048).cpu().numpy()  # run-dependent order
    st.build_prefill_tiles(gate_up_format=0)  # both copies plain: bit for bit
    assert torch.equal(run_layer(st, h)[0], plain)
    st.build_prefill_tiles()  # gate_up's copy in the fp16 format (the default)
    tiled, ids1, w1 = run_layer(st, h)
    assert torch.equal(ids0, ids1) and torch.equal(w0, w1)
    assert_close(npf(tiled), npf(plain), BF16_TOL, 'fp16 gate_up layer vs exact')
    # the SwiGLU rows of one expert against both models
    tiled_h = npf(st.workspace_view('hidden', 2048))
    rows = st.workspace_view('route_rows', 2048).cpu().numpy()
    idn = ids1.cpu().numpy()
    e = int(idn[0, 0])
    tok, slot = np.nonzero(idn == e)
    r = rows[tok, slot]
    xn = npf(st.workspace_view('normed', 2048))[tok]
    q, sc = st.gu_q[0, e].cpu().numpy(), st.gu_s[0, e].cpu().numpy()
    model = O.swiglu(f16_gate_up_model(xn, q, sc))
    exact = O.swiglu(O.w8a16_linear(xn, q, sc))
    same = np.sign(tiled_h[r]) * np.sign(model) >= 0
    steps = np.abs(tiled_h[r].view(np.int32) - model.view(np.int32)) // 65536  # bf16 steps
    assert same.mean() > 0.999 and np.median(steps) == 0 and steps[same].max() <= 2, (
        f'{int((~same).sum())} sign flips, steps max {steps[same].max()}')
    # SwiGLU rows are an intermediate: a one-step bf16 difference of a gate
    # value times a large up value can exceed the elementwise bound, so they
    # are held to the norm-wise bound; the layer output above is elementwise.
    rel = np.linalg.norm(tiled_h[r] - exact) / np.linalg.norm(exact)
    r0 = plain_rows[tok, slot]
    rel_plain = np.linalg.norm(npf(plain_h)[r0] - exact) / np.linalg.norm(exact)
    assert rel <= BF16_TOL and rel_plain <= BF16_TOL
    with capsys.disabled():
        print(f'\n[fp16 gate_up] expert {e}, {len(r)} rows: SwiGLU rel err vs exact dequant '
              f'{rel:.2e} (bf16 path {rel_plain:.2e}); vs its fp16 model: '
              f'{int((steps > 0).sum())} of {steps.size} values one bf16 step or more off')
    del st
