"""The headline workload at full size: the synthetic 40-layer MoE-FFN stack
(256 routed experts top-8 + shared expert per layer, ~33.4 GB of int8 group-128
weights resident in HBM), a 4096-token prefill in two 2048-token chunks and
33 serial decode tokens - the inputs and schedule bench.py times (stack seed
4, prompt and decode inputs from the seed-4 device generator).

The reference runs a prompt as consecutive chunks through every layer and
then decodes token by token (generation.py:39-51).  Checked here:
  * routing bit for bit at every layer of both prefill chunks and of all 33
    decode tokens: the GPU's ids equal the oracle router's on the normalized
    rows the GPU computed at that layer (its RMSNorm is bit-exact too);
  * full oracle layer outputs for sampled (layer, token) pairs, prefill
    (W8A16 routed experts) and decode (W8A8 routed experts), routing exact
    and outputs within the bf16 tolerance of tests/conftest.py;
  * the overlapped two-stream prefill captured as one HIP graph (what the
    benchmark replays) equals the serial per-layer run bit for bit, and so
    does every replay of the captured 40-layer decode step.
Each decode token starts from its own seeded N(0,1) row (bench.py's choice).
"""
import time

import numpy as np
import pytest
import torch

from localmoe35ba3b_amd.runtime.stack import EPS, HIDDEN, SyntheticMoEStack
from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(900)]

LAYERS, PROMPT, CHUNK, DECODE = 40, 4096, 2048, 33


def log(msg):
    print(f'[stack40] {msg}', flush=True)


@pytest.fixture(scope='module')
def stack40(dev):
    t0 = time.perf_counter()
    st = SyntheticMoEStack(layers=LAYERS, seed=4, device=dev, max_tokens=CHUNK)
    torch.cuda.synchronize()
    log(f'built {LAYERS} layers, {st.bank_bytes() / 1e9:.2f} GB, {time.perf_counter() - t0:.1f} s')
    yield st
    del st
    torch.cuda.empty_cache()


@pytest.fixture(scope='module')
def workload(dev):
    gen = torch.Generator(device=dev)
    gen.manual_seed(4)
    x = torch.randn((PROMPT, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    dec_in = torch.randn((DECODE, 1, HIDDEN), generator=gen, device=dev).to(torch.bfloat16)
    return x, dec_in


def npf(t):
    return t.detach().float().cpu().numpy()


def router_host(stack):
    return [stack.router_w[l].float().cpu().numpy() for l in range(stack.L)]


def check_layer_output(stack, l, h_in, h_out, ids):
    """Oracle layer on the GPU's input rows; ids exact, output within tolerance."""
    layer = stack.layer_host(l, experts=np.unique(ids))
    ref, (_, _, ri) = O.moe_layer(h_in, layer, k=8, eps=EPS)
    assert np.array_equal(ids, ri), f'layer {l}: routing'
    assert_close(h_out, ref, BF16_TOL, f'layer {l} output')


PREFILL_SAMPLES = {(0, 0), (0, 13), (1, 26), (1, 39)}  # (chunk, layer)


def test_config5_prefill_40_layers(stack40, workload, dev):
    x, _ = workload
    wr = router_host(stack40)
    h = x.clone()
    ids = torch.empty((CHUNK, 8), dtype=torch.int32, device=dev)
    sample = np.random.default_rng(5).choice(CHUNK, 4, replace=False)
    sample[0] = CHUNK - 1
    routes_checked = 0
    for c in range(PROMPT // CHUNK):
        hc = h[c * CHUNK:(c + 1) * CHUNK]
        for l in range(LAYERS):
            h_in = npf(hc) if (c, l) in PREFILL_SAMPLES else None
            stack40.layer_forward(hc, l, ids)
            xn = npf(stack40.workspace_view('normed', CHUNK))
            if h_in is not None:  # the router input is the oracle's RMSNorm, bit for bit
                assert np.array_equal(xn, O.rmsnorm(h_in, None, EPS))
            _, _, ri = O.router(xn, wr[l], 8)
            got = ids.cpu().numpy()
            assert np.array_equal(got, ri), f'chunk {c} layer {l}: routing differs'
            routes_checked += got.size
            if h_in is not None:
                check_layer_output(stack40, l, h_in[sample], npf(hc[sample]), got[sample])
            if l % 10 == 9:
                log(f'prefill chunk {c}: layers 0..{l} routing exact')
    log(f'prefill: {routes_checked} routes bit-exact over {LAYERS} layers x 2 chunks')
    # the benchmark's schedule: both chunks overlapped on two streams, captured
    # once as a HIP graph and replayed, with eager work between replays
    static = x.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack40.prefill_(static.clone(), CHUNK)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack40.prefill_(static, CHUNK)
    for i in range(2):
        static.copy_(x)
        graph.replay()
        torch.cuda.synchronize()
        other = x[:CHUNK].clone()
        stack40.layer_forward(other, i)  # eager work between replays
        torch.cuda.synchronize()
        assert torch.equal(static, h), f'graph replay {i} differs from the serial run'
    log('overlapped graph prefill equals the serial run')


DECODE_SAMPLES = {(0, 0), (11, 17), (22, 30), (32, 39)}  # (token, layer)


def test_config5_decode_33_tokens(stack40, workload, dev):
    _, dec_in = workload
    wr = router_host(stack40)
    ids = torch.empty((1, 8), dtype=torch.int32, device=dev)
    finals = []
    for i in range(DECODE):
        h = dec_in[i].clone()
        for l in range(LAYERS):
            h_in = npf(h) if (i, l) in DECODE_SAMPLES else None
            stack40.layer_forward(h, l, ids)
            xn = npf(stack40.workspace_view('normed', 1))
            _, _, ri = O.router(xn, wr[l], 8)
            got = ids.cpu().numpy()
            assert np.array_equal(got, ri), f'decode token {i} layer {l}: routing differs'
            if h_in is not None:
                assert np.array_equal(xn, O.rmsnorm(h_in, None, EPS))
                check_layer_output(stack40, l, h_in, npf(h), got)
        finals.append(h)
        if i % 8 == 7:
            log(f'decode tokens 0..{i}: routing exact at all {LAYERS} layers')
    log(f'decode: {DECODE * LAYERS} token-layers, routing bit-exact')
    # the benchmark's decode step: the 40 layers captured once as a HIP graph
    static = dec_in[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        stack40.forward(static.clone())
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stack40.forward(static)
    for i in range(DECODE):
        static.copy_(dec_in[i])
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static, finals[i]), f'graph replay of token {i} differs'
    log('graph-replayed decode equals the eager run for all 33 tokens')
