"""The allocation-free fused layer (lm_moe_layer_forward_static) against the
workspace entry point (lm_moe_layer_forward) it shares kernels with.

The static variant keeps its workspace in the library's own device array,
which keeps the previous call's contents: two calls in a row with the second
on fewer tokens (128 then 37 prefill tokens, then one decode token) must
each equal the workspace path bit for bit - output rows, routing ids and
routing weights - and a call beyond the array's token limit is refused before
anything is launched.  Static calls allocate nothing (device free memory and
torch's allocator unchanged) and can be captured in a HIP graph once the
array is resolved (lm_moe_static_init, which the stack's wrapper calls on
first use, outside any capture).
"""
import pytest
import torch

from localmoe35ba3b_amd import _lib
from localmoe35ba3b_amd.runtime.stack import SyntheticMoEStack

pytestmark = pytest.mark.gpu


def inputs(tokens, seed, dev):
    g = torch.Generator()
    g.manual_seed(seed)
    return torch.randn(tokens, 2048, generator=g).to(torch.bfloat16).to(dev)


def test_static_scratch_matches_workspace_path(dev):
    limit = _lib.lib().lm_moe_static_max_tokens()
    assert limit == 128
    st = SyntheticMoEStack(layers=2, seed=61, device=dev, max_tokens=limit)
    for i, tokens in enumerate((limit, 37, 1)):
        h = inputs(tokens, 70 + i, dev)
        for l in range(2):
            ref, got = h.clone(), h.clone()
            ids_r = torch.empty((tokens, 8), dtype=torch.int32, device=dev)
            ids_g = torch.full_like(ids_r, -1)
            w_r = torch.empty((tokens, 8), dtype=torch.bfloat16, device=dev)
            w_g = torch.zeros_like(w_r)
            st.layer_forward(ref, l, ids_r, w_r)
            st.layer_forward_static(got, l, ids_g, w_g)
            torch.cuda.synchronize()
            assert torch.equal(got, ref), f'{tokens} tokens, layer {l}: output'
            assert torch.equal(ids_g, ids_r), f'{tokens} tokens, layer {l}: ids'
            assert torch.equal(w_g, w_r), f'{tokens} tokens, layer {l}: weights'
    h = inputs(limit + 1, 80, dev)
    before = h.clone()
    with pytest.raises(MemoryError, match='static scratch'):
        st.layer_forward_static(h, 0)
    torch.cuda.synchronize()
    assert torch.equal(h, before)


def test_static_calls_allocate_nothing_and_capture(dev):
    """Static calls leave the device's free memory and torch's allocator
    untouched, and captured in a HIP graph (37 prefill tokens through both
    layers, then one decode token) every replay equals the eager calls, with
    other static calls between the replays."""
    st = SyntheticMoEStack(layers=2, seed=62, device=dev, max_tokens=64)
    h37, h1 = inputs(37, 90, dev), inputs(1, 91, dev)
    ref37, ref1 = h37.clone(), h1.clone()
    for l in range(2):
        st.layer_forward(ref37, l)
        st.layer_forward(ref1, l)
    work = [h37.clone(), h1.clone(), inputs(5, 92, dev)]
    st.layer_forward_static(inputs(3, 94, dev), 0)  # first use: resolves the array
    torch.cuda.synchronize()
    free0, alloc0 = torch.cuda.mem_get_info(dev)[0], torch.cuda.memory_allocated(dev)
    for _ in range(3):
        for x in work:
            for l in range(2):
                st.layer_forward_static(x, l)
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info(dev)[0] == free0
    assert torch.cuda.memory_allocated(dev) == alloc0
    s37, s1 = h37.clone(), h1.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for l in range(2):
            st.layer_forward_static(s37, l)
        for l in range(2):
            st.layer_forward_static(s1, l)
    for i in range(3):
        s37.copy_(h37)
        s1.copy_(h1)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(s37, ref37), f'replay {i}: 37 tokens'
        assert torch.equal(s1, ref1), f'replay {i}: 1 token'
        other = inputs(9, 93 + i, dev)
        st.layer_forward_static(other, i % 2)  # eager static work between replays
        torch.cuda.synchronize()
