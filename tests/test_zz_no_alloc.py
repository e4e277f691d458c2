"""The allocation-free fused layer (lm_moe_layer_forward_static) against the
workspace entry point (lm_moe_layer_forward) it shares kernels with.

The static variant keeps its workspace in the library's own device array,
which keeps the previous call's contents: two calls in a row with the second
on fewer tokens (128 then 37 prefill tokens, then one decode token) must
each equal the workspace path bit for bit - output rows, routing ids and
routing weights - and a call beyond the array's token limit is refused before
anything is launched.
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
