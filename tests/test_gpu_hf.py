"""GPU tests of the Transformers drop-in and the converted-checkpoint loader.

* A Transformers Qwen3_5MoeSparseMoeBlock whose experts and shared-expert
  linears are swapped (hf.install, reading a converted artifact) matches the
  same block running HF's eager expert loop on the dequantized weights
  bf16(q * s) - the reference's dequantize-then-matmul path - within the
  bf16 tolerance, for prefill (grouped GEMM) and decode (W8A16 and, after
  the module-global swap of cli.py:37-39, W8A8).  Both blocks share HF's
  router, so routing is identical.  The comparison runs HF's own module on
  the GPU; it uses only 2-D products (no batched matmul).
* A stack loaded from an artifact written from a synthetic stack reproduces
  that stack's layer outputs and routing bit for bit (decode and prefill).
"""
import copy

import numpy as np
import pytest
import torch

from localmoe35ba3b_amd import artifact as A
from localmoe35ba3b_amd.convert import quantize_g128
from localmoe35ba3b_amd.hf import install
from localmoe35ba3b_amd.operators import int8, w8a8
from localmoe35ba3b_amd.operators.int8 import Int8Experts, Int8Linear
from localmoe35ba3b_amd.runtime.stack import SyntheticMoEStack
from tests.artifact_util import block_tensors, write_artifact
from tests.conftest import BF16_TOL, assert_close

pytestmark = pytest.mark.gpu


def small_config():
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    return Qwen3_5MoeTextConfig(hidden_size=256, num_experts=16, num_experts_per_tok=4,
                                moe_intermediate_size=128, shared_expert_intermediate_size=128,
                                num_hidden_layers=1, vocab_size=512,
                                experts_implementation='eager')


class Holder(torch.nn.Module):
    """model.language_model.layers[0].mlp = block: checkpoint naming."""

    def __init__(self, block):
        super().__init__()
        self.model = torch.nn.Module()
        self.model.language_model = torch.nn.Module()
        layer = torch.nn.Module()
        layer.mlp = block
        self.model.language_model.layers = torch.nn.ModuleList([layer])


def dequant(bank):
    q, s = bank['q'], bank['scale']
    w = q.float().reshape(*q.shape[:-1], -1, 128) * s.unsqueeze(-1)
    return w.reshape(q.shape).to(torch.bfloat16)


@pytest.fixture(scope='module')
def blocks(dev, tmp_path_factory):
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeSparseMoeBlock
    torch.manual_seed(0)
    master = Qwen3_5MoeSparseMoeBlock(small_config()).to(dev)
    with torch.no_grad():
        for p in master.parameters():
            p.normal_(0.0, 0.02)
    banks = {'gate_up': quantize_g128(master.experts.gate_up_proj.float()),
             'down': quantize_g128(master.experts.down_proj.float())}
    banks = {k: {'q': v[0], 'scale': v[1]} for k, v in banks.items()}
    shared = {n: dict(zip(('q', 'scale'),
                          quantize_g128(getattr(master.shared_expert, n).weight.float())))
              for n in ('gate_proj', 'up_proj', 'down_proj')}
    # reference block: HF eager on bf16(q * s)
    ref = copy.deepcopy(master).to(torch.bfloat16)
    with torch.no_grad():
        ref.experts.gate_up_proj.copy_(dequant(banks['gate_up']))
        ref.experts.down_proj.copy_(dequant(banks['down']))
        for n, b in shared.items():
            getattr(ref.shared_expert, n).weight.copy_(dequant(b))
    prefix = A.layer_prefix(0)
    tensors = block_tensors(prefix, 16, banks['gate_up'], banks['down'], shared,
                            ref.gate.weight, ref.shared_expert_gate.weight,
                            torch.zeros(256, dtype=torch.bfloat16))
    root = write_artifact(tmp_path_factory.mktemp('artifact'), tensors)
    ours = Holder(copy.deepcopy(ref))
    plan = install(ours, artifact=A.Artifact(root), device=dev, min_dim=128)
    assert dict(plan) == {f'{prefix}.mlp.experts': 'experts',
                          f'{prefix}.mlp.shared_expert.gate_proj': 'linear',
                          f'{prefix}.mlp.shared_expert.up_proj': 'linear',
                          f'{prefix}.mlp.shared_expert.down_proj': 'linear'}
    block = ours.model.language_model.layers[0].mlp
    assert isinstance(block.experts, Int8Experts)
    assert isinstance(block.shared_expert.down_proj, Int8Linear)
    return ref, block


def hidden(tokens, seed, dev):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, tokens, 256, generator=g).to(torch.bfloat16).to(dev)


@pytest.mark.parametrize('tokens', [1, 37, 300])
def test_sparse_moe_block_drop_in(blocks, dev, tokens):
    ref, ours = blocks
    x = hidden(tokens, tokens, dev)
    with torch.no_grad():
        want = ref(x)
        got = ours(x)
    torch.cuda.synchronize()
    assert got.shape == want.shape and got.dtype == torch.bfloat16
    assert_close(got.float().cpu().numpy(), want.float().cpu().numpy(), BF16_TOL,
                 f'drop-in block, {tokens} tokens')


def test_sparse_moe_block_w8a8_decode_swap(blocks, dev):
    """cli.py:37-39 swaps int8.grouped_linear for w8a8.grouped_linear; the
    decode experts then run W8A8 (per-token activation quantization)."""
    ref, ours = blocks
    x = hidden(1, 5, dev)
    saved = int8.grouped_linear
    int8.grouped_linear = w8a8.grouped_linear
    try:
        with torch.no_grad():
            got = ours(x)
            want = ref(x)
    finally:
        int8.grouped_linear = saved
    # W8A8 adds the activation quantization error (<= 1/254 of each group max)
    assert_close(got.float().cpu().numpy(), want.float().cpu().numpy(), 3 * BF16_TOL,
                 'drop-in block, W8A8 decode')


def test_stack_from_artifact_matches_synthetic(dev, tmp_path):
    st = SyntheticMoEStack(layers=1, seed=31, device=dev, max_tokens=64)
    E, I = st.E, st.I
    q_s = lambda q, s: {'q': q.cpu(), 'scale': s.cpu()}
    tensors = block_tensors(
        A.layer_prefix(0), E, q_s(st.gu_q[0, :E], st.gu_s[0, :E]),
        q_s(st.dn_q[0, :E], st.dn_s[0, :E]),
        {'gate_proj': q_s(st.gu_q[0, E, :I], st.gu_s[0, E, :I]),
         'up_proj': q_s(st.gu_q[0, E, I:], st.gu_s[0, E, I:]),
         'down_proj': q_s(st.dn_q[0, E], st.dn_s[0, E])},
        st.router_w[0].cpu(), st.gate_w[0].reshape(1, -1).cpu(),
        torch.zeros(st.H, dtype=torch.bfloat16))
    root = write_artifact(tmp_path, tensors)
    del tensors
    st2 = A.stack_from_artifact(root, device=dev, max_tokens=64)
    assert st2.L == 1 and st2.bank_bytes() > st.bank_bytes()  # + the norm weights
    for tokens in (1, 40):
        g = torch.Generator().manual_seed(tokens)
        h = torch.randn(tokens, 2048, generator=g).to(torch.bfloat16).to(dev)
        outs = []
        for s in (st, st2):
            ids = torch.empty((tokens, 8), dtype=torch.int32, device=dev)
            out = h.clone()
            s.layer_forward(out, 0, ids)
            outs.append((out, ids))
        torch.cuda.synchronize()
        assert torch.equal(outs[0][1], outs[1][1])
        assert torch.equal(outs[0][0], outs[1][0])
