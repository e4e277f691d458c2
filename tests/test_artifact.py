"""Converted-checkpoint reader and HF module selection, on the CPU.

The reader follows the artifact format of qwen35_deploy/convert.py:40-118
and the checks of qwen35_deploy/model.py:34-55; the selection rule is
convert.py:79-81.  GPU loading and the module swap itself are covered by
tests/test_gpu_hf.py.
"""
import hashlib
import json

import pytest
import torch

from localmoe35ba3b_amd import artifact as A
from localmoe35ba3b_amd.hf import plan_install, selected_for_int8
from tests.artifact_util import block_tensors, write_artifact


def small_layer(prefix, seed, e=4, h=256, i=128):
    g = torch.Generator().manual_seed(seed)
    q = lambda *s: torch.randint(-127, 128, s, generator=g, dtype=torch.int8)
    sc = lambda *s: torch.rand(s, generator=g) * 1e-3
    return block_tensors(prefix, e,
                         {'q': q(e, 2 * i, h), 'scale': sc(e, 2 * i, h // 128)},
                         {'q': q(e, h, i), 'scale': sc(e, h, i // 128)},
                         {'gate_proj': {'q': q(i, h), 'scale': sc(i, h // 128)},
                          'up_proj': {'weight': torch.randn(i, h, generator=g).to(torch.bfloat16)},
                          'down_proj': {'q': q(h, i), 'scale': sc(h, i // 128)}},
                         torch.randn(e, h, generator=g).to(torch.bfloat16),
                         torch.randn(1, h, generator=g).to(torch.bfloat16),
                         torch.randn(h, generator=g).to(torch.bfloat16))


def test_tensor_key_is_sha256_prefix():
    name = 'model.language_model.layers.3.mlp.experts.down_proj'
    assert A.tensor_key(name) == hashlib.sha256(name.encode()).hexdigest()[:24]
    assert len(A.tensor_key(name)) == 24


def test_artifact_round_trip(tmp_path):
    t = {**small_layer(A.layer_prefix(0), 1), **small_layer(A.layer_prefix(1), 2)}
    write_artifact(tmp_path, t)
    art = A.Artifact(tmp_path)
    assert art.num_layers() == 2
    for name, values in t.items():
        got = art.load(name)
        assert set(got) == set(values)
        for k in values:
            assert torch.equal(got[k], values[k])


def test_artifact_rejects_corruption(tmp_path):
    t = small_layer(A.layer_prefix(0), 3)
    write_artifact(tmp_path, t)
    name = A.layer_prefix(0) + '.mlp.experts.down_proj'
    path = tmp_path / (A.tensor_key(name) + '.safetensors')
    data = bytearray(path.read_bytes())
    data[-1] ^= 0xFF  # same size, different content
    path.write_bytes(bytes(data))
    with pytest.raises(RuntimeError, match='Corrupt artifact'):
        A.Artifact(tmp_path)
    A.Artifact(tmp_path, verify=False)  # size still matches
    path.write_bytes(bytes(data[:-1]))
    with pytest.raises(RuntimeError, match='Corrupt artifact'):
        A.Artifact(tmp_path, verify=False)


def test_artifact_rejects_incomplete_or_foreign(tmp_path):
    write_artifact(tmp_path / 'a', small_layer(A.layer_prefix(0), 4), complete=False)
    with pytest.raises(RuntimeError, match='incomplete'):
        A.Artifact(tmp_path / 'a')
    root = write_artifact(tmp_path / 'b', small_layer(A.layer_prefix(0), 5))
    m = json.loads((root / 'manifest.json').read_text())
    m['identity']['format'] = 'something-else'
    (root / 'manifest.json').write_text(json.dumps(m))
    with pytest.raises(RuntimeError, match='Unsupported artifact format'):
        A.Artifact(root)
    good = A.Artifact(write_artifact(tmp_path / 'c', small_layer(A.layer_prefix(0), 6)))
    with pytest.raises(KeyError):
        good.load('missing.weight')


@pytest.mark.parametrize('name,shape,want', [
    ('model.language_model.layers.0.mlp.experts.gate_up_proj', (256, 1024, 2048), True),
    ('model.language_model.layers.0.mlp.shared_expert.down_proj.weight', (2048, 512), True),
    ('model.language_model.layers.0.mlp.gate.weight', (256, 2048), False),       # min 256
    ('model.language_model.layers.0.mlp.shared_expert_gate.weight', (1, 2048), False),
    ('model.language_model.embed_tokens.weight', (248320, 2048), False),
    ('lm_head.weight', (248320, 2048), True),
    ('model.language_model.layers.0.linear_attn.A_log', (32,), False),
    ('model.language_model.layers.0.self_attn.o_proj.weight', (2048, 4000), False),  # K % 128
])
def test_selection_rule(name, shape, want):
    assert selected_for_int8(name, shape) == want


def test_plan_install_on_hf_model():
    from transformers.models.qwen3_5_moe.configuration_qwen3_5_moe import Qwen3_5MoeTextConfig
    from transformers.models.qwen3_5_moe.modeling_qwen3_5_moe import Qwen3_5MoeForCausalLM
    cfg = Qwen3_5MoeTextConfig(hidden_size=256, num_experts=16, num_experts_per_tok=4,
                               moe_intermediate_size=128, shared_expert_intermediate_size=128,
                               num_hidden_layers=2, vocab_size=512, num_attention_heads=4,
                               num_key_value_heads=2, head_dim=64, linear_num_key_heads=2,
                               linear_num_value_heads=4, linear_key_head_dim=32,
                               linear_value_head_dim=32,
                               layer_types=['linear_attention', 'full_attention'])
    model = Qwen3_5MoeForCausalLM(cfg)
    plan = dict(plan_install(model, min_dim=128))
    assert plan['model.layers.0.mlp.experts'] == 'experts'
    assert plan['model.layers.1.mlp.shared_expert.down_proj'] == 'linear'
    assert plan['lm_head'] == 'linear'
    assert 'model.layers.0.mlp.gate' not in plan           # router stays bf16
    assert 'model.layers.0.mlp.shared_expert_gate' not in plan
    assert not any('embed_tokens' in n for n in plan)
    # with the converter's 512 threshold only the expert banks of this small
    # model qualify
    assert set(dict(plan_install(model)).values()) == {'experts'}
