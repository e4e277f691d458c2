"""Writes a directory in the converted-checkpoint format of
qwen35_deploy/convert.py:40-118 (manifest.json + one safetensors file per
tensor named sha256(name)[:24]) from given tensors; test infrastructure for
localmoe35ba3b_amd.artifact."""
import json
import pathlib

import torch
from safetensors.torch import save_file

from localmoe35ba3b_amd.artifact import FORMAT, INT8, ORIGINAL, file_sha256, tensor_key


def write_artifact(root, tensors, complete=True):
    """tensors: {name: {'q': int8, 'scale': fp32} | {'weight': tensor}} (CPU)."""
    root = pathlib.Path(root)
    root.mkdir(parents=True, exist_ok=True)
    records = []
    for name in sorted(tensors):
        values = {k: v.detach().cpu().contiguous() for k, v in tensors[name].items()}
        quant = 'q' in values
        path = root / (tensor_key(name) + '.safetensors')
        save_file(values, str(path))
        shape = list((values['q'] if quant else values['weight']).shape)
        records.append({'name': name, 'shape': shape,
                        'dtype': 'BF16', 'shard': 'model.safetensors', 'source_sha256': '0' * 64,
                        'file': path.name, 'sha256': file_sha256(path),
                        'bytes': path.stat().st_size, 'format': INT8 if quant else ORIGINAL,
                        'weight_relative_l2': 0.0, 'quality_validation': 'pending_model_level'})
    manifest = {'identity': {'format': FORMAT, 'source_index_sha256': '0' * 64,
                             'source_config_sha256': '0' * 64, 'source': 'synthetic'},
                'records': records, 'complete': complete,
                'bytes': sum(r['bytes'] for r in records)}
    (root / 'manifest.json').write_text(json.dumps(manifest, indent=2) + '\n')
    return root


def block_tensors(prefix, experts, gate_up, down, shared, router_w, shared_gate_w, norm_w):
    """Checkpoint tensor dict of one MoE layer (names as in the HF checkpoint).
    gate_up/down: {'q','scale'} banks; shared: {'gate_proj'|'up_proj'|'down_proj':
    {'q','scale'} or {'weight'}}."""
    out = {f'{prefix}.mlp.experts.gate_up_proj': gate_up,
           f'{prefix}.mlp.experts.down_proj': down,
           f'{prefix}.mlp.gate.weight': {'weight': router_w},
           f'{prefix}.mlp.shared_expert_gate.weight': {'weight': shared_gate_w},
           f'{prefix}.post_attention_layernorm.weight': {'weight': norm_w}}
    for k, v in shared.items():
        out[f'{prefix}.mlp.shared_expert.{k}.weight'] = v
    return out
