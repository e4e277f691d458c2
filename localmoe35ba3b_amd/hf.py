"""Installs the HIP operators into a Transformers Qwen3_5Moe model.

The reference swaps modules in place (qwen35_deploy/model.py:16-18, 57-71):
every Qwen3_5MoeExperts becomes an Int8Experts over the layer's int8 bank and
every selected nn.Linear an Int8Linear; the router (Qwen3_5MoeTopKRouter),
shared_expert_gate, norms and token mixers stay as they are.  install() does
the same over an HBM-resident bank.  Weights come from a converted artifact
(artifact.Artifact) when one is given, else the module's own weights are
quantized on the GPU with the converter's rule (convert.py:31-37).

Selection rule (convert.py:79-81): expert banks, and 2-D weights whose
smaller dimension is at least 512 and whose K is a multiple of 128, except
token embeddings.
"""
import re

import torch

from .convert import quantize_g128
from .operators.int8 import Int8Experts, Int8Linear

QUANT_MIN_DIM = 512
_LAYER = re.compile(r'layers\.(\d+)\.mlp\.experts$')


def selected_for_int8(name, shape, min_dim=QUANT_MIN_DIM):
    """convert.py:79-81 for a checkpoint tensor `name` of `shape`."""
    expert = '.mlp.experts.' in name
    return bool((expert or (len(shape) == 2 and min(shape) >= min_dim))
                and 'embed_tokens' not in name and shape[-1] % 128 == 0)


def _is_experts(module):
    return (hasattr(module, 'gate_up_proj') and hasattr(module, 'down_proj')
            and isinstance(getattr(module, 'gate_up_proj'), torch.nn.Parameter)
            and getattr(module, 'gate_up_proj').ndim == 3)


def plan_install(model, min_dim=QUANT_MIN_DIM):
    """[(module name, 'experts' | 'linear')] that install() would swap."""
    plan = []
    for name, module in model.named_modules():
        if _is_experts(module) and _LAYER.search(name):
            plan.append((name, 'experts'))
        elif isinstance(module, torch.nn.Linear) and module.bias is None and selected_for_int8(
                name + '.weight', tuple(module.weight.shape), min_dim):
            plan.append((name, 'linear'))
    return plan


def _replace(model, name, module):
    parent, _, child = name.rpartition('.')
    setattr(model.get_submodule(parent) if parent else model, child, module)


def _own_weights(module, device):
    q, s = quantize_g128(module.detach().to(device=device, dtype=torch.float32))
    return {'q': q, 'scale': s}


def install(model, artifact=None, device='cuda', min_dim=QUANT_MIN_DIM, checkpoint_name=None):
    """Swaps the selected modules of `model` in place; returns the plan.

    checkpoint_name maps a module name to the artifact's tensor prefix
    (default: identity, i.e. the model is named like the checkpoint, e.g.
    Qwen3_5MoeForConditionalGeneration).
    """
    device = torch.device(device)
    to_ckpt = checkpoint_name or (lambda n: n)
    plan = plan_install(model, min_dim)
    for name, kind in plan:
        module = model.get_submodule(name)
        if kind == 'experts':
            layer = int(_LAYER.search(name).group(1))
            if artifact is not None:
                gate_up, down = artifact.experts(layer, device)
            else:
                gate_up = _own_weights(module.gate_up_proj, device)
                down = _own_weights(module.down_proj, device)
            _replace(model, name, Int8Experts(layer, gate_up, down))
        else:
            if artifact is not None:
                bank = artifact.quantized(to_ckpt(name) + '.weight', device)
            else:
                bank = _own_weights(module.weight, device)
            _replace(model, name, Int8Linear(bank['q'], bank['scale']))
    return plan
