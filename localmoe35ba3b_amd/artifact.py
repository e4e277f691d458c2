"""Reader of the reference's converted INT8 checkpoint into HBM.

The artifact is the directory qwen35_deploy/convert.py:40-118 writes:

  manifest.json   {'identity': {'format': 'q36-w8a16-g128-rtn-fp32scale-v1', ...},
                   'records': [...], 'complete': true, ...}
  <key>.safetensors, key = sha256(tensor name)[:24]  (convert.py:70)

one record per tensor with name, shape, dtype, file, sha256, bytes and
format: 'int8_g128_fp32scale' files hold {'q': int8 [..., K], 'scale': fp32
[..., K/128]} (expert banks stacked per expert, convert.py:85-97), 'original'
files hold {'weight': tensor}.  Checks follow model.py:34-55: the manifest
must be complete, every file must have the recorded size and (with
verify=True) the recorded sha256.

Safetensors files are read with safetensors' own loader, which executes
nothing from the file.
"""
import hashlib
import json
import pathlib

import torch
from safetensors.torch import load_file

from . import _lib
from .convert import quantize_g128

FORMAT = 'q36-w8a16-g128-rtn-fp32scale-v1'
INT8 = 'int8_g128_fp32scale'
ORIGINAL = 'original'


def tensor_key(name):
    """File stem of a tensor in the artifact (convert.py:70)."""
    return hashlib.sha256(name.encode()).hexdigest()[:24]


def file_sha256(path):
    h = hashlib.sha256()
    with open(path, 'rb') as f:
        for block in iter(lambda: f.read(8 << 20), b''):
            h.update(block)
    return h.hexdigest()


def layer_prefix(layer):
    return f'model.language_model.layers.{layer}'


class Artifact:
    """Validated view of a converted checkpoint directory."""

    def __init__(self, root, verify=True):
        self.root = pathlib.Path(root)
        manifest = json.loads((self.root / 'manifest.json').read_text())
        if not manifest.get('complete'):
            raise RuntimeError('Artifact conversion is incomplete')
        if manifest.get('identity', {}).get('format') != FORMAT:
            raise RuntimeError('Unsupported artifact format')
        self.records = {}
        for r in manifest['records']:
            path = self.root / r['file']
            if r['file'] != tensor_key(r['name']) + '.safetensors':
                raise RuntimeError('Artifact file name does not match its tensor: ' + r['name'])
            if not path.exists() or path.stat().st_size != r['bytes']:
                raise RuntimeError('Corrupt artifact: ' + str(path))
            if verify and file_sha256(path) != r['sha256']:
                raise RuntimeError('Corrupt artifact: ' + str(path))
            self.records[r['name']] = r

    def __contains__(self, name):
        return name in self.records

    def load(self, name, device='cpu'):
        """Tensors of one record: {'q', 'scale'} or {'weight'}."""
        r = self.records.get(name)
        if r is None:
            raise KeyError('Tensor missing from artifact: ' + name)
        return load_file(str(self.root / r['file']), device=str(device))

    def quantized(self, name, device):
        """{'q', 'scale'} of a weight on `device`; a tensor stored in its
        original dtype is quantized there with the converter's rule
        (convert.py:31-37), so every linear of the MoE block is int8."""
        data = self.load(name, device)
        if self.records[name]['format'] == INT8:
            return {'q': data['q'].contiguous(), 'scale': data['scale'].float().contiguous()}
        q, s = quantize_g128(data['weight'].to(device))
        return {'q': q, 'scale': s}

    def num_layers(self):
        n = 0
        while f'{layer_prefix(n)}.mlp.experts.gate_up_proj' in self.records:
            n += 1
        return n

    def experts(self, layer, device):
        """(gate_up, down) banks of one layer: gate_up q int8 [E, 2I, H],
        scale fp32 [E, 2I, H/128]; down q int8 [E, H, I], scale [E, H, I/128]."""
        p = f'{layer_prefix(layer)}.mlp.experts'
        gate_up = self.quantized(p + '.gate_up_proj', device)
        down = self.quantized(p + '.down_proj', device)
        e, n2, h = gate_up['q'].shape
        if down['q'].shape != (e, h, n2 // 2):
            raise ValueError('Invalid INT8 group geometry')
        return gate_up, down


def stack_from_artifact(root, device='cuda', layers=None, max_tokens=2048, verify=True,
                        prefill_tiles=True, gate_up_format=_lib.LM_TILES_F16):
    """MoEStack of the fused layer path filled from a converted checkpoint.

    Per layer l: routed experts from mlp.experts.{gate_up_proj, down_proj};
    the shared expert (index E) from mlp.shared_expert.{gate_proj, up_proj}
    (rows concatenated) and .down_proj; router = mlp.gate.weight (bf16),
    shared gate = mlp.shared_expert_gate.weight, RMSNorm weight =
    post_attention_layernorm.weight.  With prefill_tiles the prefill GEMMs
    read a tile-layout copy of the int8 bank, gate_up's in `gate_up_format`
    (MoEStack.build_prefill_tiles).
    """
    from .runtime.stack import MoEStack
    art = Artifact(root, verify=verify)
    total = art.num_layers()
    layers = total if layers is None else layers
    if layers < 1 or layers > total:
        raise ValueError(f'artifact holds {total} MoE layers, {layers} requested')
    st = MoEStack(layers, device=device, max_tokens=max_tokens, norm=True)
    dev = st.device
    E = st.E
    for l in range(layers):
        p = layer_prefix(l)
        gate_up, down = art.experts(l, dev)
        if (tuple(gate_up['q'].shape) != (E, 2 * st.I, st.H)
                or tuple(down['q'].shape) != (E, st.H, st.I)):
            raise ValueError('Unsupported model geometry')
        st.gu_q[l, :E].copy_(gate_up['q'])
        st.gu_s[l, :E].copy_(gate_up['scale'])
        st.dn_q[l, :E].copy_(down['q'])
        st.dn_s[l, :E].copy_(down['scale'])
        gp = art.quantized(p + '.mlp.shared_expert.gate_proj.weight', dev)
        up = art.quantized(p + '.mlp.shared_expert.up_proj.weight', dev)
        dp = art.quantized(p + '.mlp.shared_expert.down_proj.weight', dev)
        st.gu_q[l, E].copy_(torch.cat([gp['q'], up['q']]))
        st.gu_s[l, E].copy_(torch.cat([gp['scale'], up['scale']]))
        st.dn_q[l, E].copy_(dp['q'])
        st.dn_s[l, E].copy_(dp['scale'])
        st.router_w[l].copy_(art.load(p + '.mlp.gate.weight', dev)['weight'].to(torch.bfloat16))
        st.gate_w[l].copy_(art.load(p + '.mlp.shared_expert_gate.weight', dev)['weight']
                           .reshape(-1).to(torch.bfloat16))
        st.norm_w[l].copy_(art.load(p + '.post_attention_layernorm.weight', dev)['weight']
                           .reshape(-1).float())
    if prefill_tiles:
        st.build_prefill_tiles(gate_up_format)
    return st
