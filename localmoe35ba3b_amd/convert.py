"""Group-128 int8 weight quantizer (the format producer of qwen35_deploy/convert.py:31-37).

s = max(amax_g|w| / 127, 1e-30) per 128-wide K group (IEEE division),
q = clamp(round_half_even(w / s), -127, 127) as int8 - computed by the
lm_quantize_weight_g128 HIP kernel.
"""
import torch

from . import _lib


def quantize_g128(w):
    """Device quantizer: fp32/bf16 CUDA w [..., K] -> (q int8 [..., K], s fp32 [..., K/128])."""
    if not w.is_cuda:
        raise ValueError('quantize_g128 expects a CUDA tensor')
    k = w.shape[-1]
    if k % 128:
        raise ValueError('Invalid INT8 group geometry')
    v = w.float().contiguous()
    rows = v.numel() // k
    q = torch.empty(v.shape, dtype=torch.int8, device=w.device)
    s = torch.empty((*v.shape[:-1], k // 128), dtype=torch.float32, device=w.device)
    _lib.call('lm_quantize_weight_g128', v.data_ptr(), q.data_ptr(), s.data_ptr(), rows, k,
              _lib.stream(w.device))
    return q, s


def quantize(w):
    """Reference-compatible converter call: (q cpu, scale cpu, squared error, energy).

    w must be a CUDA tensor (the reference converter quantizes on the GPU,
    convert.py:91-95).  Error and energy are fp64 sums over the group view.
    """
    shape = w.shape
    q, scale = quantize_g128(w)
    v = w.float().reshape(*shape[:-1], shape[-1] // 128, 128)
    err = (q.reshape(v.shape).float() * scale.unsqueeze(-1) - v).double()
    return (q.reshape(shape).cpu(), scale.cpu(), float(err.square().sum()),
            float(v.double().square().sum()))
