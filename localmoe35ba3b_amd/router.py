"""Top-k router of the MoE block (HF Qwen3_5MoeTopKRouter.forward, HF:768-776).

Logits are bf16-rounded fp64-accumulated dot products (order-independent,
hence reproducible bit for bit); the top-k rule is (logit desc, expert id asc);
weights are the fp32 softmax renormalised over the selected experts, cast to
bf16.  An optional fp32 per-expert bias is added to the logits before the
softmax (the skewed-popularity benchmark input).
"""
import torch

from . import _lib


def router_topk(hidden, weight, top_k, bias=None):
    """Returns (logits fp32 [T, E], weights bf16 [T, top_k], ids int64 [T, top_k]).

    hidden bf16 [T, H]; weight bf16 [E, H]; bias fp32 [E] or None.  ids are
    in selection order (largest logit first), like torch.topk.
    """
    hidden = hidden.reshape(-1, hidden.shape[-1]).contiguous()
    if not hidden.is_cuda or hidden.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError('router expects CUDA bf16 hidden states and weights')
    tokens, h = hidden.shape
    experts = weight.shape[0]
    if weight.shape[1] != h:
        raise ValueError('router weight does not match the hidden size')
    dev = hidden.device
    logits = torch.empty((tokens, experts), dtype=torch.float32, device=dev)
    ids = torch.empty((tokens, top_k), dtype=torch.int64, device=dev)
    weights = torch.empty((tokens, top_k), dtype=torch.bfloat16, device=dev)
    if bias is not None:
        bias = bias.to(device=dev, dtype=torch.float32).contiguous()
    _lib.call('lm_router_topk', hidden.data_ptr(), weight.contiguous().data_ptr(), _lib.ptr(bias),
              logits.data_ptr(), ids.data_ptr(), weights.data_ptr(), tokens, experts, h, top_k,
              _lib.stream(dev))
    return logits, weights, ids


def rmsnorm(x, weight=None, eps=1e-6):
    """Qwen3_5MoeRMSNorm (HF:801-815): bf16(x * rsqrt(mean(x^2) + eps) * (1 + w))."""
    x = x.contiguous()
    out = torch.empty_like(x)
    n = x.shape[-1]
    if weight is not None:
        weight = weight.to(device=x.device, dtype=torch.float32).contiguous()
    _lib.call('lm_rmsnorm', x.data_ptr(), _lib.ptr(weight), out.data_ptr(), x.numel() // n, n,
              float(eps), _lib.stream(x.device))
    return out
