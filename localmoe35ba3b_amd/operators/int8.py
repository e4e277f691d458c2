"""W8A16 group-128 operators and the HBM-resident expert dispatcher.

Drop-in for qwen35_deploy/operators/int8.py: same names, argument meaning and
error text.  The arithmetic runs in gfx950 HIP kernels (gemv.hip, gemm.hip,
route.hip) reached through the C ABI; there is no host or PyTorch fallback.

The reference's byte-budgeted host expert cache (ExpertCache, int8.py:51-124)
has no counterpart: the whole expert bank is resident in HBM, so an
Int8Experts module holds device tensors and builds its decode descriptor
table on the device without a host synchronisation.
"""
import torch

from .. import _lib
from . import w8a8 as _w8a8  # noqa: F401  (module-global swap target, cli.py:37-39)


def _require_int8_pair(q, scale):
    if q.dtype != torch.int8 or scale.dtype != torch.float32:
        raise ValueError('Invalid INT8 group geometry')
    if not (q.is_cuda and scale.is_cuda):
        raise ValueError('Invalid INT8 group geometry')
    if not (q.is_contiguous() and scale.is_contiguous()):
        raise ValueError('Invalid INT8 group geometry')


def linear(x, q, scale, large_tile=False):
    """y = x . bf16(q * s)^T with fp32 accumulation (int8.py:26-37).

    x: CUDA bf16/fp16 [..., K]; q int8 [N, K]; scale fp32 [N, K/128].
    M <= 8 rows run the HBM-streaming GEMV, larger M the MFMA GEMM;
    large_tile selects the taller MFMA tile like the reference flag.
    """
    if not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError('W8A16 requires CUDA FP16/BF16 activations')
    n, k = q.shape
    if k % 128 or x.shape[-1] != k or tuple(scale.shape) != (n, k // 128):
        raise ValueError('Invalid INT8 group geometry')
    _require_int8_pair(q, scale)
    x = x.contiguous()
    m = x.numel() // k
    out = torch.empty((*x.shape[:-1], n), device=x.device, dtype=x.dtype)
    _lib.call('lm_w8a16_linear', x.data_ptr(), q.data_ptr(), scale.data_ptr(), out.data_ptr(),
              m, n, k, _lib.dtype_code(x.dtype), int(bool(large_tile)), _lib.stream(x.device))
    return out


class Int8Linear(torch.nn.Module):
    """nn.Linear replacement holding int8 weights and fp32 group scales (int8.py:40-48)."""

    def __init__(self, q, scale):
        super().__init__()
        self.register_buffer('q', q)
        self.register_buffer('scale', scale)
        self.large_prefill_tile = False

    def forward(self, x):
        return linear(x, self.q, self.scale, self.large_prefill_tile)


def grouped_linear(x, table, experts, n, field, shared):
    """W8A16 grouped decode GEMV over a device descriptor table (int8.py:233-237).

    table: CUDA int64 [experts, 5] = [gate_up.q, gate_up.s, down.q, down.s, slot]
    data pointers; row e reads x row 0 if shared else row e.
    """
    if not x.is_cuda or x.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError('W8A16 requires CUDA FP16/BF16 activations')
    x = x.contiguous()
    out = torch.empty((experts, n), dtype=x.dtype, device=x.device)
    _lib.call('lm_w8a16_grouped_gemv', x.data_ptr(), table.data_ptr(), out.data_ptr(),
              experts, n, x.shape[-1], field, int(bool(shared)), _lib.dtype_code(x.dtype),
              _lib.stream(x.device))
    return out


def ordered_reduce(values, table, weights, out=None):
    """Decode combine (int8.py:240-250): acc = T(acc + T(v_e * w[slot_e])).

    values [E_sel, N] (bf16 or fp16, T) in ascending-expert table order;
    weights [1, top_k] (bf16, fp16 or fp32); returns [1, N] in T.
    """
    experts, n = values.shape
    if out is None:
        out = torch.empty((1, n), dtype=values.dtype, device=values.device)
    weights = weights.contiguous()
    _lib.call('lm_ordered_reduce', values.contiguous().data_ptr(), table.data_ptr(),
              weights.data_ptr(), _lib.dtype_code(weights.dtype), out.data_ptr(), n, experts,
              _lib.dtype_code(values.dtype), _lib.stream(values.device))
    return out


def swiglu(gu):
    """T(T(silu(gate)) * up) over the two halves of the last dim, T = gu.dtype."""
    gu = gu.contiguous()
    half = gu.shape[-1] // 2
    out = torch.empty((*gu.shape[:-1], half), dtype=gu.dtype, device=gu.device)
    _lib.call('lm_swiglu', gu.data_ptr(), out.data_ptr(), gu.numel() // gu.shape[-1], half,
              _lib.dtype_code(gu.dtype), _lib.stream(gu.device))
    return out


def build_descriptors(gate_up, down, ids):
    """Decode descriptor table for one token, sorted by expert id (int8.py:164-179).

    Returns a CUDA int64 [top_k, 5] table of (gate_up.q, gate_up.s, down.q,
    down.s) data pointers of each selected expert of the HBM bank plus its
    slot, built on the device (no host read of the routing ids).
    """
    flat = ids.reshape(-1)
    experts, slots = torch.sort(flat, stable=True)
    bases = torch.tensor([gate_up['q'].data_ptr(), gate_up['scale'].data_ptr(),
                          down['q'].data_ptr(), down['scale'].data_ptr()],
                         dtype=torch.int64, device=ids.device)
    strides = torch.tensor([gate_up['q'].stride(0), gate_up['scale'].stride(0) * 4,
                            down['q'].stride(0), down['scale'].stride(0) * 4],
                           dtype=torch.int64, device=ids.device)
    ptrs = bases[None, :] + experts.to(torch.int64)[:, None] * strides[None, :]
    return torch.cat([ptrs, slots.to(torch.int64)[:, None]], dim=1).contiguous()


class Int8Experts(torch.nn.Module):
    """HF Qwen3_5MoeExperts replacement over an HBM-resident int8 bank (int8.py:127-210).

    gate_up = {'q': int8 [E, 2I, H], 'scale': fp32 [E, 2I, H/128]} and
    down = {'q': int8 [E, H, I], 'scale': fp32 [E, H, I/128]}, all on the GPU.
    forward(x, top_k_index, top_k_weights) keeps the HF contract
    (Experts.forward, HF:733-757):
      * M > 1 rows: prefill_pipeline.run if one is attached, else the
        device-planned routed MoE (gpu_routes.routed_moe);
      * M == 1: grouped decode - module-level grouped_linear (W8A16, or W8A8
        after `int8.grouped_linear = w8a8.grouped_linear`), SwiGLU, and the
        ordered bf16 combine in ascending expert order.
    """

    def __init__(self, layer, gate_up, down, cache=None):
        super().__init__()
        self.layer, self.gate_up, self.down, self.cache = layer, gate_up, down, cache
        self.prefill_pipeline = None
        self.large_tile = False
        for bank in (gate_up, down):
            if not (bank['q'].is_cuda and bank['scale'].is_cuda):
                raise ValueError('Int8Experts needs an HBM-resident bank')

    def forward(self, x, top_k_index, top_k_weights):
        if x.shape[0] > 1:
            if self.prefill_pipeline is not None:
                return self.prefill_pipeline.run(self.layer, x, top_k_index, top_k_weights)
            from ..runtime import gpu_routes
            banks = [self.gate_up['q'], self.gate_up['scale'], self.down['q'], self.down['scale']]
            return gpu_routes.routed_moe(x, top_k_weights, top_k_index.contiguous(), banks,
                                         self.large_tile)
        table = build_descriptors(self.gate_up, self.down, top_k_index)
        experts = table.shape[0]
        intermediate = self.down['q'].shape[-1]
        gu = grouped_linear(x, table, experts, 2 * intermediate, 0, True)
        h = swiglu(gu)
        values = grouped_linear(h, table, experts, x.shape[-1], 2, False)
        return ordered_reduce(values, table, top_k_weights)
