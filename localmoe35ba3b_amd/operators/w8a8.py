"""W8A8 group-128 decode operators (drop-in for qwen35_deploy/operators/w8a8.py).

quantize          per-row, per-128-group dynamic int8 activation quantization
                  (w8a8.py:8-22): s = max(amax, 1e-10) * fl32(1/127), q = rint(x / s)
grouped_linear    grouped W8A8 GEMV (w8a8.py:25-48): exact int32 dot per group,
                  acc = acc + (f32(p) * xs) * ws in ascending group order, no FMA
linear            dense W8A8 linear with optional fused SwiGLU (GEMV up to 8 rows,
                  int8 MFMA GEMM beyond)
gemm              the int8 MFMA GEMM on quantized rows
group_partials    the exact int32 per-group partials the GEMV accumulates

Swapping `int8.grouped_linear = w8a8.grouped_linear` switches Int8Experts'
decode path to W8A8 exactly as cli.py:37-39 does in the reference.
"""
import torch

from .. import _lib


def quantize(x):
    """Returns (q int8 [rows, K], s fp32 [rows, K/128]) for CUDA bf16/fp16 rows."""
    x = x.contiguous()
    k = x.shape[-1]
    if not x.is_cuda or x.ndim != 2 or k % 128:
        raise ValueError('Expected CUDA rows with K divisible by 128')
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError('Expected CUDA rows with K divisible by 128')
    q = torch.empty_like(x, dtype=torch.int8)
    s = torch.empty((x.shape[0], k // 128), device=x.device, dtype=torch.float32)
    _lib.call('lm_act_quant_g128', x.data_ptr(), _lib.dtype_code(x.dtype), q.data_ptr(),
              s.data_ptr(), x.shape[0], k, _lib.stream(x.device))
    return q, s


def _check_rows(x):
    if not x.is_cuda or x.ndim != 2 or x.shape[-1] % 128:
        raise ValueError('Expected CUDA rows with K divisible by 128')
    if x.dtype not in (torch.bfloat16, torch.float16):
        raise ValueError('Expected CUDA rows with K divisible by 128')


def grouped_linear(x, table, experts, n, field, shared):
    """Grouped W8A8 decode GEMV; activation quantization is fused into the
    kernel.  x bf16 or fp16; the output is in x.dtype (w8a8.py:46)."""
    x = x.contiguous()
    _check_rows(x)
    out = torch.empty((experts, n), device=x.device, dtype=x.dtype)
    _lib.call('lm_w8a8_grouped_linear', x.data_ptr(), table.data_ptr(), out.data_ptr(), experts,
              n, x.shape[-1], field, int(bool(shared)), _lib.dtype_code(x.dtype),
              _lib.stream(x.device))
    return out


def grouped_gemv(q, s, table, experts, n, field, shared, out_dtype=torch.bfloat16):
    """Grouped W8A8 GEMV on pre-quantized activations (the _linear kernel,
    w8a8.py:25-41); the output in out_dtype (bf16 or fp16)."""
    out = torch.empty((experts, n), device=q.device, dtype=out_dtype)
    _lib.call('lm_w8a8_grouped_gemv', q.contiguous().data_ptr(), s.contiguous().data_ptr(),
              table.data_ptr(), out.data_ptr(), experts, n, q.shape[-1], field, int(bool(shared)),
              _lib.dtype_code(out_dtype), _lib.stream(q.device))
    return out


def linear(x, q, scale, swiglu=False):
    """Dense W8A8 linear of bf16 or fp16 rows: [M, N] or, with swiglu,
    [M, N/2], in x.dtype.  Up to 8 rows run as one fused quantize + GEMV
    launch; more rows are quantized (quantize) and multiplied by the int8
    MFMA GEMM (gemm)."""
    x = x.contiguous()
    _check_rows(x)
    n, k = q.shape
    if k % 128 or x.shape[-1] != k or tuple(scale.shape) != (n, k // 128):
        raise ValueError('Invalid INT8 group geometry')
    if x.shape[0] > 8:
        xq, xs = quantize(x)
        return gemm(xq, xs, q, scale, swiglu, out_dtype=x.dtype)
    out = torch.empty((x.shape[0], n // 2 if swiglu else n), device=x.device, dtype=x.dtype)
    _lib.call('lm_w8a8_linear', x.data_ptr(), q.contiguous().data_ptr(),
              scale.contiguous().data_ptr(), out.data_ptr(), x.shape[0], n, k, int(bool(swiglu)),
              _lib.dtype_code(x.dtype), _lib.stream(x.device))
    return out


def gemm(xq, xs, q, scale, swiglu=False, out_dtype=torch.bfloat16):
    """W8A8 GEMM of quantized rows (xq int8 [M, K], xs fp32 [M, K/128], as
    returned by quantize) with int8 weights q [N, K] and fp32 group scales
    [N, K/128]: w8a8._linear (w8a8.py:25-41) for every row, int32 MFMA group
    partials and the unfused fp32 rescale in ascending group order; [M, N]
    or, with swiglu, [M, N/2], in out_dtype (bf16 or fp16)."""
    if not (xq.is_cuda and q.is_cuda) or xq.dtype != torch.int8 or q.dtype != torch.int8:
        raise ValueError('Expected CUDA int8 rows and weights')
    m, k = xq.shape
    n = q.shape[0]
    if (k % 128 or q.shape[1] != k or tuple(scale.shape) != (n, k // 128)
            or tuple(xs.shape) != (m, k // 128)):
        raise ValueError('Invalid INT8 group geometry')
    if swiglu and n % 2:
        raise ValueError('SwiGLU needs an even number of weight rows')
    out = torch.empty((m, n // 2 if swiglu else n), device=xq.device, dtype=out_dtype)
    _lib.call('lm_w8a8_gemm', xq.contiguous().data_ptr(), xs.contiguous().data_ptr(),
              q.contiguous().data_ptr(), scale.contiguous().data_ptr(), out.data_ptr(), m, n, k,
              int(bool(swiglu)), _lib.dtype_code(out_dtype), _lib.stream(xq.device))
    return out


def group_partials(xq, wq):
    """int32 [M, N, K/128] partials sum_{k in g} xq[m, k] * wq[n, k] (M <= 8)."""
    m, k = xq.shape
    n = wq.shape[0]
    out = torch.empty((m, n, k // 128), device=xq.device, dtype=torch.int32)
    _lib.call('lm_w8a8_group_partials', xq.contiguous().data_ptr(), wq.contiguous().data_ptr(),
              out.data_ptr(), m, n, k, _lib.stream(xq.device))
    return out
