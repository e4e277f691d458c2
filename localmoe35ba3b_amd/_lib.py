"""ctypes binding of liblocalmoe35ba3b.so (the C ABI in include/localmoe35ba3b.h).

The library is loaded lazily on first use.  A missing library is an error,
never a fallback: every operator of this package runs on the HIP kernels or
raises.
"""
import ctypes
import pathlib
import threading

import torch

LIB_PATH = pathlib.Path(__file__).resolve().parent / 'liblocalmoe35ba3b.so'

LM_OK, LM_EINVAL, LM_ENOMEM, LM_ELAUNCH = 0, 1, 2, 3
LM_BF16, LM_FP16, LM_FP32 = 0, 1, 2
LM_TILES_PLAIN, LM_TILES_F16 = 0, 1
# fused-layer workspace regions (lm_moe_workspace_region)
WS_REGIONS = {'normed': 0, 'gate': 1, 'ids': 2, 'weights': 3, 'route_rows': 4, 'hidden': 5,
              'down': 6, 'act_q': 7, 'act_scales': 8, 'slot_ids': 9, 'slot_weights': 10,
              'gate_up_acc': 11, 'down_acc': 12, 'router_approx': 13, 'row_norms': 14,
              'router_norms': 15}

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float

# name -> (restype, argtypes); mirrors include/localmoe35ba3b.h one to one.
SIGNATURES = {
    'lm_version': (ctypes.c_char_p, []),
    'lm_last_error': (ctypes.c_char_p, []),
    'lm_quantize_weight_g128': (I32, [P, P, P, I64, I64, P]),
    'lm_w8_tile_rows': (I32, [P, I64, I64, I64, I64, P, I32, P]),
    'lm_act_quant_g128': (I32, [P, I32, P, P, I64, I64, P]),
    'lm_w8a16_linear': (I32, [P, P, P, P, I64, I64, I64, I32, I32, P]),
    'lm_w8a16_grouped_gemv': (I32, [P, P, P, I64, I64, I64, I32, I32, I32, P]),
    'lm_w8a8_grouped_gemv': (I32, [P, P, P, P, I64, I64, I64, I32, I32, I32, P]),
    'lm_w8a8_grouped_linear': (I32, [P, P, P, I64, I64, I64, I32, I32, I32, P]),
    'lm_w8a8_group_partials': (I32, [P, P, P, I64, I64, I64, P]),
    'lm_w8a8_linear': (I32, [P, P, P, P, I64, I64, I64, I32, I32, P]),
    'lm_w8a8_gemm': (I32, [P, P, P, P, P, I64, I64, I64, I32, I32, P]),
    'lm_swiglu': (I32, [P, P, I64, I64, I32, P]),
    'lm_ordered_reduce': (I32, [P, P, P, I32, P, I64, I64, I32, P]),
    'lm_routed_reduce': (I32, [P, P, P, P, I32, P, I64, I64, I64, I32, P]),
    'lm_route_plan': (I32, [P, I64, I64, I64, I64, P, P, I64, P, P, P]),
    'lm_plan_routes_host': (I32, [P, I64, I64, I64, P, P, P, P, P]),
    'lm_route_plan_host': (I32, [P, I64, I64, I64, I64, P, P, I64, P, P, P, P]),
    'lm_routed_gemm_w8a16': (I32, [P, I64, P, P, I64, I64, I64, P, P, I64, I64, P, I64, I64,
                                   I64, I32, I32, P]),
    'lm_routed_gate_up_swiglu': (I32, [P, I64, P, P, I64, I64, I64, P, P, I64, I64, P, I64,
                                       I64, I64, I32, P]),
    'lm_router_topk': (I32, [P, P, P, P, P, P, I64, I64, I64, I64, P]),
    'lm_rmsnorm': (I32, [P, P, P, I64, I64, F32, P]),
    'lm_moe_workspace_bytes': (I64, [I64, I64, I64, I64, I64]),
    'lm_moe_workspace_init': (I32, [P, I64, P]),
    'lm_moe_workspace_region': (I32, [I64, I32, P, P]),
    'lm_moe_layer_forward': (I32, [P, P, I64, I64, I64, I64, I64, F32, P, I64, P, P, P, P]),
    'lm_moe_layer_forward_chain': (I32, [P, P, I32, P, I64, I64, I64, I64, I64, F32, P, I64, P, P,
                                         P, P]),
    'lm_moe_static_max_tokens': (I64, []),
    'lm_moe_static_init': (I32, []),
    'lm_moe_layer_forward_static': (I32, [P, P, I64, I64, I64, I64, I64, F32, P, P, P, P]),
}


class MoeLayer(ctypes.Structure):
    """struct lm_moe_layer.  struct_size is filled in on construction;
    positional arguments start at router_w."""
    _fields_ = [('struct_size', I64),
                ('router_w', P), ('router_bias', P), ('shared_gate_w', P), ('norm_w', P),
                ('gu_q', P), ('gu_s', P), ('dn_q', P), ('dn_s', P),
                ('gu_q_expert_stride', I64), ('gu_s_expert_stride', I64),
                ('dn_q_expert_stride', I64), ('dn_s_expert_stride', I64),
                ('gu_q_tiles', P), ('dn_q_tiles', P), ('gu_q_tiles_format', I64)]

    def __init__(self, *args, **kw):
        super().__init__(ctypes.sizeof(MoeLayer), *args, **kw)


_lib = None
_lock = threading.Lock()


def lib():
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not LIB_PATH.exists():
                    raise RuntimeError(
                        f'{LIB_PATH.name} is not built; run __graft_entry__.build() or '
                        'python localmoe35ba3b_amd/csrc/build.py')
                handle = ctypes.CDLL(str(LIB_PATH))
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(rc):
    """Maps a C-ABI status onto the exception the reference operators raise."""
    if rc == LM_OK:
        return
    msg = lib().lm_last_error().decode(errors='replace')
    if rc == LM_EINVAL:
        raise ValueError(msg)
    if rc == LM_ENOMEM:
        raise MemoryError(msg)
    raise RuntimeError(msg)


def call(name, *args):
    check(getattr(lib(), name)(*args))


def ptr(t):
    return None if t is None else t.data_ptr()


def stream(device=None):
    return torch.cuda.current_stream(device).cuda_stream


def dtype_code(dtype):
    if dtype == torch.bfloat16:
        return LM_BF16
    if dtype == torch.float16:
        return LM_FP16
    if dtype == torch.float32:
        return LM_FP32
    raise ValueError(f'unsupported dtype {dtype}')
