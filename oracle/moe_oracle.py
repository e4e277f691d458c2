"""CPU oracle of the quantized MoE-FFN hot path - TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module, and only as the reference results are compared with (or the timed
CPU baseline).  The product
path (localmoe35ba3b_amd) never calls it.

Each function restates the arithmetic of the reference path it cites
(qwen35_deploy/... of heliosz616/LocalMoe35Ba3b, and "HF" = Transformers
5.15.0 modeling_qwen3_5_moe.py).  Integer and rounding work is numpy; the
float GEMMs are PyTorch-CPU dequantize-then-matmul (bf16 operands, fp32
accumulation), the reference's own arithmetic on the host.

Arrays: bf16 values are carried as np.float32 holding exactly representable
bf16 numbers (see bf16()); int8 / int32 / int64 as numpy integers.
"""
import numpy as np
import torch
import torch.nn.functional as F

GROUP = 128


# ----------------------------------------------------------------- rounding
def bf16(a):
    """Round-to-nearest-even to bf16, returned as float32 (bit manipulation):
    add 0x7FFF plus the lowest kept bit, clear the low 16 bits.  In uint32
    arithmetic the sum wraps only for bit patterns >= 0xFFFF8000, which are
    NaNs and are replaced by NaN."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = a.view(np.uint32)
    rounded = (b + np.uint32(0x7FFF) + ((b >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000)
    out = rounded.view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out = np.where(nan, np.float32(np.nan), out).astype(np.float32)
    return out


def fp16(a):
    """Round-to-nearest-even to fp16 (numpy's float16 conversion), returned as
    float32.  The reference runs an fp16 model with every rounding step of
    the bf16 path in fp16 instead (outputs are allocated in x.dtype)."""
    return np.asarray(a, dtype=np.float32).astype(np.float16).astype(np.float32)


def to_torch_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.bfloat16)


def from_torch(t):
    return t.detach().to(torch.float32).cpu().numpy()


# ----------------------------------------------------------------- a1 quantizer
def quantize_weight(w):
    """convert.quantize (convert.py:31-37): per 128-group s = max(amax/127, 1e-30),
    q = clamp(round_half_even(w / s), -127, 127).  w float32 [..., K]."""
    w = np.asarray(w, dtype=np.float32)
    shape = w.shape
    v = w.reshape(*shape[:-1], shape[-1] // GROUP, GROUP)
    s = np.maximum(np.abs(v).max(-1) / np.float32(127), np.float32(1e-30)).astype(np.float32)
    q = np.clip(np.rint(v / s[..., None]), -127, 127).astype(np.int8)
    return q.reshape(shape), s


def dequant(q, s, round_to=bf16):
    """int8._linear's in-kernel dequant (int8.py:19-21): dtype(f32(q) * s[n, k/128])."""
    q = np.asarray(q)
    shape = q.shape
    v = q.reshape(*shape[:-1], shape[-1] // GROUP, GROUP).astype(np.float32)
    w = (v * np.asarray(s, np.float32)[..., None]).astype(np.float32)
    return round_to(w).reshape(shape)


# ----------------------------------------------------------------- a4 act quant
INV127 = np.float32(1.0 / 127.0)


def act_quant(x):
    """w8a8._quant (w8a8.py:8-14): s = max(amax, 1e-10) * fl32(1/127); q = rint(x / s)."""
    x = np.asarray(x, dtype=np.float32)
    rows, k = x.shape
    v = x.reshape(rows, k // GROUP, GROUP)
    s = (np.maximum(np.abs(v).max(-1), np.float32(1e-10)) * INV127).astype(np.float32)
    q = np.rint(v / s[..., None]).astype(np.int8)
    return q.reshape(rows, k), s


# ----------------------------------------------------------------- a5 W8A8
def w8a8_partials(xq, wq):
    """Exact per-group int32 dots of w8a8._linear (w8a8.py:36-37): p[m, n, g]."""
    xq = np.asarray(xq, dtype=np.int64)
    wq = np.asarray(wq, dtype=np.int64)
    m, k = xq.shape
    n = wq.shape[0]
    g = k // GROUP
    p = np.einsum('mgk,ngk->mng', xq.reshape(m, g, GROUP), wq.reshape(n, g, GROUP))
    return p.astype(np.int32)


def w8a8_accumulate(p, xs, ws):
    """The w8a8.py:40 epilogue: acc = acc + (f32(p_g) * xs_g) * ws[n, g], g ascending,
    every operation rounded to fp32 (enable_fp_fusion=False).  Returns fp32 [M, N]."""
    p = np.asarray(p)
    m, n, g = p.shape
    xs = np.asarray(xs, np.float32)
    ws = np.asarray(ws, np.float32)
    acc = np.zeros((m, n), dtype=np.float32)
    for j in range(g):
        term = (p[:, :, j].astype(np.float32) * xs[:, j:j + 1]).astype(np.float32)
        term = (term * ws[None, :, j]).astype(np.float32)
        acc = (acc + term).astype(np.float32)
    return acc


def w8a8_linear(x, wq, ws, round_to=bf16):
    """w8a8.grouped_linear for one weight matrix (w8a8.py:44-48): [M, N] in
    x.dtype T (bf16 or fp16)."""
    xq, xs = act_quant(x)
    return round_to(w8a8_accumulate(w8a8_partials(xq, wq), xs, ws))


# ----------------------------------------------------------------- a2 W8A16
def w8a16_linear(x, q, s, round_to=bf16):
    """int8.linear (int8.py:9-37): T(x . T(q*s)^T) with fp32 accumulation, T =
    bf16 (torch-CPU bf16 F.linear) or fp16 (round_to=fp16: the products of
    the fp16 operands summed in float64, then rounded to fp16)."""
    if round_to is bf16:
        xt = to_torch_bf16(x)
        wt = to_torch_bf16(dequant(q, s))
        return from_torch(F.linear(xt, wt))
    w = dequant(q, s, round_to).astype(np.float64)
    return round_to((round_to(x).astype(np.float64) @ w.T).astype(np.float32))


# ----------------------------------------------------------------- a11 SwiGLU
def silu_f32(g):
    g = np.asarray(g, np.float32)
    with np.errstate(over='ignore'):  # exp(-g) = inf for g < -88 gives the limit -0
        return (g / (np.float32(1) + np.exp(-g))).astype(np.float32)


def swiglu(gu, round_to=bf16):
    """`gate, up = gu.chunk(2, -1); silu(gate) * up` on T (HF:715, prefill.py:77-78):
    h = T(T(silu(gate)) * up), T = bf16 or fp16."""
    gu = np.asarray(gu, np.float32)
    half = gu.shape[-1] // 2
    gate, up = gu[..., :half], gu[..., half:]
    return round_to(round_to(silu_f32(gate)) * up)


# ----------------------------------------------------------------- a6 / a12 combine
def ordered_combine(values, weights, round_to=bf16):
    """int8._ordered_reduce / prefill._reduce (int8.py:240-250, prefill.py:37-49):
    over rows in the given (ascending expert) order acc = T(acc + T(v * w)),
    T = bf16 or fp16 (the output dtype)."""
    values = np.asarray(values, np.float32)
    acc = np.zeros(values.shape[1:], dtype=np.float32)
    for v, w in zip(values, np.asarray(weights, np.float32)):
        acc = round_to(acc + round_to(v * np.float32(w)))
    return acc


# ----------------------------------------------------------------- a8 router
def router_logits(x, w, bias=None):
    """HF TopKRouter logits (HF:770) under this build's contract:
    f32(bf16(f32(sum_k f64(x) f64(w)))) (+ fp32 bias)."""
    acc = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    lg = bf16(acc.astype(np.float32))
    if bias is not None:
        lg = (lg + np.asarray(bias, np.float32)[None, :]).astype(np.float32)
    return lg


def topk_select(logits, k):
    """Top-k by (logit desc, expert id asc) - the fixed tie rule of this build."""
    logits = np.asarray(logits, np.float32) + np.float32(0.0)  # -0 -> +0
    t, e = logits.shape
    ids = np.empty((t, k), dtype=np.int64)
    idx = np.arange(e)
    for i in range(t):
        order = np.lexsort((idx, -logits[i]))
        ids[i] = order[:k]
    return ids


def router(x, w, k, bias=None):
    """HF TopKRouter.forward (HF:768-776): logits, fp32 softmax, top-k, renormalise,
    bf16 weights.  Returns (logits f32, weights bf16-as-f32, ids int64)."""
    lg = router_logits(x, w, bias)
    ids = topk_select(lg, k)
    mx = lg.max(-1, keepdims=True)
    ex = np.exp((lg - mx).astype(np.float32)).astype(np.float32)
    p = (ex / ex.sum(-1, keepdims=True, dtype=np.float32)).astype(np.float32)
    top = np.take_along_axis(p, ids, -1)
    wts = bf16((top / top.sum(-1, keepdims=True, dtype=np.float32)).astype(np.float32))
    return lg, wts, ids


# ----------------------------------------------------------------- a9 route plan
def plan(ids, experts, bm):
    """gpu_routes.plan + _table (gpu_routes.py:17-36, 47-63)."""
    ids = np.asarray(ids, np.int64)
    t, top = ids.shape
    flat = ids.reshape(-1)
    routes = flat.size
    original = np.argsort(flat, kind='stable')
    sorted_ids = flat[original]
    offsets = np.searchsorted(sorted_ids, np.arange(experts + 1), side='left')
    counts = offsets[1:] - offsets[:-1]
    ends = np.cumsum((counts + bm - 1) // bm)
    max_tiles = (routes + bm - 1) // bm + experts
    table = np.zeros((max_tiles, 3), dtype=np.int64)
    total = int(ends[-1])
    for tile in range(total):
        e = int(np.searchsorted(ends, tile, side='right'))
        prior = int(ends[e - 1]) if e > 0 else 0
        table[tile] = (e, offsets[e] + (tile - prior) * bm, offsets[e + 1])
    slots = np.argsort(ids, axis=1, kind='stable')
    inverse = np.empty(routes, dtype=np.int64)
    inverse[original] = np.arange(routes)
    ordered = inverse[np.arange(t)[:, None] * top + slots]
    return original // top, table, ordered, slots


def plan_routes(ids, experts):
    """routing.plan_routes (routing.py:5-20): positions [2, R] and segments."""
    ids = np.asarray(ids, np.int64)
    if ids.ndim != 2 or ids.size == 0:
        raise ValueError('Expected nonempty CPU [tokens,top_k] IDs')
    if ids.min() < 0 or ids.max() >= experts:
        raise ValueError('Out-of-range expert ID')
    flat = ids.reshape(-1)
    order = np.argsort(flat, kind='stable')
    counts = np.bincount(flat, minlength=experts)
    positions = np.stack((order // ids.shape[1], order % ids.shape[1]))
    segments, start = [], 0
    for e, c in enumerate(counts):
        if c:
            segments.append((e, start, start + int(c)))
            start += int(c)
    return positions, segments


# ----------------------------------------------------------------- a14 norm / block
def _sum_squares_tree(x):
    """Sum of squares per row in this build's fixed reduction tree: 256
    partial sums over contiguous chunks of ceil(n/256) elements (in order),
    a 64-lane xor butterfly inside each group of 64 partials, then the four
    group totals left to right - every step rounded to fp32."""
    rows, n = x.shape
    per = -(-n // 256)
    pad = np.zeros((rows, 256 * per), np.float32)
    pad[:, :n] = x
    v = pad.reshape(rows, 256, per)
    part = np.zeros((rows, 256), np.float32)
    for j in range(per):
        part = (part + (v[:, :, j] * v[:, :, j]).astype(np.float32)).astype(np.float32)
    w = part.reshape(rows, 4, 64)
    idx = np.arange(64)
    for o in (32, 16, 8, 4, 2, 1):
        w = (w + w[:, :, idx ^ o]).astype(np.float32)
    tot = w[:, 0, 0]
    for i in range(1, 4):
        tot = (tot + w[:, i, 0]).astype(np.float32)
    return tot


def rmsnorm(x, w=None, eps=1e-6):
    """Qwen3_5MoeRMSNorm (HF:807-815): bf16((x * rsqrt(mean(x^2) + eps)) * (1 + w)),
    with the mean taken over the fixed reduction tree above and
    rsqrt = 1 / sqrt (IEEE), so kernel and oracle agree bit for bit."""
    x = np.asarray(x, np.float32)
    shape = x.shape
    x2 = x.reshape(-1, shape[-1])
    ms = (_sum_squares_tree(x2) / np.float32(shape[-1])).astype(np.float32)
    r = (np.float32(1) / np.sqrt((ms + np.float32(eps)).astype(np.float32))).astype(np.float32)
    y = (x2 * r[:, None]).astype(np.float32)
    if w is not None:
        y = (y * (np.float32(1) + np.asarray(w, np.float32))).astype(np.float32)
    return bf16(y).reshape(shape)


def expert_w8a16(x, gu_q, gu_s, dn_q, dn_s, round_to=bf16):
    """One expert MLP in W8A16 (int8.linear twice + SwiGLU), [M, H] in T."""
    h = swiglu(w8a16_linear(x, gu_q, gu_s, round_to), round_to)
    return w8a16_linear(h, dn_q, dn_s, round_to)


def expert_w8a8(x, gu_q, gu_s, dn_q, dn_s, round_to=bf16):
    """One expert MLP in W8A8 (w8a8.grouped_linear twice + SwiGLU), [M, H] in T."""
    h = swiglu(w8a8_linear(x, gu_q, gu_s, round_to), round_to)
    return w8a8_linear(h, dn_q, dn_s, round_to)


def moe_block(x, layer, k=8, w8a8_routed=None, routing=None):
    """One MoE-FFN block on normalized rows x bf16 [T, H] (HF:787-797):
    routed experts combined in ascending expert order (int8.py:185-186,
    prefill.py:83-84) plus the sigmoid-gated W8A16 shared expert.
    w8a8_routed defaults to True for one row (decode) and False otherwise.
    layer: dict of numpy arrays router_w [E,H], router_bias [E] or None,
    shared_gate_w [H], gu_q [E+1,2I,H], gu_s, dn_q [E+1,H,I], dn_s.
    routing: optional (weights, ids) to use instead of the router's.
    Returns (block_out bf16 [T, H], (logits, weights, ids))."""
    x = np.asarray(x, np.float32)
    t = x.shape[0]
    if w8a8_routed is None:
        w8a8_routed = t == 1
    e_routed = layer['router_w'].shape[0]
    lg, wts, ids = router(x, layer['router_w'], k, layer.get('router_bias'))
    if routing is not None:
        wts, ids = routing
    expert = expert_w8a8 if w8a8_routed else expert_w8a16
    routed = np.zeros_like(x)
    for e in np.unique(ids):
        token, slot = np.nonzero(ids == e)
        y = expert(x[token], layer['gu_q'][e], layer['gu_s'][e], layer['dn_q'][e], layer['dn_s'][e])
        contrib = bf16(y * wts[token, slot][:, None])
        routed[token] = bf16(routed[token] + contrib)
    sh = expert_w8a16(x, layer['gu_q'][e_routed], layer['gu_s'][e_routed],
                      layer['dn_q'][e_routed], layer['dn_s'][e_routed])
    gl = router_logits(x, layer['shared_gate_w'][None, :])[:, 0]
    with np.errstate(over='ignore'):  # exp(-gl) = inf gives the limit 0
        sig = bf16((np.float32(1) / (np.float32(1) + np.exp(-gl))).astype(np.float32))
    out = bf16(routed + bf16(sig[:, None] * sh))
    return out, (lg, wts, ids)


def moe_layer(h, layer, k=8, eps=1e-6, routing=None):
    """Synthetic stack layer: h = bf16(h + block(rmsnorm(h))) (HF:866-875)."""
    x = rmsnorm(h, layer.get('norm_w'), eps)
    out, route = moe_block(x, layer, k, routing=routing)
    return bf16(np.asarray(h, np.float32) + out), route
