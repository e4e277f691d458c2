"""HBM-resident MoE-FFN stack (L x [RMSNorm -> MoE block -> residual]).

Replaces the reference's CPU-pinned expert bank, 7 GiB slab arena and
frequency-retention cache (runtime/prefill.py:88-164, runtime/slab_cache.py,
runtime/frequency_seed.py): on a 288 GB MI355X the whole int8 bank of every
layer is resident in HBM, so prefill reads each active expert straight from
HBM and decode needs no cache, no host routing read and no H2D copy.

Bank layout, per stack (all contiguous, expert-major like the reference's
converted artifact, convert.py:96-97):
  gu_q  int8 [L, E+1, 2I, H]   gu_s fp32 [L, E+1, 2I, H/128]
  dn_q  int8 [L, E+1, H, I]    dn_s fp32 [L, E+1, H, I/128]
expert index E is the always-on shared expert (its gate_proj / up_proj rows
concatenated, exact because scales are per row).  Router weights bf16
[L, E, H], shared-expert gate bf16 [L, H], optional RMSNorm weights fp32
[L, H] (post_attention_layernorm, scale 1 + w).

SyntheticMoEStack fills the bank with random weights drawn on the GPU from
per-(layer, matrix) seeds, N(0, 0.02) fp32, quantized by the group-128 HIP
quantizer, and a zero RMSNorm weight; artifact.stack_from_artifact fills it
from a converted checkpoint.
"""
import ctypes
import math

import numpy as np
import torch

from .. import _lib
from ..convert import quantize_g128

HIDDEN, INTER, EXPERTS, TOP_K = 2048, 512, 256, 8
EPS = 1e-6


def matrix_seed(base, layer, matrix, chunk=0):
    """Seed of one generated weight block: matrix 0 router, 1 shared gate,
    2 gate_up, 3 down; chunk = expert block index."""
    return (base * 1_000_003 + layer * 10_007 + matrix * 101 + chunk) % (2 ** 63)


def zipf_bias(experts=EXPERTS, s=1.1, seed=3):
    """Per-expert router-logit offset that skews popularity like Zipf(s):
    offset_e = ln(r_e^-s / sum_j j^-s) - mean_e(...), r = seeded permutation of
    the ranks 1..E (numpy default_rng(seed).permutation).  fp64 -> fp32 once."""
    ranks = np.random.default_rng(seed).permutation(experts) + 1
    logp = -s * np.log(ranks.astype(np.float64)) - math.log(
        np.sum(np.arange(1, experts + 1, dtype=np.float64) ** -s))
    return (logp - logp.mean()).astype(np.float32)


class MoEStack:
    """HBM-resident MoE-FFN stack: the int8 bank, router and gate weights of
    every layer plus the fused-layer workspace.  Subclasses / constructors
    fill the tensors (random init: SyntheticMoEStack; converted checkpoint:
    artifact.stack_from_artifact).

    layers may be reduced for tests; the fused layer kernels require hidden
    2048, intermediate 512, 256 experts and top-8.
    """

    def __init__(self, layers, device='cuda', max_tokens=2048, router_bias=None, norm=False):
        self.L = layers
        self.E, self.H, self.I, self.K = EXPERTS, HIDDEN, INTER, TOP_K
        self.device = torch.device(device)
        self.max_tokens = max_tokens
        dev = self.device
        E1 = self.E + 1
        self.gu_q = torch.empty((layers, E1, 2 * self.I, self.H), dtype=torch.int8, device=dev)
        self.gu_s = torch.empty((layers, E1, 2 * self.I, self.H // 128), dtype=torch.float32,
                                device=dev)
        self.dn_q = torch.empty((layers, E1, self.H, self.I), dtype=torch.int8, device=dev)
        self.dn_s = torch.empty((layers, E1, self.H, self.I // 128), dtype=torch.float32,
                                device=dev)
        self.router_w = torch.empty((layers, self.E, self.H), dtype=torch.bfloat16, device=dev)
        self.gate_w = torch.empty((layers, self.H), dtype=torch.bfloat16, device=dev)
        # RMSNorm weight w of (1 + w); None = zeros, as for a freshly initialised norm
        self.norm_w = (torch.zeros((layers, self.H), dtype=torch.float32, device=dev)
                       if norm else None)
        self.router_bias = None
        if router_bias is not None:
            self.router_bias = torch.as_tensor(router_bias, dtype=torch.float32).to(dev)
        nbytes = _lib.lib().lm_moe_workspace_bytes(max_tokens, self.H, self.I, self.E, self.K)
        if nbytes < 0:
            raise ValueError('unsupported MoE geometry')
        self.workspace = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        _lib.call('lm_moe_workspace_init', self.workspace.data_ptr(), nbytes, _lib.stream(dev))
        self._structs = [self._layer_struct(l) for l in range(layers)]
        self._side = self._side_ws = None  # second stream and workspace of prefill_
        self.gu_q_tiles = self.dn_q_tiles = None  # see build_prefill_tiles
        self._tiles_of = None  # versions of gu_q / dn_q the tile copies were built from
        self._static_ready = False

    # ------------------------------------------------------------------ views
    def bank_bytes(self):
        tensors = [self.gu_q, self.gu_s, self.dn_q, self.dn_s, self.router_w, self.gate_w]
        if self.norm_w is not None:
            tensors.append(self.norm_w)
        return sum(t.numel() * t.element_size() for t in tensors)

    def tile_bytes(self):
        """Bytes of the prefill tile copy (0 when build_prefill_tiles has not run)."""
        if self.gu_q_tiles is None:
            return 0
        return (self.gu_q_tiles.numel() + self.dn_q_tiles.numel()) * self.gu_q_tiles.element_size()

    def build_prefill_tiles(self, gate_up_format=_lib.LM_TILES_F16):
        """Copies of gu_q and dn_q in the 16-row tile layout (lm_w8_tile_rows)
        for the prefill grouped GEMMs, which then read each 16-row x 64-K
        weight block as one contiguous 1 KB wave load.  gu_q's copy is in
        `gate_up_format`: LM_TILES_F16 (default) runs the gate_up GEMM on
        fp16 operands with the group scales applied to the fp32 sums (within
        the bf16 tolerance of the reference's arithmetic, faster);
        LM_TILES_PLAIN keeps the exact bf16(q * s) dequantization, bit for
        bit.  dn_q's copy is plain.  Costs a second int8 bank in HBM (about
        32 GB for 40 layers).  Call again after changing gu_q / dn_q."""
        if self.gu_q_tiles is None:
            self.gu_q_tiles = torch.empty_like(self.gu_q)
            self.dn_q_tiles = torch.empty_like(self.dn_q)
        st = _lib.stream(self.device)
        for l in range(self.L):
            for q, t, fmt in ((self.gu_q, self.gu_q_tiles, gate_up_format),
                              (self.dn_q, self.dn_q_tiles, _lib.LM_TILES_PLAIN)):
                _lib.call('lm_w8_tile_rows', q[l].data_ptr(), q.shape[1], q.shape[2], q.shape[3],
                          q.stride(1), t[l].data_ptr(), fmt, st)
            self._structs[l].gu_q_tiles = self.gu_q_tiles[l].data_ptr()
            self._structs[l].dn_q_tiles = self.dn_q_tiles[l].data_ptr()
            self._structs[l].gu_q_tiles_format = gate_up_format
        self._tiles_of = self._bank_versions()
        return self

    def _bank_versions(self):
        return (self.gu_q._version, self.dn_q._version)

    def check_tiles(self):
        """Raises when gu_q or dn_q were written in place after the tile
        copies were built: prefill would read the old weights through the
        copies while decode reads the new ones."""
        if self._tiles_of is not None and self._tiles_of != self._bank_versions():
            raise RuntimeError('gu_q / dn_q changed after build_prefill_tiles(); call it again '
                               'so that the prefill tile copies hold the same weights')

    def _layer_struct(self, l):
        s = _lib.MoeLayer()
        s.router_w = self.router_w[l].data_ptr()
        s.router_bias = self.router_bias.data_ptr() if self.router_bias is not None else None
        s.shared_gate_w = self.gate_w[l].data_ptr()
        s.norm_w = self.norm_w[l].data_ptr() if self.norm_w is not None else None
        s.gu_q = self.gu_q[l].data_ptr()
        s.gu_s = self.gu_s[l].data_ptr()
        s.dn_q = self.dn_q[l].data_ptr()
        s.dn_s = self.dn_s[l].data_ptr()
        s.gu_q_expert_stride = self.gu_q.stride(1)
        s.gu_s_expert_stride = self.gu_s.stride(1)
        s.dn_q_expert_stride = self.dn_q.stride(1)
        s.dn_s_expert_stride = self.dn_s.stride(1)
        return s

    def banks(self, l):
        """Routed-expert banks of layer l in the reference routed_moe format."""
        return [self.gu_q[l, :self.E], self.gu_s[l, :self.E], self.dn_q[l, :self.E],
                self.dn_s[l, :self.E]]

    # ------------------------------------------------------------------ forward
    def new_workspace(self):
        """Another fused-layer workspace of this stack's size, for a chunk that
        runs concurrently with the one using `self.workspace`."""
        ws = torch.empty_like(self.workspace)
        _lib.call('lm_moe_workspace_init', ws.data_ptr(), ws.numel(), _lib.stream(self.device))
        return ws

    def layer_forward(self, h, l, ids_out=None, weights_out=None, events=None, workspace=None,
                      next_layer=None, input_normed=False):
        """h bf16 [T, H] updated in place: h = h + block(rmsnorm(h)).  Chunks
        in flight at the same time need workspaces of their own.

        Chained calls (lm_moe_layer_forward_chain): with next_layer, the call
        also leaves layer next_layer's normalized inputs for these rows in the
        workspace; the following call for next_layer, on the same rows and
        workspace, passes input_normed=True and skips its norm kernel.  The
        results are bit-identical to unchained calls."""
        if h.dtype != torch.bfloat16 or not h.is_contiguous() or h.shape[-1] != self.H:
            raise ValueError('expected contiguous bf16 [tokens, 2048] hidden states')
        tokens = h.shape[0]
        if tokens > self.max_tokens:
            raise MemoryError('token count exceeds the workspace of this stack')
        self.check_tiles()
        ev = None
        if events is not None:
            ev = (ctypes.c_void_p * len(events))(*[e.cuda_event for e in events])
        ws = self.workspace if workspace is None else workspace
        if next_layer is None and not input_normed:
            _lib.call('lm_moe_layer_forward', ctypes.byref(self._structs[l]), h.data_ptr(), tokens,
                      self.H, self.I, self.E, self.K, EPS, ws.data_ptr(), ws.numel(),
                      _lib.ptr(ids_out), _lib.ptr(weights_out), ev, _lib.stream(h.device))
            return h
        nxt = None if next_layer is None else ctypes.byref(self._structs[next_layer])
        _lib.call('lm_moe_layer_forward_chain', ctypes.byref(self._structs[l]), nxt,
                  int(bool(input_normed)), h.data_ptr(), tokens, self.H, self.I, self.E, self.K,
                  EPS, ws.data_ptr(), ws.numel(), _lib.ptr(ids_out), _lib.ptr(weights_out), ev,
                  _lib.stream(h.device))
        return h

    _REGION_TYPES = {'normed': (torch.bfloat16, 'H'), 'gate': (torch.float32, None),
                     'ids': (torch.int64, 'K'), 'weights': (torch.bfloat16, 'K'),
                     'route_rows': (torch.int32, 'K'), 'hidden': (torch.bfloat16, 'I'),
                     'down': (torch.bfloat16, 'H'), 'act_q': (torch.int8, None),
                     'act_scales': (torch.float32, None), 'slot_ids': (torch.int32, None),
                     'slot_weights': (torch.float32, None),
                     'gate_up_acc': (torch.float32, '2I'), 'down_acc': (torch.float32, 'H'),
                     'router_approx': (torch.float32, 'E'), 'row_norms': (torch.float32, None),
                     'router_norms': (torch.float32, None)}

    def workspace_view(self, region, tokens, workspace=None):
        """Typed view of one intermediate a call on `tokens` rows left in the
        workspace (lm_moe_workspace_region): 'normed', 'gate', 'ids',
        'weights', 'hidden', 'down'; of prefill calls 'route_rows' and the
        approximate router logits with the norms of their error bound
        'router_approx', 'row_norms', 'router_norms'; the W8A8 intermediates
        of decode calls 'act_q', 'act_scales', 'slot_ids', 'slot_weights',
        'gate_up_acc', 'down_acc'.  Valid until the next call that uses the
        same workspace."""
        ws = self.workspace if workspace is None else workspace
        off, nbytes = ctypes.c_int64(), ctypes.c_int64()
        _lib.call('lm_moe_workspace_region', tokens, _lib.WS_REGIONS[region],
                  ctypes.byref(off), ctypes.byref(nbytes))
        dtype, inner = self._REGION_TYPES[region]
        raw = ws[off.value:off.value + nbytes.value].view(dtype)
        if inner is None:
            return raw
        return raw.view(-1, {'H': self.H, 'I': self.I, 'K': self.K, '2I': 2 * self.I,
                             'E': self.E}[inner])

    def layer_forward_static(self, h, l, ids_out=None, weights_out=None):
        """layer_forward through lm_moe_layer_forward_static: the workspace is
        the library's own device array, so the call allocates nothing (at most
        lm_moe_static_max_tokens() tokens; calls on one device must not
        overlap)."""
        if h.dtype != torch.bfloat16 or not h.is_contiguous() or h.shape[-1] != self.H:
            raise ValueError('expected contiguous bf16 [tokens, 2048] hidden states')
        if h.device != self.device:
            raise ValueError(f'hidden states on {h.device}, stack on {self.device}')
        self.check_tiles()
        with torch.cuda.device(h.device):
            if not self._static_ready:
                # resolves the library's array on this device; kept out of graph capture
                _lib.call('lm_moe_static_init')
                self._static_ready = True
            _lib.call('lm_moe_layer_forward_static', ctypes.byref(self._structs[l]),
                      h.data_ptr(), h.shape[0], self.H, self.I, self.E, self.K, EPS,
                      _lib.ptr(ids_out), _lib.ptr(weights_out), None, _lib.stream(h.device))
        return h

    def forward(self, h, layers=None, workspace=None, chain=True):
        """All (or the first `layers`) layers over h in place, one workspace;
        with chain, each layer's combine prepares the next layer's normalized
        rows (layer_forward's next_layer / input_normed)."""
        n = self.L if layers is None else layers
        for l in range(n):
            self.layer_forward(h, l, workspace=workspace,
                               next_layer=l + 1 if chain and l + 1 < n else None,
                               input_normed=chain and l > 0)
        return h

    def prefill(self, x, chunk=2048, overlap=True):
        """Runs all layers over x [T, H] in chunks of `chunk` tokens; returns h."""
        out = x.clone()
        self.prefill_(out, chunk, overlap)
        return out

    def prefill_(self, h, chunk=2048, overlap=True):
        """In-place chunked prefill of h [T, H], as the reference's chunked
        profile runs the model over consecutive `chunk`-token slices of the
        prompt (generation.py:39-42).

        With overlap, consecutive chunks alternate between the current stream
        and a second stream with a workspace of its own, and chunk c enters
        layer l as soon as chunk c-1 has left layer l-1.  That is the order a
        model with attention between its MoE blocks allows: chunk c's layer-l
        attention reads the keys and values chunk c-1 made from its layer-l
        input.  One chunk's latency-bound routing kernels then run beside the
        other's grouped GEMMs.  Every chunk computes exactly what it computes
        alone, so the result is bit-identical to overlap=False.  The schedule
        is stream-ordered and HIP-graph capturable.
        """
        if h.dtype != torch.bfloat16 or not h.is_contiguous() or h.dim() != 2 or h.shape[-1] != self.H:
            raise ValueError('expected contiguous bf16 [tokens, 2048] hidden states')
        if chunk < 1:
            raise ValueError('chunk must be positive')
        if min(chunk, h.shape[0]) > self.max_tokens:  # before anything is queued
            raise MemoryError('token count exceeds the workspace of this stack')
        starts = list(range(0, h.shape[0], chunk))
        if not starts:  # no tokens: nothing to queue, no second workspace
            return h
        if not overlap or len(starts) == 1:
            for c0 in starts:
                self.forward(h[c0:c0 + chunk])
            return h
        if self._side is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError('run prefill_ once outside graph capture first: the second '
                                   'workspace must not come from the graph pool')
            self._side = torch.cuda.Stream(self.device)
            self._side_ws = self.new_workspace()
        cur = torch.cuda.current_stream(self.device)
        streams, spaces = (cur, self._side), (self.workspace, self._side_ws)
        self._side.wait_stream(cur)
        done = [[torch.cuda.Event() for _ in range(self.L)] for _ in starts]
        # chained layers need a workspace per chunk (two chunks, two workspaces)
        chain = len(starts) == 2
        for l in range(self.L):
            for c, c0 in enumerate(starts):
                st = streams[c % 2]
                with torch.cuda.stream(st):
                    if c and l:
                        st.wait_event(done[c - 1][l - 1])
                    self.layer_forward(h[c0:c0 + chunk], l, workspace=spaces[c % 2],
                                       next_layer=l + 1 if chain and l + 1 < self.L else None,
                                       input_normed=chain and l > 0)
                    done[c][l].record(st)
        cur.wait_stream(self._side)
        self._done_events = done  # kept alive until the next call
        return h

    # ------------------------------------------------------------------ oracle views
    def layer_host(self, l, experts=None):
        """Host (numpy) copy of layer l for the CPU oracle.  With `experts`
        only those routed experts (plus the shared expert E) are copied and the
        bank entries are dicts keyed by expert id."""
        E = self.E
        names = ('gu_q', 'gu_s', 'dn_q', 'dn_s')
        src = (self.gu_q, self.gu_s, self.dn_q, self.dn_s)
        if experts is None:
            banks = {n: t[l].cpu().numpy() for n, t in zip(names, src)}
        else:
            sel = sorted(set(int(e) for e in experts) | {E})
            banks = {n: {e: t[l, e].cpu().numpy() for e in sel} for n, t in zip(names, src)}
        return dict(router_w=self.router_w[l].float().cpu().numpy(),
                    router_bias=None if self.router_bias is None
                    else self.router_bias.cpu().numpy(),
                    shared_gate_w=self.gate_w[l].float().cpu().numpy(),
                    norm_w=None if self.norm_w is None else self.norm_w[l].cpu().numpy(),
                    **banks)


class SyntheticMoEStack(MoEStack):
    """Random-init 35B-A3B-class MoE-FFN stack resident in HBM: weights drawn
    on the GPU from per-(layer, matrix) seeds, N(0, 0.02) fp32, quantized by
    the group-128 HIP quantizer; RMSNorm weight zero (norm=True allocates a
    zero weight tensor the caller may fill, norm_w).  With prefill_tiles the
    prefill GEMMs read a tile-layout copy of the int8 bank, gate_up's in
    `gate_up_format` (build_prefill_tiles)."""

    def __init__(self, layers=40, seed=4, device='cuda', max_tokens=2048, router_bias=None,
                 chunk_experts=32, prefill_tiles=True, gate_up_format=_lib.LM_TILES_F16,
                 norm=False):
        super().__init__(layers, device, max_tokens, router_bias, norm)
        dev = self.device
        E1 = self.E + 1
        gen = torch.Generator(device=dev)
        for l in range(layers):
            gen.manual_seed(matrix_seed(seed, l, 0))
            self.router_w[l] = (torch.randn((self.E, self.H), generator=gen, device=dev)
                                * 0.02).to(torch.bfloat16)
            gen.manual_seed(matrix_seed(seed, l, 1))
            self.gate_w[l] = (torch.randn(self.H, generator=gen, device=dev) * 0.02).to(
                torch.bfloat16)
            for c0 in range(0, E1, chunk_experts):
                c1 = min(E1, c0 + chunk_experts)
                gen.manual_seed(matrix_seed(seed, l, 2, c0 // chunk_experts))
                w = torch.randn((c1 - c0, 2 * self.I, self.H), generator=gen, device=dev) * 0.02
                self.gu_q[l, c0:c1], self.gu_s[l, c0:c1] = quantize_g128(w)
                gen.manual_seed(matrix_seed(seed, l, 3, c0 // chunk_experts))
                w = torch.randn((c1 - c0, self.H, self.I), generator=gen, device=dev) * 0.02
                self.dn_q[l, c0:c1], self.dn_s[l, c0:c1] = quantize_g128(w)
                del w
        if prefill_tiles:
            self.build_prefill_tiles(gate_up_format)
