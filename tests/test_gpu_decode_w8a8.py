"""Bit-level parity of the fused decode layer's W8A8 path (the three decode
kernels of lm_moe_layer_forward at one token) against the oracle.

The layer leaves its intermediates in the workspace (lm_moe_workspace_region):
the normalized row and its W8A8 quantization, the selected experts in
combine order with their weights, the fp32 epilogue sums of the 8 routed
gate_up and down rows, the SwiGLU rows and the per-slot down rows.  Each
stage is checked on the exact inputs the kernels consumed:

  quantized row     == O.act_quant(normed row)                 (w8a8.py:8-14)
  gate_up sums      == O.w8a8_accumulate(int32 partials, ...)  (w8a8.py:33-41)
  SwiGLU rows       == O.swiglu(bf16(sums)), except where the last ulp of
                       SiLU's exp decides the bf16 rounding (counted, bounded)
  down sums         == the same W8A8 arithmetic on O.act_quant(SwiGLU rows)
  down rows         == bf16(down sums)
  layer output      == residual + bf16(ordered combine + gated shared)
                                                   (int8.py:240-250, HF:790-796)

fp32 sums compared bit for bit pin the int32 group partials and the
unfused, ascending-group epilogue: a wrong partial, group order or a fused
multiply-add changes them.  The shared expert is W8A16 (within the bf16
tolerance); its gate weight is zero here, so sigmoid(0) = 0.5 exactly and no
transcendental enters the combine check.
"""
import numpy as np
import pytest
import torch

from localmoe35ba3b_amd.runtime.stack import EPS, SyntheticMoEStack, zipf_bias
from oracle import moe_oracle as O
from tests.conftest import BF16_TOL, assert_close

pytestmark = pytest.mark.gpu


def npf(t):
    return t.detach().float().cpu().numpy()


def silu_neighbours(gate, up, ulps=2):
    """The SwiGLU values bf16(bf16(s') * up) for SiLU results s' within
    `ulps` fp32 ulps of the oracle's SiLU (gate, up fp32 [n])."""
    s = O.silu_f32(gate)
    bits = s.view(np.int32).astype(np.int64)
    out = []
    for d in range(-ulps, ulps + 1):
        sd = (bits + np.where(s >= 0, d, -d)).astype(np.int32).view(np.float32)
        out.append(O.bf16(O.bf16(sd) * up))
    return np.stack(out)


@pytest.mark.parametrize('bias', [False, True])
def test_decode_w8a8_intermediates_bit_exact(dev, bias, capsys):
    st = SyntheticMoEStack(layers=1, seed=81, device=dev, max_tokens=16,
                           router_bias=zipf_bias() if bias else None)
    st.gate_w.zero_()
    E, H, I = 256, 2048, 512
    silu_ulp = total = 0
    for seed in range(90, 94):
        g = torch.Generator()
        g.manual_seed(seed)
        h = torch.randn(1, H, generator=g).to(torch.bfloat16).to(dev)
        out = h.clone()
        ids = torch.empty((1, 8), dtype=torch.int32, device=dev)
        wts = torch.empty((1, 8), dtype=torch.bfloat16, device=dev)
        st.layer_forward(out, 0, ids, wts)
        torch.cuda.synchronize()
        view = lambda name: st.workspace_view(name, 1).clone()
        xn = npf(view('normed'))
        assert np.array_equal(xn, O.rmsnorm(npf(h), None, EPS))
        xq, xs = view('act_q').cpu().numpy()[None, :], view('act_scales').cpu().numpy()[None, :]
        rq, rs = O.act_quant(xn)
        assert np.array_equal(xq, rq) and np.array_equal(xs, rs)
        sel = view('slot_ids').cpu().numpy()
        selw = view('slot_weights').cpu().numpy()
        idn, wn = ids.cpu().numpy()[0], npf(wts)[0]
        order = np.argsort(idn)
        assert np.array_equal(sel, idn[order]) and np.array_equal(selw, wn[order])
        layer = st.layer_host(0, experts=sel)
        _, rw, ri = O.router(xn, layer['router_w'], 8, layer['router_bias'])
        assert np.array_equal(idn, ri[0])
        gu_acc, dn_acc = view('gate_up_acc').cpu().numpy(), view('down_acc').cpu().numpy()
        hid, down = npf(view('hidden')), npf(view('down'))
        for s, e in enumerate(sel):
            # gate_up: int32 group partials and the unfused ascending-group epilogue
            ref = O.w8a8_accumulate(O.w8a8_partials(xq, layer['gu_q'][e]), xs, layer['gu_s'][e])
            assert np.array_equal(gu_acc[s], ref[0]), f'gate_up sums, slot {s}, expert {e}'
            gate, up = O.bf16(gu_acc[s, :I]), O.bf16(gu_acc[s, I:])
            exact = O.bf16(O.bf16(O.silu_f32(gate)) * up)
            diff = hid[s] != exact
            if diff.any():  # only SiLU's last ulp may decide the rounding
                near = silu_neighbours(gate[diff], up[diff])
                assert (near == hid[s][diff][None, :]).any(0).all(), f'SwiGLU, slot {s}'
            silu_ulp += int(diff.sum())
            total += I
            # down: the kernel's own row quantization of the SwiGLU row, then W8A8
            hq, hs = O.act_quant(hid[s][None, :])
            ref = O.w8a8_accumulate(O.w8a8_partials(hq, layer['dn_q'][e]), hs, layer['dn_s'][e])
            assert np.array_equal(dn_acc[s], ref[0]), f'down sums, slot {s}, expert {e}'
            assert np.array_equal(down[s], O.bf16(dn_acc[s])), f'down row, slot {s}'
        # shared expert (W8A16) within the bf16 tolerance
        sh_h = O.swiglu(O.w8a16_linear(xn, layer['gu_q'][E], layer['gu_s'][E]))
        assert_close(hid[8:9], sh_h, BF16_TOL, 'shared SwiGLU row')
        assert_close(down[8:9], O.w8a16_linear(hid[8:9], layer['dn_q'][E], layer['dn_s'][E]),
                     BF16_TOL, 'shared down row')
        # combine (ascending expert id), gated shared (sigmoid(0) = 0.5), residual
        routed = O.ordered_combine(down[:8], selw)
        block = O.bf16(routed + O.bf16(np.float32(0.5) * down[8]))
        assert np.array_equal(npf(out)[0], O.bf16(npf(h)[0] + block))
    assert silu_ulp <= total // 50
    with capsys.disabled():
        print(f'\n[decode W8A8] SwiGLU values set by the last ulp of SiLU: {silu_ulp} of {total}')
