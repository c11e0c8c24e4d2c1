"""GPU parity over the benchmark configurations' full (shape, batch) grid.

Every case is within 1e-2 relative L2 of the fp32 reconstruct + matmul
reference (the oracle's ``dequantize_layer`` W, then an fp32 product; bf16
cases 2e-2 for the bf16 input and output roundings):

* configuration 1 — Llama-2-7B q/k/v/o 4096x4096, gate/up 11008x4096, down
  4096x11008, 0.1% critical blocks, batch 1 and 8;
* configuration 2 — Llama-3-8B q/o 4096x4096, k/v 1024x4096, gate/up
  14336x4096, down 4096x14336 with S_group (qb = 128), 0.2% critical blocks,
  batch 1, 4 and 16;
* bf16 activations at batch 1 and at 2, 3, 4, 8 and 16 (the reference's
  default decode output type,
  ``kernels/triton_e8d4.py:181``), with and without S_group, through the
  single-layer and the multi-layer entry points;
* configuration 3 — Llama-2-13B 5120x5120, 13824x5120, 5120x13824 at 2048
  tokens, through the C-ABI prefill kernel and through ``EPTQLinear``.

The oracle's W is computed once per layer and shared by its batch sizes.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels import decode_workspace, linear_forward, linear_forward_multi
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2
TOL_BF16 = 2e-2

_W = {}


def _layer(out, inp, seed, p, qb=None, bias=False):
    """(QuantizedLayerData, oracle fp32 W) — W cached per layer."""
    key = (out, inp, seed, p, qb, bias)
    if key not in _W:
        qd = make_layer(out, inp, seed=seed, percmask=p, qb_size=qb, bias=bias)
        n = layer_np(qd)
        W = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4", n["S_group"])
        _W.clear()          # one full-size layer at a time in host memory
        _W[key] = (qd, W.astype(np.float32))
    return _W[key]


def _ref(qd, W, x):
    y = x.float().numpy() @ W.T
    if qd.bias is not None:
        y = y + qd.bias.float().numpy()
    return y


def _dev(qd):
    ocol, orp = csr_dev(qd.Q)
    return dict(Q=qd.Q.cuda(), g=qd.g.cuda(), h=qd.h.cuda(), O_vals=qd.O.cuda(), O_col=ocol, O_row_ptr=orp,
                bias=None if qd.bias is None else qd.bias.cuda(),
                S_group=None if qd.S_group is None else qd.S_group.cuda())


def _single(L, x):
    t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    y = linear_forward("e8_d4", L["Q"], t, L["g"], L["h"], x.cuda(), L["O_vals"], L["O_col"], L["O_row_ptr"],
                       L["bias"], L["S_group"])
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


CONFIG1 = [(4096, 4096), (11008, 4096), (4096, 11008)]
CONFIG2 = [(4096, 4096), (1024, 4096), (14336, 4096), (4096, 14336)]


@pytest.mark.parametrize("out,inp", CONFIG1, ids=lambda v: str(v))
def test_config1_batches(out, inp):
    qd, W = _layer(out, inp, seed=100 + out + inp, p=0.001)
    L = _dev(qd)
    for B in (1, 8):
        print(f"config 1 {out}x{inp} B={B}", flush=True)
        x = make_x(B, inp, seed=B + 7)
        e = rel_l2(_single(L, x), _ref(qd, W, x))
        print(f"  rel_l2 {e:.2e}", flush=True)
        assert e <= TOL, (out, inp, B)


@pytest.mark.parametrize("out,inp", CONFIG2, ids=lambda v: str(v))
def test_config2_batches(out, inp):
    qd, W = _layer(out, inp, seed=200 + out + inp, p=0.002, qb=128)
    L = _dev(qd)
    for B in (1, 4, 16):
        print(f"config 2 {out}x{inp} qb=128 B={B}", flush=True)
        x = make_x(B, inp, seed=B + 11)
        e = rel_l2(_single(L, x), _ref(qd, W, x))
        print(f"  rel_l2 {e:.2e}", flush=True)
        assert e <= TOL, (out, inp, B)


@pytest.mark.parametrize("qb", [None, 128])
def test_bf16_batches_2_to_16(qb):
    """bf16 x and y at B = 2, 3, 4, 8 and 16 (the reference decodes bf16 for
    every B < 256, kernels/triton_e8d4.py:160-193): the vector kernel's bf16
    instances up to 8 rows and the matrix-core kernel's from 5, single-layer
    and multi-layer (q|k|v-like shapes, with the split-K workspace)."""
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096)]
    qds, Ws = [], []
    for k, (o, i) in enumerate(shapes):
        qd = make_layer(o, i, seed=500 + k + (qb or 0), percmask=0.002, qb_size=qb, bias=k == 2)
        n = layer_np(qd)
        Ws.append(dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4",
                                   n["S_group"]).astype(np.float32))
        qds.append(qd)
    Ls = [_dev(qd) for qd in qds]
    t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    work = decode_workspace("cuda")
    for B in (2, 3, 4, 8, 16):
        x = make_x(B, 4096, seed=40 + B).bfloat16()
        xf = x.float()
        print(f"bf16 B={B} qb={qb}: single-layer and multi-layer", flush=True)
        for qd, W, L in zip(qds[:2], Ws[:2], Ls[:2]):
            y = linear_forward("e8_d4", L["Q"], t, L["g"], L["h"], x.cuda(), L["O_vals"], L["O_col"], L["O_row_ptr"],
                               L["bias"], L["S_group"])
            assert y.dtype == torch.bfloat16
            e = rel_l2(y.float().cpu().numpy(), _ref(qd, W, xf))
            print(f"  single rel_l2 {e:.2e}", flush=True)
            assert e <= TOL_BF16, (B, qb)
        y = linear_forward_multi(Ls, t, x.cuda(), work=work)
        torch.cuda.synchronize()
        assert y.dtype == torch.bfloat16
        want = np.concatenate([_ref(qd, W, xf) for qd, W in zip(qds, Ws)], axis=1)
        e = rel_l2(y.float().cpu().numpy(), want)
        print(f"  multi rel_l2 {e:.2e}", flush=True)
        assert e <= TOL_BF16, (B, qb)


@pytest.mark.parametrize("qb", [None, 128])
def test_bf16_batch1(qb):
    """bf16 x and y at batch 1 (the vector decode kernel's bf16 instance),
    single-layer and multi-layer (q|k|v-like, with the split-K workspace)."""
    shapes = [(4096, 4096), (1024, 4096), (1024, 4096)]
    qds, Ws = [], []
    for k, (o, i) in enumerate(shapes):
        qd = make_layer(o, i, seed=300 + k + (qb or 0), percmask=0.002, qb_size=qb, bias=k == 1)
        n = layer_np(qd)
        Ws.append(dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4",
                                   n["S_group"]).astype(np.float32))
        qds.append(qd)
    Ls = [_dev(qd) for qd in qds]
    x = make_x(1, 4096, seed=31).bfloat16()
    xf = x.float()
    print(f"bf16 B=1 qb={qb}: single-layer", flush=True)
    for qd, W, L in zip(qds, Ws, Ls):
        t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
        y = linear_forward("e8_d4", L["Q"], t, L["g"], L["h"], x.cuda(), L["O_vals"], L["O_col"], L["O_row_ptr"],
                           L["bias"], L["S_group"])
        assert y.dtype == torch.bfloat16
        e = rel_l2(y.float().cpu().numpy(), _ref(qd, W, xf))
        print(f"  rel_l2 {e:.2e}", flush=True)
        assert e <= TOL_BF16
    print(f"bf16 B=1 qb={qb}: multi-layer with workspace", flush=True)
    work = decode_workspace("cuda")
    t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    y = linear_forward_multi(Ls, t, x.cuda(), work=work)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    want = np.concatenate([_ref(qd, W, xf) for qd, W in zip(qds, Ws)], axis=1)
    e = rel_l2(y.float().cpu().numpy(), want)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert e <= TOL_BF16


CONFIG3 = [(5120, 5120), (13824, 5120), (5120, 13824)]


@pytest.mark.parametrize("out,inp", CONFIG3, ids=lambda v: str(v))
def test_config3_prefill(out, inp):
    """2048 tokens: the C-ABI fused prefill kernel and the module forward."""
    qd, W = _layer(out, inp, seed=400 + out + inp, p=0.002)
    x = make_x(2048, inp, seed=401)
    print(f"config 3 {out}x{inp} T=2048: reference", flush=True)
    ref = _ref(qd, W, x)
    L = _dev(qd)
    print(f"config 3 {out}x{inp} T=2048: C-ABI prefill kernel", flush=True)
    e = rel_l2(_single(L, x), ref)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert e <= TOL
    print(f"config 3 {out}x{inp} T=2048: EPTQLinear", flush=True)
    lin = EPTQLinear.from_quantized_data(qd, E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    with torch.no_grad():
        y = lin(x.cuda())
    torch.cuda.synchronize()
    e = rel_l2(y.float().cpu().numpy(), ref)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert e <= TOL
