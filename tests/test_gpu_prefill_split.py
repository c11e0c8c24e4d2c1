"""GPU: split-K prefill of the LDS-decode GEMM at mid token counts.

With a decode workspace (``decode_workspace``; the modules pass the stream's
own), prefill launches whose tiles leave half the CUs idle or more split
their K-steps over up to 4 parts; the parts' fp32 sums (times the
activation scale) meet in the workspace's prefill area and a second launch
adds them in part order.  Checks, against the fp32 reconstruct + matmul
oracle within the 1e-2 relative-L2 bar: Llama-2-7B shapes at 256, 512 and
1024 tokens through the multi-layer C ABI (gate|up as two layers of one
call), the unsplit form (no workspace) within rounding of the split one,
repeats bit-identical; a layer with more critical blocks than the LDS stage
holds (20% of blocks), so the corrections after the K loop run in every part
with their column ranges; and ``EPTQLinear`` at 512 tokens (stream
workspace).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels import decode_workspace, linear_forward_multi
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _dev(qd):
    ocol, orp = csr_dev(qd.Q)
    return dict(Q=qd.Q.cuda(), g=qd.g.cuda(), h=qd.h.cuda(), O_vals=qd.O.reshape(-1, 8).cuda(), O_col=ocol,
                O_row_ptr=orp, bias=None if qd.bias is None else qd.bias.cuda(), S_group=None)


def _W(qd):
    n = layer_np(qd)
    return dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4").astype(np.float32)


@pytest.mark.parametrize("shapes,p", [([(4096, 4096)], 0.001), ([(11008, 4096), (11008, 4096)], 0.001),
                                      ([(4096, 11008)], 0.001), ([(2048, 4096)], 0.2)])
def test_split_prefill_matches_oracle(shapes, p):
    qds = [make_layer(o, i, seed=70 + k + int(1000 * p), percmask=p, bias=k == 0) for k, (o, i) in enumerate(shapes)]
    Ls = [_dev(qd) for qd in qds]
    Ws = [_W(qd) for qd in qds]
    t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    work = decode_workspace("cuda")
    for T in (256, 512, 1024):
        print(f"split prefill {shapes} p={p} T={T}", flush=True)
        x = make_x(T, shapes[0][1], seed=T)
        y = linear_forward_multi(Ls, t, x.cuda(), work=work)
        y2 = linear_forward_multi(Ls, t, x.cuda(), work=work)
        y0 = linear_forward_multi(Ls, t, x.cuda(), work=None)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
        want = np.concatenate([x.float().numpy() @ W.T + (qd.bias.float().numpy() if qd.bias is not None else 0)
                               for qd, W in zip(qds, Ws)], axis=1)
        e = rel_l2(y.float().cpu().numpy(), want)
        e0 = rel_l2(y.float().cpu().numpy(), y0.float().cpu().numpy())
        print(f"  rel_l2 vs oracle {e:.2e}, vs unsplit {e0:.2e}", flush=True)
        assert e <= TOL and e0 <= 1e-3, (T, e, e0)


def test_module_prefill_uses_the_stream_workspace():
    print("EPTQLinear prefill at 512 tokens (stream workspace, split K)", flush=True)
    qd = make_layer(4096, 4096, seed=91, percmask=0.002)
    lin = EPTQLinear.from_quantized_data(qd, E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    x = make_x(512, 4096, seed=5)
    with torch.no_grad():
        y = lin(x.cuda())
        y2 = lin(x.cuda())
    torch.cuda.synchronize()
    assert torch.equal(y, y2)
    e = rel_l2(y.float().cpu().numpy(), x.float().numpy() @ _W(qd).T)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert e <= TOL
