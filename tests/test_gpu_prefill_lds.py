"""GPU parity of the prefill GEMM that decodes the weight tile into LDS
(``k_gemm_lds_e8d4``: E8-D4, fp16 x, no S_group, more than 128 tokens,
in_features a multiple of 64, out_features a multiple of 64 or 160) through
the C ABI's ``eptq_e8d4_forward``.

Every case is within 1e-2 relative L2 of the fp32 reconstruct + matmul
oracle (``dequantize_layer`` W, then an fp32 product).  The cases cover the
four tile widths (160 features when out_features / 160 gives fewer rounds
of the CUs; else 128 when 0.8 x its rounds is below the 256-feature tiles'
rounds, and 64 in its place when that is still one round; else 256), token
counts that are not a multiple of the 256-token tile, one and two K-steps,
a bias, a layer with no critical block, workgroups whose critical blocks
exceed the entries they stage in LDS (2272 for 160-feature, 3712 for
64-feature, 2784 for 128-feature, 944 for 256-feature tiles; the rest are
corrected after the K loop), and h below and far above 1 (the 2^-e scaling
of the table).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels import linear_forward
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2

CASES = [
    # out, in, tokens, critical-block fraction, bias, h scale
    (1280, 2048, 512, 0.002, True, 1.0),     # 160-feature tiles (8 of them beat 5 of 256)
    (1024, 2048, 300, 0.002, True, 1.0),     # 64-feature tiles (1024 / 160 is not whole; one round)
    (512, 1024, 257, 0.15, False, 1.0),      # 64: ~1200 entries per workgroup
    (256, 4096, 300, 0.15, False, 1.0),      # 64: ~4900 entries per workgroup, past its 3712
    (4096, 1024, 1280, 0.002, True, 1.0),    # 128: 320 tiles of 64 would take two rounds
    (4096, 1024, 1280, 0.2, False, 1.0),     # 128: ~3300 entries per workgroup, past its 2784
    (1024, 2048, 12800, 0.002, True, 1.0),   # 256: 200 tiles (one round) against 400 of 128 (two)
    (1024, 2048, 12800, 0.15, False, 1.0),   # 256: ~9800 entries per workgroup, past its 944
    (640, 1024, 200, 0.15, False, 1.0),      # 160: ~3100 entries per workgroup, past its 2272
    (160, 8256, 129, 0.02, True, 1.0),       # 160, 129 K-steps: ~3300 entries, past its 2272
    (2560, 1024, 129, 0.0, True, 1.0),       # no critical blocks, one token past a tile
    (256, 64, 300, 0.01, False, 1.0),        # one K-step
    (160, 128, 1000, 0.01, True, 1.0),       # two K-steps, four token tiles
    (1280, 1024, 384, 0.01, False, 0.05),    # max |h| < 1: no table scaling
    (1280, 1024, 384, 0.01, True, 300.0),    # max |h| ~ 1000: table scaled by 2^-10
]


@pytest.mark.parametrize("out,inp,T,p,bias,hs", CASES, ids=lambda v: str(v))
def test_prefill_lds_kernel_matches_oracle(out, inp, T, p, bias, hs):
    print(f"prefill lds kernel {out}x{inp} T={T} p={p} bias={bias} h*{hs}", flush=True)
    qd = make_layer(out, inp, seed=900 + out + T, percmask=p, bias=bias)
    if hs != 1.0:
        qd.h = (qd.h.float() * hs).half()
    n = layer_np(qd)
    W = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4", None).astype(np.float32)
    x = make_x(T, inp, seed=901)
    ref = x.float().numpy() @ W.T
    if qd.bias is not None:
        ref = ref + qd.bias.float().numpy()
    ocol, orp = csr_dev(qd.Q)
    codes = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    y = linear_forward("e8_d4", qd.Q.cuda(), codes, qd.g.cuda(), qd.h.cuda(), x.cuda(), qd.O.cuda(), ocol, orp,
                       None if qd.bias is None else qd.bias.cuda(), None)
    torch.cuda.synchronize()
    got = y.float().cpu().numpy()
    e = rel_l2(got, ref)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert e <= TOL


def test_prefill_lds_kernel_graph_replays_match_eager():
    """Captured in a HIP graph, the kernel's replays (with new x copied in and
    eager launches between them) equal eager launches bit for bit: it keeps no
    state between calls and records no memset."""
    out, inp, T = 1280, 1024, 300
    print(f"prefill lds kernel graph replay {out}x{inp} T={T}", flush=True)
    qd = make_layer(out, inp, seed=950, percmask=0.01, bias=True)
    ocol, orp = csr_dev(qd.Q)
    codes = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    args = [qd.Q.cuda(), codes, qd.g.cuda(), qd.h.cuda()]
    rest = [qd.O.cuda(), ocol, orp, qd.bias.cuda(), None]
    x_static = make_x(T, inp, seed=951).cuda()
    linear_forward("e8_d4", *args, x_static, *rest)   # first call sets the LDS attribute
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y_static = linear_forward("e8_d4", *args, x_static, *rest)
    for rep in range(3):
        x_new = make_x(T, inp, seed=960 + rep).cuda()
        x_static.copy_(x_new)
        g.replay()
        eager = linear_forward("e8_d4", *args, x_new, *rest)
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager), f"replay {rep} differs from the eager launch"
