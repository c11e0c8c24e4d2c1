"""GPU parity: the fused HIP quantized Linear (decode matvec B<=16, GEMM above)
is within 1e-2 relative L2 of the fp32 reconstruct+matmul reference
(oracle.matvec.linear_ref), on the benchmark configurations' layer distributions (g, h, x, O)."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import linear_forward
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import fused_ref64, linear_ref, rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2   # relative L2 vs fp32 reconstruct + matmul


def _gpu(kind, radius, qd, x, codes_dtype=torch.float16):
    t = torch.from_numpy(table(kind, radius)).to(codes_dtype).cuda()
    ocol, orp = csr_dev(qd.Q)
    y = linear_forward(kind, qd.Q.cuda(), t, qd.g.cuda(), qd.h.cuda(), x.cuda(), qd.O.cuda(),
                       ocol, orp, None if qd.bias is None else qd.bias.cuda(),
                       None if qd.S_group is None else qd.S_group.cuda())
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


def _refs(kind, radius, qd, x):
    n = layer_np(qd)
    xf = x.float().numpy()
    args = (n["Q"], n["g"], n["h"], n["O"], table(kind, radius), kind, n["bias"], n["S_group"])
    return linear_ref(xf, *args), fused_ref64(xf, *args)


CASES = [
    # (kind, radius, out, in, B, percmask, bias, qb)
    ("e8_d4", 1.75, 4096, 4096, 1, 0.001, False, None),
    ("e8_d4", 1.75, 4096, 4096, 8, 0.001, False, None),
    ("e8_d4", 1.75, 11008, 4096, 1, 0.001, False, None),
    ("e8_d4", 1.75, 4096, 11008, 1, 0.001, False, None),
    ("e8_d4", 1.75, 1024, 4096, 4, 0.002, False, 128),
    ("e8_d4", 1.75, 4096, 4096, 16, 0.002, False, 128),
    ("e8_d4", 1.75, 512, 14336, 3, 0.002, False, 128),
    # Llama-3-8B gate/up and down (benchmark configuration 2) at full size.
    ("e8_d4", 1.75, 14336, 4096, 1, 0.002, False, 128),
    ("e8_d4", 1.75, 4096, 14336, 16, 0.002, False, 128),
    ("e8_d4", 1.75, 1376 * 8 // 8, 768, 5, 0.01, True, None),
    ("e8_lattice", 1.6, 3072, 768, 1, 0.002, True, None),
    ("e8_lattice", 1.6, 512, 4096, 7, 0.002, False, None),
    ("e8_lattice", 1.6, 256, 1024, 2, 0.01, False, 64),
    ("e8_d4", 1.75, 512, 1024, 40, 0.002, True, None),
    ("e8_lattice", 1.6, 256, 512, 33, 0.002, False, None),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: f"{c[0]}-{c[2]}x{c[3]}-B{c[4]}-qb{c[7]}")
def test_linear_rel_l2(case):
    kind, r, out, inp, B, p, bias, qb = case
    print(f"linear {case}", flush=True)
    qd = make_layer(out, inp, seed=out + inp + B, percmask=p, bias=bias, qb_size=qb)
    x = make_x(B, inp, seed=B + 17)
    y = _gpu(kind, r, qd, x)
    ref32, ref64 = _refs(kind, r, qd, x)
    e32, e64 = rel_l2(y, ref32), rel_l2(y, ref64)
    print(f"  rel_l2 vs fp32 reconstruct {e32:.2e}, vs fp64 fused {e64:.2e}")
    assert e32 <= TOL and e64 <= TOL


@pytest.mark.parametrize("kind,r", [("e8_d4", 1.75), ("e8_lattice", 1.6)])
def test_fp32_codebook_and_bf16(kind, r):
    print(f"linear fp32 codes / bf16 {kind}", flush=True)
    qd = make_layer(512, 2048, seed=3, percmask=0.002, bias=True)
    x = make_x(2, 2048, seed=4)
    y16 = _gpu(kind, r, qd, x)
    y32 = _gpu(kind, r, qd, x, codes_dtype=torch.float32)
    ybf = _gpu(kind, r, qd, x.bfloat16())
    ref32, _ = _refs(kind, r, qd, x)
    assert rel_l2(y16, ref32) <= TOL
    assert rel_l2(y32, ref32) <= TOL
    assert rel_l2(ybf, ref32) <= 2e-2   # bf16 input and output rounding


def test_zero_input_gives_bias_and_linearity():
    print("linear properties", flush=True)
    qd = make_layer(4096, 4096, seed=11, percmask=0.001, bias=True)
    x1 = make_x(2, 4096, seed=1)
    x2 = make_x(2, 4096, seed=2)
    y0 = _gpu("e8_d4", 1.75, qd, torch.zeros_like(x1))
    np.testing.assert_array_equal(y0, np.broadcast_to(qd.bias.float().numpy(), y0.shape))
    ya = _gpu("e8_d4", 1.75, qd, x1)
    yb = _gpu("e8_d4", 1.75, qd, x2)
    # Bias-free linearity in x (up to fp16 rounding of x1 + x2 and of y).
    yab = _gpu("e8_d4", 1.75, qd, (x1.float() + x2.float()).half())
    b = qd.bias.float().numpy()
    assert rel_l2(yab - b, (ya - b) + (yb - b)) < 5e-3


def test_no_critical_blocks_and_empty_rows():
    print("linear nnz=0", flush=True)
    qd = make_layer(256, 1024, seed=21, percmask=0.0)
    x = make_x(1, 1024, seed=22)
    y = _gpu("e8_d4", 1.75, qd, x)
    ref32, _ = _refs("e8_d4", 1.75, qd, x)
    assert rel_l2(y, ref32) <= TOL


def test_dense_markers():
    print("linear dense markers", flush=True)
    qd = make_layer(64, 512, seed=31, percmask=0.0)
    Q = qd.Q.clone()
    Q[:, ::3] = 32767          # a third of all blocks critical, many per row
    Q[5, :] = 32767            # one row entirely critical
    qd.Q = Q
    qd.O = torch.randn((int((Q == 32767).sum()), 8)).half()
    for kind, r in (("e8_d4", 1.75), ("e8_lattice", 1.6)):
        for B in (1, 16):
            x = make_x(B, 512, seed=B)
            y = _gpu(kind, r, qd, x)
            ref32, _ = _refs(kind, r, qd, x)
            assert rel_l2(y, ref32) <= TOL
