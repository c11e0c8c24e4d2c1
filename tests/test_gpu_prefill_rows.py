"""GPU parity of the prefill GEMM with the weights decoded in registers
(``k_gemm_rows_e8d4``: E8-D4, no S_group, more than 128 tokens, out_features
a multiple of 256; four-wave workgroups of 256 features, or five-wave ones of
320 when the layer fits one round of the CUs) through the C ABI's
``eptq_e8d4_forward``.  fp16 layers reach it when in_features is not a
multiple of 64 (the LDS-decode kernel takes the rest); bf16 layers always.

Every case is within 1e-2 relative L2 of the fp32 reconstruct + matmul
oracle (``dequantize_layer`` W, then an fp32 product).  The cases cover
token counts that are not a multiple of the 128-token tile, a bias, an odd
number of 32-column K-steps (1056 = 33 x 32), workgroups whose critical
blocks exceed the entries they stage in LDS (1024 for four-wave, 2048 for
five-wave workgroups; the rest are corrected after the K loop), and a layer
with no critical block at all.
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
    # out, in (an odd number of 32-column steps), tokens, critical-block fraction, bias
    (1024, 2080, 300, 0.002, True),
    (512, 1056, 257, 0.15, False),     # ~5000 entries per workgroup: past the LDS stage
    (256, 4128, 129, 0.0, True),       # no critical blocks
    (2048, 1056, 640, 0.01, False),
    (640, 1056, 300, 0.01, True),      # five-wave workgroups (80 Q-rows: two of 40)
    (640, 1056, 200, 0.1, False),      # five-wave, ~4200 entries per workgroup: past its 2048 in LDS
]


@pytest.mark.parametrize("out,inp,T,p,bias", CASES, ids=lambda v: str(v))
def test_prefill_rows_kernel_matches_oracle(out, inp, T, p, bias):
    print(f"prefill rows kernel {out}x{inp} T={T} p={p} bias={bias}", flush=True)
    qd = make_layer(out, inp, seed=700 + out + T, percmask=p, bias=bias)
    n = layer_np(qd)
    W = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4", None).astype(np.float32)
    x = make_x(T, inp, seed=701)
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


BF16_CASES = [
    # out, in, tokens, critical-block fraction, bias
    (1024, 2048, 300, 0.002, True),    # four-wave workgroups
    (640, 1024, 257, 0.05, False),     # five-wave workgroups, entries past their LDS stage
]


@pytest.mark.parametrize("out,inp,T,p,bias", BF16_CASES, ids=lambda v: str(v))
def test_prefill_rows_kernel_bf16(out, inp, T, p, bias):
    """bf16 x and y (the activation operand fp16(x·h·2^-e) from the exact
    fp32 product): within 2e-2 relative L2 of the fp32 oracle on the same bf16
    input, the bf16 output rounding included."""
    print(f"prefill rows kernel bf16 {out}x{inp} T={T} p={p} bias={bias}", flush=True)
    qd = make_layer(out, inp, seed=800 + out + T, percmask=p, bias=bias)
    n = layer_np(qd)
    W = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4", None).astype(np.float32)
    x = make_x(T, inp, seed=801).bfloat16()
    ref = x.float().numpy() @ W.T
    if qd.bias is not None:
        ref = ref + qd.bias.float().numpy()
    ocol, orp = csr_dev(qd.Q)
    codes = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    y = linear_forward("e8_d4", qd.Q.cuda(), codes, qd.g.cuda(), qd.h.cuda(), x.cuda(), qd.O.cuda(), ocol, orp,
                       None if qd.bias is None else qd.bias.cuda(), None)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16
    got = y.float().cpu().numpy()
    e = rel_l2(got, ref)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert e <= 2e-2
