"""GPU parity for the prefill path (batch > 16): E8-D4 launches of up to 128
tokens run as 16-token slices of the matrix-core decode kernel, larger ones
(and E8) the dequant-to-LDS MFMA GEMM; both within 1e-2 relative L2 of the
fp32 reconstruct+matmul reference (oracle.matvec.linear_ref), including
critical blocks, S_group, bias, a ragged last slice and partial token
tiles."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import linear_forward
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _run(qd, x, kind="e8_d4", radius=1.75):
    t = torch.from_numpy(table(kind, radius)).half().cuda()
    ocol, orp = csr_dev(qd.Q)
    y = linear_forward(kind, qd.Q.cuda(), t, qd.g.cuda(), qd.h.cuda(), x.cuda(), qd.O.cuda(),
                       ocol, orp, None if qd.bias is None else qd.bias.cuda(),
                       None if qd.S_group is None else qd.S_group.cuda())
    torch.cuda.synchronize()
    n = layer_np(qd)
    ref = linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], n["O"], table(kind, radius), kind,
                     n["bias"], n["S_group"])
    return y.float().cpu().numpy(), ref


@pytest.mark.parametrize("out,inp,T,p,bias,qb", [
    (1024, 1024, 128, 0.002, False, None),     # 8 slices of 16 tokens
    (1024, 1024, 256, 0.002, False, None),     # GEMM: two whole token tiles
    (1024, 2048, 300, 0.002, True, None),      # partial token tile
    (2048, 1024, 64, 0.01, False, 128),        # S_group, more critical blocks
    (512, 512, 17, 0.002, False, None),        # just above the matvec range: a 1-token last slice
    (256, 4096, 1000, 0.05, True, 64),         # dense markers: > LDS entry cap per tile
    (1152, 1024, 200, 0.002, True, 128),       # 144 Q-rows: 9 row tiles, S_group and bias
])
def test_gemm_rel_l2(out, inp, T, p, bias, qb):
    print(f"gemm {out}x{inp} T={T} p={p} bias={bias} qb={qb}", flush=True)
    qd = make_layer(out, inp, seed=out + T, percmask=p, bias=bias, qb_size=qb)
    x = make_x(T, inp, seed=T)
    y, ref = _run(qd, x)
    e = rel_l2(y, ref)
    print(f"  rel_l2 {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("out,inp,T,p,bias,qb", [
    (1024, 1024, 128, 0.002, False, None),
    (3072, 768, 64, 0.002, True, None),        # OPT-125m fc1 (configuration 0) at 64 tokens
    (2048, 1024, 300, 0.01, False, 128),       # S_group, partial token tile
    (256, 4096, 200, 0.05, True, None),        # dense markers: > LDS entry cap per tile
])
def test_gemm_e8_rel_l2(out, inp, T, p, bias, qb):
    """E8-lattice layers at prefill batch sizes take the same MFMA GEMM with
    table rows gathered from global memory."""
    print(f"gemm e8 {out}x{inp} T={T} p={p} bias={bias} qb={qb}", flush=True)
    qd = make_layer(out, inp, seed=out + 3 * T, percmask=p, bias=bias, qb_size=qb)
    x = make_x(T, inp, seed=T + 1)
    y, ref = _run(qd, x, kind="e8_lattice", radius=1.6)
    e = rel_l2(y, ref)
    print(f"  rel_l2 {e:.2e}")
    assert e <= TOL


def test_gemm_config3_shape():
    """Llama-2-13B q/k/v/o layer, 2048 tokens (the prefill benchmark shape)."""
    print("gemm 5120x5120 T=2048", flush=True)
    qd = make_layer(5120, 5120, seed=3000, percmask=0.002)
    x = make_x(2048, 5120, seed=3001)
    y, ref = _run(qd, x)
    e = rel_l2(y, ref)
    print(f"  rel_l2 {e:.2e}")
    assert e <= TOL


def test_gemm_markers_in_every_step_and_column_edges():
    print("gemm marker edges", flush=True)
    qd = make_layer(256, 1024, seed=77, percmask=0.0)
    Q = qd.Q.clone()
    Q[:, 0] = 32767
    Q[:, 31] = 32767
    Q[:, 32] = 32767
    Q[:, -1] = 32767
    Q[7, ::2] = 32767             # a row with critical blocks in every column pair
    qd.Q = Q
    qd.O = torch.randn((int((Q == 32767).sum()), 8)).half()
    x = make_x(130, 1024, seed=5)
    y, ref = _run(qd, x)
    e = rel_l2(y, ref)
    assert e <= TOL
    # The critical blocks really carry O: against the product that decodes
    # every marker as the table's reserved row instead, the error is far larger.
    n = layer_np(qd)
    tab = table("e8_d4", 1.75)
    wrong_O = np.tile(np.concatenate([tab[511], tab[511]]), (n["O"].shape[0], 1)).astype(np.float16)
    wrong = linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], wrong_O, tab, "e8_d4", n["bias"], n["S_group"])
    assert rel_l2(y, wrong) > 10 * e
