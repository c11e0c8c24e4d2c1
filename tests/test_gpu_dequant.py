"""GPU parity: the HIP dequantizer is bit-exact with the oracle's dequantize_layer
(reference algorithms/eptq.py:406-471) on the same Q/g/h/O/S_group/table."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import dequant
from eptq_amd.synthetic import make_layer
from oracle.dequant import dequantize_layer

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu


def _run(kind, radius, qd):
    t = table(kind, radius)
    ocol, orp = csr_dev(qd.Q)
    W = dequant(kind, qd.Q.cuda(), torch.from_numpy(t).cuda(), qd.g.cuda(), qd.h.cuda(),
                qd.O.cuda(), ocol, orp, None if qd.S_group is None else qd.S_group.cuda())
    torch.cuda.synchronize()
    n = layer_np(qd)
    ref = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], t, kind, n["S_group"])
    return W.cpu().numpy(), ref


def _assert_bits(W, ref):
    a, b = W.view(np.uint16), ref.view(np.uint16)
    bad = np.argwhere(a != b)
    assert bad.size == 0, f"{len(bad)} mismatches, first at {bad[:3].tolist()}: {a[tuple(bad[0])]:#x} vs {b[tuple(bad[0])]:#x}"


@pytest.mark.parametrize("kind,radius", [("e8_d4", 1.75), ("e8_lattice", 1.6)])
@pytest.mark.parametrize("shape,p,qb", [((64, 256), 0.01, None), ((256, 1000), 0.002, None),
                                        ((512, 4096), 0.001, None), ((256, 512), 0.002, 128),
                                        ((3072, 768), 0.002, None), ((24, 20), 0.05, 8),
                                        ((11008, 4096), 0.001, None)])
def test_dequant_bit_exact(kind, radius, shape, p, qb):
    print(f"dequant {kind} {shape} p={p} qb={qb}", flush=True)
    qd = make_layer(*shape, seed=shape[0] * 7 + shape[1] + len(kind), percmask=p, qb_size=qb)
    W, ref = _run(kind, radius, qd)
    _assert_bits(W, ref)


def test_dequant_subnormal_outputs():
    print("dequant subnormals", flush=True)
    qd = make_layer(128, 512, seed=5, percmask=0.01)
    qd.g = (qd.g.float() * 1e-5).half()     # pushes W into the fp16 subnormal range
    W, ref = _run("e8_d4", 1.75, qd)
    assert (np.abs(ref.astype(np.float32)) < 6.1e-5).mean() > 0.5
    _assert_bits(W, ref)


def test_dequant_all_indices_roundtrip():
    """An index sweep over all 65535 codes with g = h = 1 dumps the table."""
    print("dequant sweep", flush=True)
    u = torch.arange(65535, dtype=torch.int32)
    Q = (u - 32768).to(torch.int16).reshape(1, 65535)
    from eptq_amd.config import QuantizedLayerData
    qd = QuantizedLayerData(Q=Q.contiguous(), g=torch.ones(8, dtype=torch.float16),
                            h=torch.ones(65535, dtype=torch.float16),
                            O=torch.zeros((0, 8), dtype=torch.float16))
    for kind, r in (("e8_d4", 1.75), ("e8_lattice", 1.6)):
        W, ref = _run(kind, r, qd)
        _assert_bits(W, ref)


def test_dequant_markers_first_last_column_and_full_rows():
    print("dequant marker edges", flush=True)
    qd = make_layer(64, 64, seed=9, percmask=0.0)
    Q = qd.Q.clone()
    Q[:, 0] = 32767
    Q[:, -1] = 32767
    Q[3, :] = 32767
    nnz = int((Q == 32767).sum())
    qd.Q = Q
    qd.O = torch.randn((nnz, 8)).half()
    for kind, r in (("e8_d4", 1.75), ("e8_lattice", 1.6)):
        W, ref = _run(kind, r, qd)
        _assert_bits(W, ref)
