"""GPU: the allocation-free multi-layer entry point
(``eptq_e8d4_forward_multi_noalloc``) against ``eptq_e8d4_forward_multi``
with a caller workspace, through the C ABI.

Two calls in a row, the second with a smaller input (fewer layers, fewer
rows, a narrower x), both at batch sizes that take the matrix-core decode
kernel with its columns split over several workgroups, so the partial sums
and tile counters go through the library's static scratch.  With a workspace
of the scratch's size both entry points choose the same split, so the
outputs are bit-identical; both are also within 1e-2 relative L2 of the fp32
reconstruct + matmul oracle.  A third call at 24 rows (two 16-row slices
launched back to back on the same scratch) checks that a launch finds the
counters the previous one returned to zero.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from eptq_amd.kernels import _lib, decode_workspace
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2
SCRATCH_BYTES = 1130496   # EPTQ_NOALLOC_SCRATCH_BYTES


def _layers(shapes, seed):
    out = []
    for k, (o, i) in enumerate(shapes):
        qd = make_layer(o, i, seed=seed + k, percmask=0.002, bias=k == 1)
        n = layer_np(qd)
        W = dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4", None)
        ocol, orp = csr_dev(qd.Q)
        d = dict(Q=qd.Q.cuda(), g=qd.g.cuda(), h=qd.h.cuda(), O_vals=qd.O.cuda(), O_col=ocol, O_row_ptr=orp,
                 bias=None if qd.bias is None else qd.bias.cuda())
        out.append((d, W.astype(np.float32), None if qd.bias is None else qd.bias.float().numpy()))
    return out


def _arr(layers):
    arr = (_lib.EptqLayer * len(layers))()
    off = 0
    for i, (d, _, _) in enumerate(layers):
        M = int(d["Q"].shape[0])
        p = lambda t: None if t is None or t.numel() == 0 else t.data_ptr()
        arr[i] = _lib.EptqLayer(p(d["Q"]), p(d["g"]), p(d["h"]), p(d["O_vals"]), p(d["O_col"]),
                                p(d["O_row_ptr"]), p(d["bias"]), None, 0, M, off)
        off += 8 * M
    return arr, off


def _call(layers, codes, x, work=None, noalloc=False):
    lib = _lib.load()
    arr, width = _arr(layers)
    B, N = x.shape
    y = torch.full((B, width), float("nan"), dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.eptq_e8d4_forward_multi_noalloc(len(layers), arr, codes.data_ptr(), _lib.EPTQ_F16, x.data_ptr(),
                                                 _lib.EPTQ_F16, N, B, y.data_ptr(), width, stream)
        _lib.check(rc, "eptq_e8d4_forward_multi_noalloc")
    else:
        rc = lib.eptq_e8d4_forward_multi(len(layers), arr, codes.data_ptr(), _lib.EPTQ_F16, x.data_ptr(),
                                         _lib.EPTQ_F16, N, B, y.data_ptr(), width, work.data_ptr(), work.numel(),
                                         stream)
        _lib.check(rc, "eptq_e8d4_forward_multi")
    torch.cuda.synchronize()
    return y


def _oracle(layers, x):
    xf = x.float().cpu().numpy()
    cols = []
    for _, W, b in layers:
        y = xf @ W.T
        cols.append(y if b is None else y + b)
    return np.concatenate(cols, axis=1)


def _check(tag, layers, codes, x, same_split):
    work = decode_workspace("cuda")
    print(f"{tag}: {len(layers)} layers, x {tuple(x.shape)}, workspace {work.numel()} B", flush=True)
    want = _call(layers, codes, x, work=work)
    got = _call(layers, codes, x, noalloc=True)
    e = rel_l2(got.float().cpu().numpy(), _oracle(layers, x))
    print(f"  noalloc vs oracle rel_l2 {e:.2e}; bit-identical to the workspace form: {torch.equal(got, want)}",
          flush=True)
    assert torch.isfinite(got).all()
    assert e <= TOL
    if same_split:
        assert torch.equal(got, want)
    else:
        assert rel_l2(got.float().cpu().numpy(), want.float().cpu().numpy()) <= 1e-3


def test_noalloc_matches_workspace_form_on_two_calls():
    lib = _lib.load()
    same_split = int(lib.eptq_e8d4_work_bytes()) <= SCRATCH_BYTES
    codes = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    # Call 1: q|k|v-like, 96 tiles at batch 8 (columns split over 2 workgroups).
    big = _layers([(4096, 4096), (1024, 4096), (1024, 4096)], seed=500)
    _check("call 1", big, codes, make_x(8, 4096, seed=51).cuda(), same_split)
    # Call 2, smaller: two 1024x2048 layers, 32 tiles at batch 6 (split 4 ways).
    small = _layers([(1024, 2048), (1024, 2048)], seed=600)
    _check("call 2", small, codes, make_x(6, 2048, seed=52).cuda(), same_split)
    # Call 3: 24 rows = two 16-row slices, one after the other on the scratch.
    _check("call 3", small, codes, make_x(24, 2048, seed=53).cuda(), same_split)
