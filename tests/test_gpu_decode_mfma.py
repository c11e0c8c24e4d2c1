"""GPU parity of the matrix-core E8-D4 decode (batches 5..16) at the edges of
its work split: a last tile with fewer than 8 block rows, N not a multiple of
the 64-column block, one S_group row per 64-row tile (qb = 64), more critical
blocks in a tile than the 256 staged in LDS, a bias at B = 16, and the
multi-layer launch (q|k|v with GQA widths).  Each output is within 1e-2
relative L2 of the fp32 reconstruct + matmul oracle."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import linear_forward, linear_forward_multi
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _run(qd, x):
    t = torch.from_numpy(table("e8_d4", 1.75)).half().cuda()
    ocol, orp = csr_dev(qd.Q)
    y = linear_forward("e8_d4", qd.Q.cuda(), t, qd.g.cuda(), qd.h.cuda(), x.cuda(), qd.O.cuda(), ocol, orp,
                       None if qd.bias is None else qd.bias.cuda(),
                       None if qd.S_group is None else qd.S_group.cuda())
    torch.cuda.synchronize()
    return y.float().cpu().numpy()


def _ref(qd, x):
    n = layer_np(qd)
    return linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4",
                      n["bias"], n["S_group"])


@pytest.mark.parametrize("out,inp,B,p,bias,qb", [
    (520, 776, 9, 0.002, False, None),      # last tile of 1 block row; 776 = 12 blocks + 8 columns
    (1024, 1000, 12, 0.002, True, 64),      # one S row per tile
    (512, 4096, 16, 0.02, True, None),      # ~650 critical blocks per tile (> 256 staged)
    (4096, 4096, 5, 0.001, False, None),
    (2048, 11008, 8, 0.001, False, None),   # down-projection width
    (768, 2048, 16, 0.002, True, 128),
])
def test_mfma_decode_rel_l2(out, inp, B, p, bias, qb):
    print(f"mfma decode {out}x{inp} B={B} p={p} bias={bias} qb={qb}", flush=True)
    qd = make_layer(out, inp, seed=out * 7 + inp + B, percmask=p, bias=bias, qb_size=qb)
    x = make_x(B, inp, seed=B + 3)
    y = _run(qd, x)
    e = rel_l2(y, _ref(qd, x))
    print(f"  rel_l2 {e:.2e}")
    assert np.isfinite(y).all() and e <= TOL


def test_mfma_decode_multi_layer_gqa():
    """q|k|v of different widths in one launch, each layer its own scales."""
    print("mfma decode q|k|v multi-layer", flush=True)
    q = E8D4Quantizer(radius=1.75)
    shapes = [(2048, 2048), (512, 2048), (512, 2048)]
    lins, qds = [], []
    for k, (o, i) in enumerate(shapes):
        qd = make_layer(o, i, seed=100 + k, percmask=0.002, qb_size=128)
        qds.append(qd)
        lins.append(EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda())
    for B in (4, 16):
        x = make_x(B, 2048, seed=B)
        layers = [dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr,
                       bias=l.bias, S_group=l.S_group) for l in lins]
        y = linear_forward_multi(layers, lins[0]._codebook, x.cuda()).float().cpu().numpy()
        want = np.concatenate([_ref(qd, x) for qd in qds], axis=1)
        assert rel_l2(y, want) <= TOL, B
        # Each layer's columns on their own as well.
        off = 0
        for qd, (o, _) in zip(qds, shapes):
            assert rel_l2(y[:, off:off + o], _ref(qd, x)) <= TOL
            off += o


def test_mfma_decode_batch_rows_independent():
    """Row b of a batch equals the same input run at B = 1 (the vector kernel)
    within fp16 output rounding: no batch row leaks into another."""
    print("mfma decode batch-row independence", flush=True)
    qd = make_layer(1024, 4096, seed=5, percmask=0.002, bias=True)
    x = make_x(16, 4096, seed=6)
    y16 = _run(qd, x)
    for b in (0, 7, 15):
        y1 = _run(qd, x[b:b + 1])
        assert rel_l2(y16[b:b + 1], y1) < 2e-3, b


@pytest.mark.parametrize("out,inp,B,qb", [
    (4096, 4096, 8, None),     # 64 tiles: columns split over 4 workgroups
    (1024, 11008, 16, 128),
    (520, 776, 6, None),       # 13 column blocks over 4 parts: some waves get none
])
def test_mfma_decode_split_columns(out, inp, B, qb):
    """With a workspace, a layer with few row tiles has each tile's columns
    split over several workgroups: the result matches the oracle and the
    unsplit launch (up to fp32 summation order), repeated calls are
    bit-identical, the counters are back at zero after each call, and graph
    replays (eager calls in between) reproduce the eager result."""
    from eptq_amd.kernels import decode_workspace
    print(f"mfma decode split columns {out}x{inp} B={B} qb={qb}", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qd = make_layer(out, inp, seed=out + 3 * inp, percmask=0.002, bias=True, qb_size=qb)
    lin = EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda()
    layers = [dict(Q=lin.Q, g=lin.g, h=lin.h, O_vals=lin.O_vals, O_col=lin.O_col, O_row_ptr=lin.O_row_ptr,
                   bias=lin.bias, S_group=lin.S_group)]
    x = make_x(B, inp, seed=9).cuda()
    work = decode_workspace(x.device)
    y0 = linear_forward_multi(layers, lin._codebook, x)
    y1 = linear_forward_multi(layers, lin._codebook, x, work=work)
    torch.cuda.synchronize()
    ref = _ref(qd, x.cpu())
    assert rel_l2(y1.float().cpu().numpy(), ref) <= TOL
    assert rel_l2(y1.float().cpu().numpy(), y0.float().cpu().numpy()) < 1e-3
    assert int(work[:65536].view(torch.int32).abs().sum()) == 0
    y2 = linear_forward_multi(layers, lin._codebook, x, work=work)
    assert torch.equal(y1, y2)
    yg = torch.empty_like(y1)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg.copy_(linear_forward_multi(layers, lin._codebook, x, work=work))
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        yg.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), rep
        assert torch.equal(linear_forward_multi(layers, lin._codebook, x, work=work), y1), rep
    assert int(work[:65536].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("shapes,B,qb", [
    ([(11008, 4096)] * 2, 8, None),    # gate|up: 344 tiles, more than one workgroup per CU
    ([(20480, 1024)], 16, 128),        # 320 tiles of one layer, S_group
])
def test_mfma_decode_tail_tiles_split(shapes, B, qb):
    """More tiles than CUs: the first round takes whole tiles and the tiles
    left for the second have their columns split.  Every layer matches the
    oracle and the launch without a workspace (up to fp32 summation order),
    repeated calls and graph replays are bit-identical, and the counters are
    back at zero."""
    from eptq_amd.kernels import decode_workspace
    print(f"mfma decode tail split {shapes} B={B} qb={qb}", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(o, i, seed=500 + k, percmask=0.002, bias=True, qb_size=qb) for k, (o, i) in enumerate(shapes)]
    lins = [EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds]
    layers = [dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr,
                   bias=l.bias, S_group=l.S_group) for l in lins]
    x = make_x(B, shapes[0][1], seed=11).cuda()
    work = decode_workspace(x.device)
    y0 = linear_forward_multi(layers, lins[0]._codebook, x)
    y1 = linear_forward_multi(layers, lins[0]._codebook, x, work=work)
    torch.cuda.synchronize()
    off = 0
    for qd, (o, _) in zip(qds, shapes):
        want = _ref(qd, x.cpu())
        assert rel_l2(y1[:, off:off + o].float().cpu().numpy(), want) <= TOL
        off += o
    assert rel_l2(y1.float().cpu().numpy(), y0.float().cpu().numpy()) < 1e-3
    assert int(work[:65536].view(torch.int32).abs().sum()) == 0
    assert torch.equal(linear_forward_multi(layers, lins[0]._codebook, x, work=work), y1)
    yg = torch.empty_like(y1)
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            yg.copy_(linear_forward_multi(layers, lins[0]._codebook, x, work=work))
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        yg.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, y1), rep
    assert int(work[:65536].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("B", [17, 40, 128])
def test_mfma_decode_row_slices(B):
    """17..128 rows through the multi-layer entry point: 16-row slices of the
    matrix-core kernel, every layer in each slice's launch, with and without
    the workspace; each layer within 1e-2 of the oracle, the two runs within
    fp32 summation order, repeated calls bit-identical, counters at zero."""
    from eptq_amd.kernels import decode_workspace
    print(f"mfma decode row slices B={B}", flush=True)
    q = E8D4Quantizer(radius=1.75)
    shapes = [(2048, 2048), (512, 2048), (512, 2048)]
    qds = [make_layer(o, i, seed=700 + k, percmask=0.002, bias=k == 0, qb_size=128) for k, (o, i) in enumerate(shapes)]
    lins = [EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds]
    layers = [dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr,
                   bias=l.bias, S_group=l.S_group) for l in lins]
    x = make_x(B, 2048, seed=B).cuda()
    work = decode_workspace(x.device)
    y0 = linear_forward_multi(layers, lins[0]._codebook, x)
    y1 = linear_forward_multi(layers, lins[0]._codebook, x, work=work)
    torch.cuda.synchronize()
    off = 0
    for qd, (o, _) in zip(qds, shapes):
        want = _ref(qd, x.cpu())
        assert rel_l2(y0[:, off:off + o].float().cpu().numpy(), want) <= TOL
        assert rel_l2(y1[:, off:off + o].float().cpu().numpy(), want) <= TOL
        off += o
    assert rel_l2(y1.float().cpu().numpy(), y0.float().cpu().numpy()) < 1e-3
    assert torch.equal(linear_forward_multi(layers, lins[0]._codebook, x, work=work), y1)
    assert int(work[:65536].view(torch.int32).abs().sum()) == 0


@pytest.mark.parametrize("n_layers,out,inp,B,work", [
    (3, 1024, 2048, 3, False),
    (3, 1024, 2048, 8, True),     # 48 tiles, each split over 4 parts
    (2, 4096, 1024, 5, True),
    (2, 1000, 1024, 8, False),    # last tile of 5 block rows
])
def test_mfma_decode_equal_layers(n_layers, out, inp, B, work):
    """Layers of equal shape in one launch (q|k|v, gate|up): within 1e-2 of
    the oracle, and without a workspace bit-identical to each layer launched
    on its own (same tiles, same sums, same order)."""
    from eptq_amd.kernels import decode_workspace
    print(f"mfma decode equal layers {n_layers}x{out}x{inp} B={B} work={work}", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(out, inp, seed=300 + 7 * k + B, percmask=0.002) for k in range(n_layers)]
    lins = [EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds]
    x = make_x(B, inp, seed=B + 40)
    layers = [dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr,
                   bias=l.bias, S_group=l.S_group) for l in lins]
    w = decode_workspace("cuda") if work else None
    y = linear_forward_multi(layers, lins[0]._codebook, x.cuda(), work=w)
    torch.cuda.synchronize()
    yn = y.float().cpu().numpy()
    want = np.concatenate([_ref(qd, x) for qd in qds], axis=1)
    e = rel_l2(yn, want)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert np.isfinite(yn).all() and e <= TOL
    if not work:
        alone = torch.cat([linear_forward_multi([L], lins[0]._codebook, x.cuda()) for L in layers], dim=1)
        assert torch.equal(y, alone)
