"""GPU parity of ``eptq_llama_linear``: the matrix-core decode Linear with the
decoder's RMSNorm folded in (the weights multiplied by norm_w ⊙ x, the sums by
1/rms(x) per batch row) and the residual add at its output.

* With the norm: within 1e-2 relative L2 of the oracle (fp64 RMSNorm, then
  the fp32 reconstruct + matmul of ``linear_ref``), and within 3e-3 of the
  two-launch form (``eptq_llama_rmsnorm`` then the multi-layer Linear), for
  q|k|v-like launches (whole tiles, and with the workspace split over
  parts), a gate|up-like launch with more tiles than CUs (whole tiles, then
  split ones: the parts' x² sums meet in the workspace), and one S_group row
  per 128 output rows.
* With the residual: bit-identical to the Linear followed by the fp16 add,
  with resid a separate tensor and with resid = y (in place).
* EPTQ_EUNSUPPORTED (never a silent wrong result) where the kernel does not
  take the norm: B = 9, N not a multiple of 64.
"""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import _lib, decode_workspace
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.llama import _layer_array, rmsnorm_
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _lins(shapes, seed, qb=None):
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(o, i, seed=seed + k, percmask=0.002, qb_size=qb) for k, (o, i) in enumerate(shapes)]
    return qds, [EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds]


def _call(lins, x, norm_w=None, resid=None, y=None, work=None):
    arr, width = _layer_array(lins)
    B, N = x.shape
    if y is None:
        y = torch.empty((B, width), dtype=torch.float16, device="cuda")
    rc = _lib.load().eptq_llama_linear(
        len(arr), arr, lins[0]._codebook.data_ptr(), x.data_ptr(), N, B,
        None if norm_w is None else norm_w.data_ptr(), EPS, None if resid is None else resid.data_ptr(),
        y.data_ptr(), width, None if work is None else work.data_ptr(), 0 if work is None else work.numel(),
        torch.cuda.current_stream().cuda_stream)
    return rc, y


def _plain(lins, x, work=None):
    """The multi-layer Linear on its own (eptq_e8d4_forward_multi)."""
    arr, width = _layer_array(lins)
    B, N = x.shape
    y = torch.empty((B, width), dtype=torch.float16, device="cuda")
    rc = _lib.load().eptq_e8d4_forward_multi(
        len(arr), arr, lins[0]._codebook.data_ptr(), _lib.EPTQ_F16, x.data_ptr(), _lib.EPTQ_F16, N, B,
        y.data_ptr(), width, None if work is None else work.data_ptr(), 0 if work is None else work.numel(),
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "eptq_e8d4_forward_multi")
    return y


def _oracle(qds, x, w):
    xf = x.double().numpy()
    t = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + EPS) * w.double().numpy()
    outs = []
    for qd in qds:
        n = layer_np(qd)
        outs.append(linear_ref(t, n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4",
                               n["bias"], n["S_group"]))
    return np.concatenate(outs, axis=1)


def _norm_w(N, seed):
    gen = torch.Generator().manual_seed(seed)
    return (0.5 + torch.rand(N, generator=gen)).half()


@pytest.mark.parametrize("shapes,N,B,qb,use_work", [
    ([(1024, 1024), (256, 1024), (256, 1024)], 1024, 3, None, False),   # q|k|v-like, whole tiles
    ([(1024, 1024), (256, 1024), (256, 1024)], 1024, 8, None, True),    # split over parts
    ([(11008, 1024), (11008, 1024)], 1024, 8, None, True),              # gate|up-like: 344 tiles
    ([(2048, 4096)], 4096, 5, 128, True),                                # S_group, one row per 128 rows
    ([(1024, 1024), (1024, 1024), (1024, 1024)], 1024, 8, None, True),  # three equal layers, split over parts
    ([(1024, 2048), (1024, 2048)], 2048, 4, None, False),               # two equal layers, whole tiles
])
def test_llama_linear_norm(shapes, N, B, qb, use_work):
    print(f"eptq_llama_linear norm {shapes} B={B} qb={qb} work={use_work}", flush=True)
    qds, lins = _lins(shapes, seed=N + B, qb=qb)
    x = make_x(B, N, seed=B + 11) * 3
    w = _norm_w(N, seed=N)
    work = decode_workspace("cuda") if use_work else None
    xd, wd = x.cuda(), w.cuda()
    rc, y = _call(lins, xd, norm_w=wd, work=work)
    _lib.check(rc, "eptq_llama_linear")
    torch.cuda.synchronize()
    yn = y.float().cpu().numpy()
    e = rel_l2(yn, _oracle(qds, x, w))
    # The two-launch form: RMSNorm to fp16, then the Linear.
    t = rmsnorm_(xd.clone(), None, wd, EPS)
    y2 = _plain(lins, t, work).float().cpu().numpy()
    e2 = rel_l2(yn, y2)
    print(f"  rel_l2 vs oracle {e:.2e}, vs rmsnorm + Linear {e2:.2e}", flush=True)
    assert np.isfinite(yn).all() and e <= 1e-2 and e2 <= 3e-3


@pytest.mark.parametrize("B,use_work", [(4, True), (8, False)])
def test_llama_linear_residual(B, use_work):
    print(f"eptq_llama_linear residual B={B} work={use_work}", flush=True)
    _, lins = _lins([(1024, 2048)], seed=70 + B)
    x = make_x(B, 2048, seed=B).cuda()
    r = make_x(B, 1024, seed=B + 100).cuda() * 4
    work = decode_workspace("cuda") if use_work else None
    want = (r.float() + _plain(lins, x, work).float()).half()
    rc, y = _call(lins, x, resid=r, work=work)
    _lib.check(rc, "eptq_llama_linear")
    assert torch.equal(y, want)
    # In place: the residual buffer is y.
    r2 = r.clone()
    rc, y2 = _call(lins, x, resid=r2, y=r2, work=work)
    _lib.check(rc, "eptq_llama_linear")
    torch.cuda.synchronize()
    assert y2.data_ptr() == r2.data_ptr() and torch.equal(r2, want)


def test_llama_linear_norm_unsupported():
    _, lins = _lins([(512, 1024)], seed=5)
    w = _norm_w(1024, seed=1).cuda()
    x = make_x(9, 1024, seed=2).cuda()
    rc, _ = _call(lins, x, norm_w=w)
    assert rc == _lib.EPTQ_EUNSUPPORTED
    _, lins2 = _lins([(512, 1000)], seed=6)
    x2 = make_x(4, 1000, seed=3).cuda()
    rc, _ = _call(lins2, x2, norm_w=_norm_w(1000, seed=2).cuda())
    assert rc == _lib.EPTQ_EUNSUPPORTED


def _swiglu(lins, x, norm_w, work):
    arr, width = _layer_array(lins)
    B, N = x.shape
    gu = torch.empty((B, width), dtype=torch.float16, device="cuda")
    act = torch.empty((B, width // 2), dtype=torch.float16, device="cuda")
    rc = _lib.load().eptq_llama_linear_swiglu(
        arr, lins[0]._codebook.data_ptr(), x.data_ptr(), N, B, None if norm_w is None else norm_w.data_ptr(), EPS,
        gu.data_ptr(), act.data_ptr(), work.data_ptr(), work.numel(), torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "eptq_llama_linear_swiglu")
    return gu, act


@pytest.mark.parametrize("F,N,Bs,norm", [
    (11008, 4096, (8, 5), True),    # Llama-2-7B gate|up: 344 tiles, whole then split over parts
    (1024, 1024, (3, 2), False),    # 32 tiles, every tile split
    (2048, 2048, (16, 9), False),   # B = 16
    (512, 1024, (4, 3), True),
])
def test_llama_linear_swiglu(F, N, Bs, norm):
    """The SwiGLU form: gu bit-identical to eptq_llama_linear, the product
    bit-identical to eptq_llama_silu_mul of it, on two calls in a row (the
    second smaller: the pair counters return to zero)."""
    from eptq_amd.llama import silu_mul
    _, lins = _lins([(F, N), (F, N)], seed=F + N)
    w = _norm_w(N, seed=N + 1).cuda() if norm else None
    work = decode_workspace("cuda")
    for B in Bs:
        print(f"eptq_llama_linear_swiglu F={F} N={N} B={B} norm={norm}", flush=True)
        x = (make_x(B, N, seed=B + 3) * 2).cuda()
        gu, act = _swiglu(lins, x, w, work)
        rc, want_gu = _call(lins, x, norm_w=w, work=work)
        _lib.check(rc, "eptq_llama_linear")
        want_act = silu_mul(want_gu)
        torch.cuda.synchronize()
        assert torch.equal(gu, want_gu)
        assert torch.equal(act, want_act)
        assert torch.isfinite(act.float()).all() and act.float().abs().max() > 0
    tiles = 2 * ((F // 8 + 7) // 8)
    assert int(work[: 4 * (tiles + tiles // 2)].view(torch.int32).abs().sum()) == 0
