"""GPU parity of the drop-in module's prefill (many-token) forward.

``EPTQLinear`` and ``EPTQMultiLinear`` send every token count to this
library's own kernels — 16-row slices of the matrix-core decode up to 128
rows, the prefill GEMMs that decode weight tiles into LDS or registers above
(the reference's module does the same with its fused GEMM,
``kernels/linear.py:199-210`` → ``csrc/eptq_kernels.cu:520-537``), and from
2048 fp16 tokens (256 for E8-D4 layers with S_group or bf16 x, 64 for E8
layers) the two-pass prefill (``eptq_e8d4_dequant`` / ``eptq_e8_dequant`` into a
transient fp16 W, then ``eptq_f16_gemm``).  Checks:

* within 1e-2 relative L2 of the fp32 reconstruct + matmul oracle (the
  north-star tolerance) at both sides of the 128-row switch;
* no torch GEMM runs inside the forward (``F.linear`` / ``torch.matmul``
  raise while the module is called), and the forward leaves only its output
  allocated (the two-pass prefill's W is freed on return);
* at 2048+ tokens (two-pass) within 3e-3 of the fused prefill kernel on the
  same layers;
* multi-layer stacking (GQA q|k|v with a bias on one layer only), S_group,
  E8 layers, dense critical blocks, bf16 input.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from eptq_amd.kernels import stream_workspace
from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _quantizer(kind, r):
    return E8D4Quantizer(radius=r) if kind == "e8_d4" else E8LatticeQuantizer(radius=r)


class _NoTorchGemm:
    """Makes torch's dense products raise while active."""

    def __enter__(self):
        self.saved = (F.linear, torch.matmul, torch.mm)

        def boom(*a, **k):
            raise AssertionError("a torch GEMM ran inside the quantized forward")
        F.linear = torch.matmul = torch.mm = boom
        return self

    def __exit__(self, *exc):
        F.linear, torch.matmul, torch.mm = self.saved
        return False


def _check(mod, qds, kind, r, T, seed, dtype=torch.float16):
    x = make_x(T, qds[0].Q.shape[1], seed=seed).to(dtype)
    stream_workspace("cuda")          # the stream's split-K workspace exists before the count
    torch.cuda.synchronize()
    before = torch.cuda.memory_allocated()
    with torch.no_grad(), _NoTorchGemm():
        y = mod(x.cuda())
    torch.cuda.synchronize()
    grown = torch.cuda.memory_allocated() - before     # the output alone (allocator rounding aside)
    y_bytes = y.numel() * y.element_size()
    assert grown <= y_bytes + 65536, f"forward left {grown} bytes allocated for a {y_bytes}-byte output"
    assert y.dtype == dtype and y.shape == (T, sum(8 * qd.Q.shape[0] for qd in qds))
    ref = np.concatenate([linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], n["O"], table(kind, r), kind,
                                     n["bias"], n["S_group"]) for n in map(layer_np, qds)], axis=1)
    e = rel_l2(y.float().cpu().numpy(), ref)
    print(f"  rel_l2 vs fp32 oracle {e:.2e}", flush=True)
    assert e <= (TOL if dtype == torch.float16 else 2 * TOL)
    return y


@pytest.mark.parametrize("kind,r,out,inp,T,p,bias,qb", [
    ("e8_d4", 1.75, 1024, 2048, 64, 0.002, True, None),     # matrix-core decode slices
    ("e8_d4", 1.75, 1024, 2048, 128, 0.002, False, None),
    ("e8_d4", 1.75, 1280, 2048, 300, 0.002, True, None),    # LDS-decode GEMM, ragged token tile
    ("e8_d4", 1.75, 2048, 1024, 300, 0.01, False, 128),     # S_group: two-pass from 256 tokens
    ("e8_d4", 1.75, 256, 4096, 130, 0.05, True, 64),        # dense critical blocks, S_group GEMM
    ("e8_lattice", 1.6, 3072, 768, 40, 0.002, True, None),    # E8 GEMM
    ("e8_lattice", 1.6, 3072, 768, 300, 0.002, True, None),   # E8 two-pass (from 64 tokens)
    ("e8_lattice", 1.6, 1024, 512, 260, 0.002, False, 64),    # E8 two-pass with S_group
    ("e8_d4", 1.75, 1024, 1024, 2048, 0.002, True, 128),      # E8-D4 two-pass with S_group and bias
])
def test_module_prefill(kind, r, out, inp, T, p, bias, qb):
    print(f"module prefill {kind} {out}x{inp} T={T} p={p} bias={bias} qb={qb}", flush=True)
    qd = make_layer(out, inp, seed=out + T, percmask=p, bias=bias, qb_size=qb)
    mod = EPTQLinear.from_quantized_data(qd, _quantizer(kind, r), kind).cuda()
    _check(mod, [qd], kind, r, T, seed=T + 5)


@pytest.mark.parametrize("T", [96, 320])
def test_multi_layer_module_prefill_gqa(T):
    print(f"module prefill q|k|v 1280+256+256 x 1024, T={T}, bias on k only", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(o, 1024, seed=400 + k, percmask=0.002, bias=(k == 1))
           for k, o in enumerate((1280, 256, 256))]
    mod = EPTQMultiLinear([EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds])
    _check(mod, qds, "e8_d4", 1.75, T, seed=11)


def test_module_prefill_bf16_and_row_consistency():
    print("module prefill: bf16 input, and a token's row does not depend on the batch", flush=True)
    qd = make_layer(1280, 2048, seed=9, percmask=0.002)
    mod = EPTQLinear.from_quantized_data(qd, E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    y16 = _check(mod, [qd], "e8_d4", 1.75, 260, seed=3)
    ybf = _check(mod, [qd], "e8_d4", 1.75, 260, seed=3, dtype=torch.bfloat16)
    assert rel_l2(ybf.float().cpu().numpy(), y16.float().cpu().numpy()) < 2 * TOL
    x = make_x(260, 2048, seed=3).cuda()
    with torch.no_grad():
        y_small = mod(x[:8])           # decode kernel
    torch.cuda.synchronize()
    assert rel_l2(y_small.float().cpu().numpy(), y16[:8].float().cpu().numpy()) < 2e-3


@pytest.mark.parametrize("out,inp,T,dtype", [
    (1024, 2048, 17, torch.float16),      # first row past the decode kernels
    (1024, 2048, 129, torch.float16),     # first row past the 16-row slices
    (1280, 2048, 257, torch.float16),     # a 256-token tile plus one row
    (1024, 2048, 100, torch.bfloat16),    # bf16 at mid counts (no matrix-core slices)
    (1024, 2048, 2048, torch.bfloat16),   # bf16 two-pass (rows to fp16 with a power-of-two scale)
    (1024, 2080, 200, torch.float16),     # in_features an odd multiple of 32
    (512, 1000, 150, torch.float16),      # in_features not a multiple of 32
    (1024, 2048, 0, torch.float16),       # empty batch
])
def test_module_prefill_edges(out, inp, T, dtype):
    print(f"module prefill edge {out}x{inp} T={T} {dtype}", flush=True)
    qd = make_layer(out, inp, seed=out + inp + T, percmask=0.002, bias=True)
    mod = EPTQLinear.from_quantized_data(qd, E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    if T == 0:
        with torch.no_grad():
            y = mod(torch.empty((0, inp), dtype=dtype, device="cuda"))
        assert y.shape == (0, out) and y.dtype == dtype
        return
    _check(mod, [qd], "e8_d4", 1.75, T, seed=T + 1, dtype=dtype)


@pytest.mark.parametrize("T", [2048, 2100])
def test_module_prefill_two_pass(T):
    print(f"module prefill two-pass q|k|v 1280+256+256 x 1024, T={T}, bias on k only", flush=True)
    from eptq_amd.kernels import TWO_PASS_MIN_TOKENS, _lib
    assert T >= TWO_PASS_MIN_TOKENS
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(o, 1024, seed=500 + k, percmask=0.002, bias=(k == 1))
           for k, o in enumerate((1280, 256, 256))]
    lins = [EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds]
    y = _check(EPTQMultiLinear(lins), qds, "e8_d4", 1.75, T, seed=13)
    # The fused prefill kernel on the same layers (one C-ABI launch each).
    x = make_x(T, 1024, seed=13).cuda()
    outs = []
    for lin in lins:
        yl = torch.empty((T, lin.out_features), dtype=torch.float16, device="cuda")
        _lib.forward_into("e8_d4", lin.Q, lin._codebook, lin.g, lin.h, x, lin.O_vals, lin.O_col,
                          lin.O_row_ptr, lin.bias, None, yl, torch.cuda.current_stream().cuda_stream)
        outs.append(yl)
    fused = torch.cat(outs, dim=1)
    torch.cuda.synchronize()
    e = rel_l2(y.float().cpu().numpy(), fused.float().cpu().numpy())
    print(f"  rel_l2 vs the fused kernel {e:.2e}", flush=True)
    assert e <= 3e-3
