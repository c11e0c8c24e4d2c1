"""GPU parity of the module forward's prefill form (``dequant_linear``).

From ``PREFILL_DEQUANT_MIN_TOKENS`` fp16 rows on, ``EPTQLinear`` and
``EPTQMultiLinear`` compute y = x·Wᵀ + bias with W written by the library's
bit-exact dequantization kernel into one stacked fp16 scratch and the
contraction on the library fp16 GEMM.  Checks:

* the result equals torch's own ``F.linear`` over the oracle's
  ``dequantize_layer`` W (stacked in layer order, biases concatenated) bit for
  bit — so every layer's W landed in its rows exactly;
* within 1e-2 relative L2 of the fp32 reconstruct + matmul oracle;
* multi-layer stacking (GQA q|k|v with a bias on one layer only), S_group,
  E8 layers, dense critical blocks;
* below the threshold, and for bf16 input, the fused kernels run instead
  (same values within the fused kernels' own tolerance).
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

import eptq_amd.kernels.linear as KL
from eptq_amd.kernels import PREFILL_DEQUANT_MIN_TOKENS
from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import linear_ref, rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _quantizer(kind, r):
    return E8D4Quantizer(radius=r) if kind == "e8_d4" else E8LatticeQuantizer(radius=r)


def _oracle_W(qd, kind, r):
    n = layer_np(qd)
    return dequantize_layer(n["Q"], n["g"], n["h"], n["O"], table(kind, r), kind, n["S_group"])


def _check(mod, qds, kind, r, T, seed):
    x = make_x(T, qds[0].Q.shape[1], seed=seed)
    with torch.no_grad():
        y = mod(x.cuda())
    torch.cuda.synchronize()
    Ws = [_oracle_W(qd, kind, r) for qd in qds]
    W = torch.from_numpy(np.concatenate(Ws, axis=0)).cuda()
    biases = [qd.bias if qd.bias is not None else torch.zeros(8 * qd.Q.shape[0], dtype=torch.float16)
              for qd in qds]
    bias = torch.cat(biases).cuda() if any(qd.bias is not None for qd in qds) else None
    want = F.linear(x.cuda(), W, bias)
    assert y.dtype == torch.float16 and y.shape == want.shape
    assert torch.equal(y, want), f"{int((y != want).sum())} of {y.numel()} differ"
    ref = np.concatenate([linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], n["O"], table(kind, r), kind,
                                     n["bias"], n["S_group"]) for n in map(layer_np, qds)], axis=1)
    e = rel_l2(y.float().cpu().numpy(), ref)
    print(f"  rel_l2 vs fp32 oracle {e:.2e}")
    assert e <= TOL


@pytest.mark.parametrize("kind,r,out,inp,T,p,bias,qb", [
    ("e8_d4", 1.75, 1024, 2048, PREFILL_DEQUANT_MIN_TOKENS, 0.002, True, None),
    ("e8_d4", 1.75, 2048, 1024, 300, 0.01, False, 128),
    ("e8_d4", 1.75, 256, 4096, 130, 0.05, True, 64),    # dense critical blocks
    ("e8_lattice", 1.6, 3072, 768, 200, 0.002, True, None),
])
def test_linear_prefill_form(kind, r, out, inp, T, p, bias, qb):
    print(f"prefill form {kind} {out}x{inp} T={T} p={p} bias={bias} qb={qb}", flush=True)
    qd = make_layer(out, inp, seed=out + T, percmask=p, bias=bias, qb_size=qb)
    mod = EPTQLinear.from_quantized_data(qd, _quantizer(kind, r), kind).cuda()
    _check(mod, [qd], kind, r, T, seed=T + 5)


def test_multi_layer_prefill_form_gqa():
    print("prefill form q|k|v 1024+256+256 x 1024, T=96, bias on k only", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(o, 1024, seed=400 + k, percmask=0.002, bias=(k == 1))
           for k, o in enumerate((1024, 256, 256))]
    mod = EPTQMultiLinear([EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds])
    _check(mod, qds, "e8_d4", 1.75, 96, seed=11)


def test_below_threshold_and_bf16_take_the_fused_kernels():
    print("prefill form: threshold and bf16 dispatch", flush=True)
    qd = make_layer(1024, 1024, seed=9, percmask=0.002)
    mod = EPTQLinear.from_quantized_data(qd, E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    T = PREFILL_DEQUANT_MIN_TOKENS
    x = make_x(T, 1024, seed=3).cuda()
    calls = []
    orig = KL.dequant_linear

    def spy(*a, **k):
        calls.append(a[0])
        return orig(*a, **k)

    KL.dequant_linear = spy
    try:
        with torch.no_grad():
            y_dq = mod(x)
            y_small = mod(x[:T - 1])
            y_bf = mod(x.bfloat16())
    finally:
        KL.dequant_linear = orig
    torch.cuda.synchronize()
    assert calls == ["e8_d4"]                  # only the fp16 call at the threshold
    assert y_bf.dtype == torch.bfloat16
    assert rel_l2(y_small.float().cpu().numpy(), y_dq[:T - 1].float().cpu().numpy()) < 2e-3
    assert rel_l2(y_bf.float().cpu().numpy(), y_dq.float().cpu().numpy()) < TOL
