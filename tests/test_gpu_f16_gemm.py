"""GPU parity of the two-pass prefill's GEMM (``eptq_f16_gemm``: y = x·Wᵀ +
bias over fp16 W streamed by LDS DMA into the fused kernel's tiles).

* Against torch's fp32 matmul of the same fp16 operands: within 2e-3
  relative L2 (fp32 accumulation, fp16 output), for each tile the launcher
  picks on a 256-CU MI355X (160 x 256, 256 x 256, 128 x 256 and 64 x 256
  features x tokens), ragged last feature tiles (160 and 128), token counts
  that leave a ragged last token tile, with and without bias.
* The two passes together (``eptq_e8d4_dequant`` then the GEMM) within 1e-2
  of the oracle's reconstruct + matmul on a synthetic E8-D4 layer.
* EPTQ_EUNSUPPORTED for F or N not a multiple of 64.
"""

import numpy as np
import pytest
import torch

from eptq_amd.kernels import _lib, dequant, f16_gemm
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import csr_dev, layer_np, table

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("F,N,T,bias", [
    (5120, 512, 2000, False),    # 160 x 256 tiles
    (13824, 256, 2000, True),    # 160 x 256, ragged last feature tile (64 of 160 rows)
    (13824, 128, 2100, False),   # 256 x 256 (the two-stage kernel), ragged last token tile
    (4096, 256, 1900, True),     # 128 x 256
    (5184, 256, 2048, True),     # 128 x 256, ragged last feature tile (64 of 128 rows)
    (1024, 2048, 257, True),     # 64 x 256 (few tiles: the narrowest)
    (64, 256, 17, False),        # 64 x 256, one token tile
])
def test_f16_gemm_vs_torch(F, N, T, bias):
    print(f"eptq_f16_gemm F={F} N={N} T={T} bias={bias}", flush=True)
    gen = torch.Generator("cuda").manual_seed(F + N + T)
    W = (torch.randn((F, N), generator=gen, device="cuda") * 0.05).half()
    x = torch.randn((T, N), generator=gen, device="cuda").half()
    b = torch.randn(F, generator=gen, device="cuda").half() if bias else None
    y = f16_gemm(W, x, b)
    want = x.float() @ W.float().t() + (b.float() if bias else 0.0)
    e = rel_l2(y.float().cpu().numpy(), want.cpu().numpy())
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert torch.isfinite(y).all() and e <= 2e-3


def test_two_pass_prefill_vs_oracle():
    print("two-pass prefill 2048x1024 at 600 tokens vs the oracle", flush=True)
    qd = make_layer(2048, 1024, seed=77, percmask=0.002)
    x = make_x(600, 1024, seed=5)
    codes32 = torch.from_numpy(table("e8_d4", 1.75)).float().cuda()
    ocol, orp = csr_dev(qd.Q)
    W = dequant("e8_d4", qd.Q.cuda(), codes32, qd.g.cuda(), qd.h.cuda(), qd.O.cuda(), ocol, orp)
    y = f16_gemm(W, x.cuda()).float().cpu().numpy()
    n = layer_np(qd)
    want = linear_ref(x.float().numpy(), n["Q"], n["g"], n["h"], n["O"], table("e8_d4", 1.75), "e8_d4",
                      n["bias"], n["S_group"])
    e = rel_l2(y, want)
    print(f"  rel_l2 {e:.2e}", flush=True)
    assert np.isfinite(y).all() and e <= 1e-2


def test_bf16_rows_to_f16_exact():
    """Rows of very different magnitudes: x16 · row_scale gives back x exactly,
    row_scale is a power of two, and each row's largest |x16| is in
    [2^14, 2^15)."""
    T, N = 9, 4096
    gen = torch.Generator("cuda").manual_seed(3)
    base = torch.randn((T, N), generator=gen, device="cuda")
    mags = torch.tensor([2.0 ** k for k in (-60, -30, -10, -1, 0, 3, 12, 40, 90)], device="cuda")
    x = (base * mags[:, None]).bfloat16()
    x[4, 17] = 0.0
    x16 = torch.empty((T, N), dtype=torch.float16, device="cuda")
    rs = torch.empty(T, dtype=torch.float32, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.load().eptq_bf16_rows_to_f16(x.data_ptr(), N, T, x16.data_ptr(), rs.data_ptr(), stream),
               "eptq_bf16_rows_to_f16")
    torch.cuda.synchronize()
    back = x16.double() * rs.double()[:, None]
    xd = x.double()
    # Elements above 2^-28 of their row's maximum come back exactly.
    keep = xd.abs() >= xd.abs().amax(dim=1, keepdim=True) * 2.0 ** -28
    assert torch.equal(back[keep], xd[keep])
    assert torch.all(torch.log2(rs.double()) == torch.round(torch.log2(rs.double())))
    top = x16.double().abs().amax(dim=1)
    assert torch.all(top >= 2.0 ** 14) and torch.all(top < 2.0 ** 15)


@pytest.mark.parametrize("F,N,T", [(5120, 512, 2000), (1024, 2048, 300)])
def test_f16_gemm_rows_bf16(F, N, T):
    """bf16 x through the row conversion, then the row-scaled GEMM with bf16
    output, against torch's fp32 matmul: within 5e-3 relative L2 (bf16
    output rounding), rows of different magnitudes."""
    print(f"eptq_f16_gemm_rows bf16 F={F} N={N} T={T}", flush=True)
    gen = torch.Generator("cuda").manual_seed(F + T)
    W = (torch.randn((F, N), generator=gen, device="cuda") * 0.05).half()
    scale = 2.0 ** torch.randint(-20, 20, (T, 1), generator=gen, device="cuda").float()
    x = (torch.randn((T, N), generator=gen, device="cuda") * scale).bfloat16()
    b = torch.randn(F, generator=gen, device="cuda").half()
    lib, stream = _lib.load(), torch.cuda.current_stream().cuda_stream
    x16 = torch.empty((T, N), dtype=torch.float16, device="cuda")
    rs = torch.empty(T, dtype=torch.float32, device="cuda")
    _lib.check(lib.eptq_bf16_rows_to_f16(x.data_ptr(), N, T, x16.data_ptr(), rs.data_ptr(), stream),
               "eptq_bf16_rows_to_f16")
    y = torch.empty((T, F), dtype=torch.bfloat16, device="cuda")
    _lib.check(lib.eptq_f16_gemm_rows(W.data_ptr(), x16.data_ptr(), b.data_ptr(), F, N, T, rs.data_ptr(),
                                      y.data_ptr(), _lib.EPTQ_BF16, F, stream), "eptq_f16_gemm_rows")
    want = x.float() @ W.float().t() + b.float()
    # Per row (magnitudes differ by 2^40 across rows).
    err = ((y.float() - want).norm(dim=1) / want.norm(dim=1)).max().item()
    print(f"  max row rel_l2 {err:.2e}", flush=True)
    assert torch.isfinite(y.float()).all() and err <= 5e-3


def test_f16_gemm_unsupported():
    W = torch.zeros((100, 256), dtype=torch.float16, device="cuda")
    x = torch.zeros((8, 256), dtype=torch.float16, device="cuda")
    with pytest.raises(_lib.EptqError) as err:
        f16_gemm(W, x)
    assert err.value.code == _lib.EPTQ_EUNSUPPORTED
