"""GPU parity of the SwiGLU decode launch (``eptq_llama_norm_swiglu``): the
gate and up rows of the same block rows in one workgroup, out = silu(gate(t))
⊙ up(t) for t the fused RMSNorm of resid + delta.

Against the two-launch path (``eptq_llama_norm_linear`` over gate|up, then
``eptq_llama_silu_mul``), which rounds the same way, the result is
bit-identical where that path also runs whole-row waves (the Llama-2-7B FFN
shape, B = 1 and 2), and so is the residual written to resid_out.  On small
shapes (where the separate launch splits rows over waves), with bias,
S_group and dense critical blocks, it is within 1e-2 relative L2 of a
float32 oracle: RMSNorm, reconstruct + matmul per layer, SiLU product."""

import numpy as np
import pytest
import torch

from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from eptq_amd.llama import norm_linear, norm_swiglu, silu_mul
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

EPS = 1e-5


def _pair(F, N, seed, qb=None, bias=False, p=0.002):
    q = E8D4Quantizer(radius=1.75)
    qds = [make_layer(F, N, seed=seed + k, percmask=p, bias=bias, qb_size=qb) for k in range(2)]
    return qds, EPTQMultiLinear([EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda() for qd in qds])


def _inputs(B, N, seed):
    gen = torch.Generator().manual_seed(seed)
    resid = make_x(B, N, seed=seed)
    delta = (0.5 * make_x(B, N, seed=seed + 1).float()).half()
    w = (1.0 + 0.05 * torch.randn(N, generator=gen)).half()
    return resid, delta, w


@pytest.mark.parametrize("B", [1, 2])
def test_swiglu_bit_identical_to_two_launches(B):
    print(f"swiglu launch vs norm_linear + silu_mul, 11008x4096, B={B}", flush=True)
    _, mod = _pair(11008, 4096, seed=40)
    resid, delta, w = (t.cuda() for t in _inputs(B, 4096, seed=B))
    r1, r2 = torch.empty_like(resid), torch.empty_like(resid)
    a = norm_swiglu(mod, resid, delta, w, EPS, r1)
    b = silu_mul(norm_linear(mod, resid, delta, w, EPS, r2))
    torch.cuda.synchronize()
    assert a.shape == (B, 11008)
    d = (a.float() - b.float()).abs()
    assert torch.equal(a, b), f"{int((a != b).sum())} of {a.numel()} differ, max |diff| {float(d.max()):.3e}"
    assert torch.equal(r1, r2)
    assert torch.equal(r1, (resid.float() + delta.float()).half())


@pytest.mark.parametrize("F,N,B,qb,bias,p", [
    (1024, 512, 1, None, True, 0.002),
    (1024, 512, 2, None, False, 0.02),     # many critical blocks per row
    (768, 2048, 2, 128, True, 0.002),      # S_group
    (520, 776, 1, None, False, 0.002),     # last row group half full; 776 = 12 blocks + 8 columns
])
def test_swiglu_matches_fp32_oracle(F, N, B, qb, bias, p):
    print(f"swiglu launch vs oracle F={F} N={N} B={B} qb={qb} bias={bias} p={p}", flush=True)
    qds, mod = _pair(F, N, seed=F + N + B, qb=qb, bias=bias, p=p)
    resid, delta, w = _inputs(B, N, seed=7 * B)
    r = torch.empty_like(resid).cuda()
    got = norm_swiglu(mod, resid.cuda(), delta.cuda(), w.cuda(), EPS, r).float().cpu().numpy()
    # Oracle: r = fp16(resid + delta), t = fp16(r · rsqrt(mean(r²) + eps) · w).
    rr = (resid.float() + delta.float()).half()
    assert torch.equal(r.cpu(), rr)
    ms = (rr.float() ** 2).mean(-1, keepdim=True)
    t = (rr.float() * torch.rsqrt(ms + EPS) * w.float()).half().float().numpy()
    tab = table("e8_d4", 1.75)
    ys = []
    for qd in qds:
        n = layer_np(qd)
        ys.append(linear_ref(t, n["Q"], n["g"], n["h"], n["O"], tab, "e8_d4", n["bias"], n["S_group"]))
    gate, upv = ys
    want = gate / (1.0 + np.exp(-gate)) * upv
    assert np.isfinite(got).all()
    e = rel_l2(got, want)
    print(f"  rel_l2 {e:.2e}")
    assert e <= 1e-2


def test_decode_step_uses_swiglu_launch_and_matches_separate_silu():
    """The fused decode step (B <= 2 takes the SwiGLU launch) against the same
    step with the SiLU product as a launch of its own: same logits."""
    from eptq_amd.llama import LlamaConfig, build_synthetic
    print("synthetic llama: swiglu launch in the decode step", flush=True)
    cfg = LlamaConfig(hidden=512, ffn=1024, layers=2, heads=4, kv_heads=4, vocab=256)
    model = build_synthetic(cfg, device="cuda", seed=13)
    for B in (1, 2):
        model.alloc_cache(B, 32, "cuda")
        tok = torch.randint(0, cfg.vocab, (B, 1), device="cuda", generator=torch.Generator("cuda").manual_seed(B))
        pos = torch.tensor([0], device="cuda")
        with torch.no_grad():
            kc0 = [k.clone() for k in model.kc]
            vc0 = [v.clone() for v in model.vc]
            got = model.decode_tokens(tok, pos).float()
            for i in range(cfg.layers):
                model.kc[i].copy_(kc0[i])
                model.vc[i].copy_(vc0[i])
            def separate(mod, x, delta, w):   # fused-norm gate|up launch, then the SiLU kernel
                gu, r = model._norm_into(mod, x, delta, w)
                return silu_mul(gu), r

            model._norm_swiglu = separate
            try:
                ref = model.decode_tokens(tok, pos).float()
            finally:
                del model._norm_swiglu
        assert rel_l2(got.cpu().numpy(), ref.cpu().numpy()) < 2e-3, B
