"""GPU parity of the fused decode attention (rotary on q and k, k/v written
to the cache at pos, softmax(q·Kᵀ/√D)·V over positions 0..pos) against a
float32 PyTorch reference of the same steps on the CPU, for one workgroup
per head and for positions split over workgroups.  The cases cross the
kernel's 256-row chunks (255/256, 511/512), a cache shorter than one chunk,
GQA head groups, positions outside the cache, and cache rows past pos that
hold NaN (they must not reach the output)."""

import math

import numpy as np
import pytest
import torch

from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu

D = 128


def _tables(L, theta=10000.0):
    inv = 1.0 / (theta ** (torch.arange(0, D, 2).float() / D))
    f = torch.outer(torch.arange(L).float(), inv)
    emb = torch.cat((f, f), dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


def _ref(qkv, p, cos, sin, kc, vc, H, Hk):
    """out (B, H·D) fp32 and the fp16 k, v rows written at p."""
    B = qkv.shape[0]
    x = qkv.float().view(B, H + 2 * Hk, D)
    q, k, v = x[:, :H], x[:, H:H + Hk], x[:, H + Hk:]
    c, s = cos[p], sin[p]

    def rot(t):
        return torch.cat((-t[..., D // 2:], t[..., :D // 2]), -1)

    qr = (q * c + rot(q) * s).half().float()
    kr = (k * c + rot(k) * s).half()
    K = kc.float().clone()
    V = vc.float().clone()
    K[:, :, p] = kr.float()
    V[:, :, p] = v
    g = H // Hk
    Kh = K[:, :, :p + 1].repeat_interleave(g, dim=1)
    Vh = V[:, :, :p + 1].repeat_interleave(g, dim=1)
    sc = (qr.unsqueeze(2) * Kh).sum(-1) / math.sqrt(D)
    pr = torch.softmax(sc, dim=-1)
    o = (pr.unsqueeze(-1) * Vh).sum(2)
    return o.reshape(B, H * D), kr, v.half()


def _run(lib, qkv, p, cos, sin, kc, vc, H, Hk, L, work):
    B = qkv.shape[0]
    pos = torch.tensor([p], device="cuda")
    out = torch.full((B, H * D), 7.0, dtype=torch.float16, device="cuda")
    rc = lib.eptq_llama_rope_attn(qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), kc.data_ptr(),
                                  vc.data_ptr(), out.data_ptr(), B, H, Hk, D, L,
                                  None if work is None else work.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("B,H,Hk,L,positions", [
    (1, 32, 32, 1024, (0, 5, 255, 256, 300, 511, 512, 700, 1023)),
    (2, 8, 2, 384, (0, 100, 255, 256, 383)),
    (3, 4, 4, 40, (0, 39)),
])
@pytest.mark.parametrize("split", [False, True])
def test_attention_matches_fp32_reference(B, H, Hk, L, positions, split):
    from eptq_amd.kernels import _lib
    lib = _lib.load()
    print(f"decode attention B={B} H={H} Hk={Hk} L={L} split={split}", flush=True)
    gen = torch.Generator().manual_seed(B * 100 + H + L)
    cos, sin = _tables(L)
    work = None
    if split:
        work = torch.zeros(lib.eptq_llama_attn_work_bytes(B, H), dtype=torch.uint8, device="cuda")
    for p in positions:
        qkv = torch.randn((B, (H + 2 * Hk) * D), generator=gen).half()
        kc = (torch.randn((B, Hk, L, D), generator=gen) * 0.5).half()
        vc = torch.randn((B, Hk, L, D), generator=gen).half()
        kc[:, :, p + 1:] = float("nan")   # never read as data
        vc[:, :, p + 1:] = float("nan")
        want, kr, vr = _ref(qkv, p, cos, sin, kc, vc, H, Hk)
        kd, vd = kc.cuda(), vc.cuda()
        got = _run(lib, qkv.cuda(), p, cos.cuda(), sin.cuda(), kd, vd, H, Hk, L, work).float().cpu()
        assert torch.isfinite(got).all(), p
        e = rel_l2(got.numpy(), want.numpy())
        print(f"  pos {p}: rel_l2 {e:.2e}")
        assert e < 2e-3, p
        kc2, vc2 = kd.cpu(), vd.cpu()
        assert torch.equal(kc2[:, :, p], kr) and torch.equal(vc2[:, :, p], vr), p
        others = [i for i in range(L) if i != p]
        assert torch.equal(kc2[:, :, others].view(torch.int16), kc[:, :, others].view(torch.int16)), p
        assert torch.equal(vc2[:, :, others].view(torch.int16), vc[:, :, others].view(torch.int16)), p
    if split:
        cnt = work[-4 * B * H:].view(torch.int32)
        assert int(cnt.abs().sum()) == 0


@pytest.mark.parametrize("split", [False, True])
def test_attention_position_outside_cache(split):
    """pos < 0 or pos >= L: zero output and the caches untouched."""
    from eptq_amd.kernels import _lib
    lib = _lib.load()
    print(f"decode attention: pos outside the cache, split={split}", flush=True)
    B, H, Hk, L = 2, 8, 4, 64
    gen = torch.Generator().manual_seed(3)
    cos, sin = _tables(L)
    qkv = torch.randn((B, (H + 2 * Hk) * D), generator=gen).half().cuda()
    kc = torch.randn((B, Hk, L, D), generator=gen).half().cuda()
    vc = torch.randn((B, Hk, L, D), generator=gen).half().cuda()
    k0, v0 = kc.clone(), vc.clone()
    work = None
    if split:
        work = torch.zeros(lib.eptq_llama_attn_work_bytes(B, H), dtype=torch.uint8, device="cuda")
    for p in (-1, L, L + 100):
        out = _run(lib, qkv, p, cos.cuda(), sin.cuda(), kc, vc, H, Hk, L, work)
        assert int(out.view(torch.int16).abs().sum()) == 0, p
        assert torch.equal(kc, k0) and torch.equal(vc, v0), p
    if split:
        assert int(work[-4 * B * H:].view(torch.int32).abs().sum()) == 0
