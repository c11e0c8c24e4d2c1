"""GPU parity of the fused attention + o projection launch
(``eptq_llama_attn_o``, batch 1): the first H workgroups run the rotary,
cache write and attention of one head each (the unsplit path of
``eptq_llama_rope_attn``) and publish it device-coherently, while every
workgroup streams the o layer's indices; the layer reads the published
attention once all heads are counted.

Against the two-launch path (``eptq_llama_rope_attn`` then the o Linear),
which runs the same arithmetic with the same work split, the attention
output, the cache rows and y are bit-identical, over several positions (one
and two 256-row chunks), with GQA, and on repeated calls (the counters reset
themselves); the decode step of the synthetic Llama gives the same logits
with and without the fused launch."""

import ctypes

import pytest
import torch

from eptq_amd.kernels import _lib
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.llama import LlamaConfig, build_synthetic
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer

pytestmark = pytest.mark.gpu


def _layer_array(mod):
    arr = (_lib.EptqLayer * 1)()
    arr[0] = _lib.EptqLayer(mod.Q.data_ptr(), mod.g.data_ptr(), mod.h.data_ptr(),
                            mod.O_vals.data_ptr() if mod.O_vals.numel() else None,
                            mod.O_col.data_ptr() if mod.O_col.numel() else None,
                            mod.O_row_ptr.data_ptr(), None, None, 0, mod.Q.shape[0], 0)
    return arr


@pytest.mark.parametrize("H,Hk,positions", [(32, 32, (0, 5, 255, 256, 300)), (8, 2, (17, 511))])
def test_attn_o_bit_identical_to_two_launches(H, Hk, positions):
    print(f"attn+o fused vs two launches H={H} Hk={Hk} positions={positions}", flush=True)
    D, L = 128, 512
    lib = _lib.load()
    gen = torch.Generator(device="cuda").manual_seed(H + Hk)
    mod = EPTQLinear.from_quantized_data(make_layer(H * D, H * D, seed=H, percmask=0.002),
                                         E8D4Quantizer(radius=1.75), "e8_d4").cuda()
    arr = _layer_array(mod)
    inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
    f = torch.outer(torch.arange(L, device="cuda").float(), inv)
    emb = torch.cat((f, f), dim=-1)
    cos, sin = emb.cos().contiguous(), emb.sin().contiguous()
    kc0 = (0.5 * torch.randn((1, Hk, L, D), device="cuda", generator=gen)).half()
    vc0 = torch.randn((1, Hk, L, D), device="cuda", generator=gen).half()
    work = torch.zeros(lib.eptq_llama_attn_o_work_bytes(), dtype=torch.uint8, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    for p in positions:
        qkv = torch.randn((1, (H + 2 * Hk) * D), device="cuda", generator=gen).half()
        pos = torch.tensor([p], dtype=torch.int64, device="cuda")
        kc1, vc1, kc2, vc2 = kc0.clone(), vc0.clone(), kc0.clone(), vc0.clone()
        att1 = torch.empty((1, H * D), dtype=torch.float16, device="cuda")
        att2 = torch.empty_like(att1)
        y1 = torch.empty((1, H * D), dtype=torch.float16, device="cuda")
        y2 = torch.empty_like(y1)
        _lib.check(lib.eptq_llama_rope_attn(qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                            kc1.data_ptr(), vc1.data_ptr(), att1.data_ptr(), 1, H, Hk, D, L, None,
                                            st), "rope_attn")
        _lib.check(lib.eptq_e8d4_forward_multi(1, arr, mod._codebook.data_ptr(), _lib.EPTQ_F16, att1.data_ptr(),
                                               _lib.EPTQ_F16, H * D, 1, y1.data_ptr(), H * D, None, 0, st),
                   "forward_multi")
        for rep in range(2):   # the counters must reset themselves
            _lib.check(lib.eptq_llama_attn_o(qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                             kc2.data_ptr(), vc2.data_ptr(), att2.data_ptr(), H, Hk, D, L, arr,
                                             mod._codebook.data_ptr(), y2.data_ptr(), work.data_ptr(), st),
                       "attn_o")
            torch.cuda.synchronize()
            w = work.view(torch.int32).cpu()
            assert int(w.abs().sum()) == 0, w
            assert torch.equal(att1, att2), (p, rep)
            assert torch.equal(kc1, kc2) and torch.equal(vc1, vc2), (p, rep)
            assert torch.equal(y1, y2), (p, rep, int((y1 != y2).sum()))


def test_decode_step_with_and_without_fused_attn_o():
    print("synthetic llama: fused attention + o in the decode step", flush=True)
    cfg = LlamaConfig(hidden=1024, ffn=2048, layers=2, heads=8, kv_heads=8, vocab=512)
    model = build_synthetic(cfg, device="cuda", seed=21)
    model.alloc_cache(1, 64, "cuda")
    assert model.attn_o_work is not None
    calls = []
    orig = model._attn_o

    def spy(*a):
        y = orig(*a)
        calls.append(y is not None)
        return y

    model._attn_o = spy
    tok = torch.tensor([[7]], device="cuda")
    pos = torch.tensor([3], device="cuda")
    kc0 = [k.clone() for k in model.kc]
    vc0 = [v.clone() for v in model.vc]
    outs = []
    for fuse in (True, False):
        model.fuse_attn_o = fuse
        for i in range(cfg.layers):
            model.kc[i].copy_(kc0[i])
            model.vc[i].copy_(vc0[i])
        with torch.no_grad():
            outs.append(model.decode_tokens(tok, pos).float())
    del model._attn_o
    assert calls[:cfg.layers] == [True] * cfg.layers and not any(calls[cfg.layers:])
    assert torch.equal(outs[0], outs[1])
