"""GPU: the drop-in model path end to end.

* ``load_quantized_model`` on a synthetic tiny Llama checkpoint (reference
  directory layout) produces the logits of the same model with dense fp32
  weights reconstructed by the oracle (``dequantize_layer``), within the
  fp16-activation tolerance.
* The synthetic Llama decoder of ``eptq_amd.llama``: a graph-captured decode
  step reproduces the eager step, token for token.
"""

from __future__ import annotations

import dataclasses

import numpy as np
import pytest
import torch

from eptq_amd.kernels.linear import EPTQLinear
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny_dir(tmp_path_factory):
    from transformers import LlamaConfig
    from eptq_amd.synthetic import write_quantized_model
    from test_host import _tiny_tokenizer
    d = tmp_path_factory.mktemp("qmodel_gpu")
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    write_quantized_model(d, cfg, percmask=0.02, seed=5, tokenizer=_tiny_tokenizer())
    return d


def test_load_quantized_model_logits_match_dense_reconstruction(tiny_dir):
    from transformers import AutoConfig, AutoModelForCausalLM
    from eptq_amd.kernels.patch import load_quantized_model
    print("tiny quantized llama: logits vs dense reconstruction", flush=True)
    model, _ = load_quantized_model(str(tiny_dir), device="cuda")
    ids = torch.tensor([[1, 5, 9, 33, 2, 7, 64, 100]], device="cuda")
    with torch.no_grad():
        got = model(ids).logits.float().cpu().numpy()

    cfg = AutoConfig.from_pretrained(tiny_dir)
    ref = AutoModelForCausalLM.from_config(cfg).float().eval()
    sd = {}
    for name, mod in model.named_modules():
        if isinstance(mod, EPTQLinear):
            tab = mod._table_f32.cpu().numpy()
            W = dequantize_layer(mod.Q.cpu().numpy(), mod.g.cpu().numpy(), mod.h.cpu().numpy(),
                                 mod.O_vals.cpu().numpy(), tab, mod.quantizer_type)
            sd[name + ".weight"] = torch.from_numpy(W.astype(np.float32))
    for name, p in model.named_parameters():
        sd[name] = p.detach().float().cpu()
    missing, unexpected = ref.load_state_dict(sd, strict=False)
    assert not [m for m in missing if "rotary" not in m], missing
    with torch.no_grad():
        want = ref(ids.cpu()).logits.numpy()
    assert rel_l2(got, want) <= 2e-2


@pytest.fixture(scope="module")
def warped_dir(tmp_path_factory):
    from transformers import LlamaConfig
    from eptq_amd.synthetic import write_quantized_model
    from test_host import _tiny_tokenizer
    d = tmp_path_factory.mktemp("qmodel_warp")
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    write_quantized_model(d, cfg, percmask=0.02, seed=8, tokenizer=_tiny_tokenizer(), warp_alpha=1.3,
                          chosen_r=[None, 1.9, None, 1.6, 1.75])
    return d


def test_load_quantized_model_warped_chosen_r(warped_dir):
    """A warped table (warp_alpha 1.3) and layers with their own chosen_r,
    loaded through load_quantized_model on the GPU: each layer's table follows
    the reference's load order (the warp holds until the first radius switch,
    which drops it — pinned on the CPU by tests/test_loader_golden.py), the
    GPU dequantization is bit-exact with the oracle on the layer's table, and
    the logits match a dense fp32 model over the oracle's W."""
    from transformers import AutoConfig, AutoModelForCausalLM
    from eptq_amd.kernels.linear import _table_for
    from eptq_amd.kernels.patch import load_quantized_model
    from eptq_amd.reconstruct import load_quantized_layer, load_quantizer
    from eptq_amd.handlers import ModelHandler, get_model_handler_by_type
    print("warped chosen_r checkpoint: tables, dequant, logits", flush=True)
    model, _ = load_quantized_model(str(warped_dir), device="cuda")
    # The same load order replayed on the CPU with the loader pinned by the
    # golden tests; the GPU's tables come from torch on the GPU (division and
    # the warp's norm/pow), so they agree to fp32 rounding.
    qcpu = load_quantizer(warped_dir, device="cpu")
    handler = get_model_handler_by_type(ModelHandler.detect_model_type(model))
    n_warped = n_plain = 0
    for lid, layer in enumerate(handler.get_layers(model)):
        # The loader swapped the layer's Linears in named_modules order.
        for name, lin in [(n, m) for n, m in layer.named_modules() if isinstance(m, EPTQLinear)]:
            qd = load_quantized_layer(warped_dir / f"layer_{lid}", name)
            want, _ = _table_for(qcpu, "e8_d4", qd.chosen_r)
            got = lin._table_f32.cpu()
            ulps = (got.view(torch.int32).long() - want.view(torch.int32).long()).abs().max().item()
            print(f"  layer {lid} {name} chosen_r={qd.chosen_r}: table within {ulps} ulp of the CPU replay")
            assert ulps <= 4, (lid, name, ulps)
            plain = torch.equal(want, (qcpu._raw_codes / (qd.chosen_r or 1.75)).reshape(512, 4))
            n_plain += plain
            n_warped += not plain
            W = lin.dequantize().cpu().numpy()
            ref = dequantize_layer(lin.Q.cpu().numpy(), lin.g.cpu().numpy(), lin.h.cpu().numpy(),
                                   lin.O_vals.cpu().numpy(), got.numpy(), "e8_d4")
            assert np.array_equal(W.view(np.uint16), ref.view(np.uint16)), (lid, name)
    assert n_warped >= 1 and n_plain >= 1, (n_warped, n_plain)
    ids = torch.tensor([[3, 1, 4, 1, 5, 9, 2, 6]], device="cuda")
    with torch.no_grad():
        got = model(ids).logits.float().cpu().numpy()
    cfg = AutoConfig.from_pretrained(warped_dir)
    ref = AutoModelForCausalLM.from_config(cfg).float().eval()
    sd = {}
    for name, mod in model.named_modules():
        if isinstance(mod, EPTQLinear):
            W = dequantize_layer(mod.Q.cpu().numpy(), mod.g.cpu().numpy(), mod.h.cpu().numpy(),
                                 mod.O_vals.cpu().numpy(), mod._table_f32.cpu().numpy(), "e8_d4")
            sd[name + ".weight"] = torch.from_numpy(W.astype(np.float32))
    for name, p in model.named_parameters():
        sd[name] = p.detach().float().cpu()
    ref.load_state_dict(sd, strict=False)
    with torch.no_grad():
        want = ref(ids.cpu()).logits.numpy()
    assert rel_l2(got, want) <= 2e-2


def test_llama_graph_decode_matches_eager():
    from eptq_amd.llama import GraphDecoder, LlamaConfig, build_synthetic
    print("synthetic llama: graph vs eager decode", flush=True)
    cfg = LlamaConfig(hidden=512, ffn=1024, layers=2, heads=4, kv_heads=4, vocab=512)
    model = build_synthetic(cfg, device="cuda", seed=9)
    dec = GraphDecoder(model, 2, 48, device="cuda")
    prompt = torch.randint(0, cfg.vocab, (2, 16), device="cuda", generator=torch.Generator("cuda").manual_seed(1))
    dec.prefill(prompt)
    eager = []
    for _ in range(6):
        dec.step()
        eager.append(dec.tok.clone())
    dec.prefill(prompt)
    dec.capture()
    for i in range(6):
        dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.tok, eager[i]), f"token {i}"


def test_fused_decode_step_matches_pytorch_path():
    """The fused decode kernels (RMSNorm, rotary + cache + attention, SiLU,
    multi-layer q|k|v and gate|up launches) against the PyTorch path on the
    same caches: logits and the cache entries written at the position."""
    from eptq_amd.llama import LlamaConfig, build_synthetic
    print("synthetic llama: fused decode step vs pytorch path", flush=True)
    for kv in (4, 2):
        cfg = LlamaConfig(hidden=512, ffn=1024, layers=2, heads=4, kv_heads=kv, vocab=256)
        model = build_synthetic(cfg, device="cuda", seed=11)
        for B in (1, 3):
            model.alloc_cache(B, 64, "cuda")
            prompt = torch.randint(0, cfg.vocab, (B, 20), device="cuda",
                                   generator=torch.Generator("cuda").manual_seed(B))
            with torch.no_grad():
                model.forward_tokens(prompt, torch.arange(20, device="cuda"))
                kc0 = [k.clone() for k in model.kc]
                vc0 = [v.clone() for v in model.vc]
                tok = torch.randint(0, cfg.vocab, (B, 1), device="cuda")
                pos = torch.tensor([20], device="cuda")
                ref = model.forward_tokens(tok, pos)[:, -1].float()
                kref = [k[:, :, 20].clone() for k in model.kc]
                for i in range(cfg.layers):
                    model.kc[i].copy_(kc0[i])
                    model.vc[i].copy_(vc0[i])
                got = model.decode_tokens(tok, pos).float()
            assert rel_l2(got.cpu().numpy(), ref.cpu().numpy()) < 1e-2, (kv, B)
            for i in range(cfg.layers):
                assert rel_l2(model.kc[i][:, :, 20].float().cpu().numpy(), kref[i].float().cpu().numpy()) < 1e-2


def test_multi_linear_matches_separate_layers():
    from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer
    print("multi-layer launch vs separate layers", flush=True)
    q = E8D4Quantizer(radius=1.75)
    for shapes, bias, qb in ((((512, 256), (128, 256), (128, 256)), False, None),
                             (((1024, 512), (1024, 512)), True, None),
                             (((256, 128), (256, 128), (512, 128), (128, 128)), False, 64)):
        ls = [EPTQLinear.from_quantized_data(make_layer(o, i, seed=o + 7 * k, percmask=0.01, bias=bias,
                                                        qb_size=qb), q, "e8_d4").cuda()
              for k, (o, i) in enumerate(shapes)]
        multi = EPTQMultiLinear(ls)
        for B in (1, 2, 5, 8, 12, 40):
            x = torch.randn(B, shapes[0][1], device="cuda").half()
            want = torch.cat([l(x) for l in ls], dim=1).float().cpu().numpy()
            got = multi(x).float().cpu().numpy()
            assert rel_l2(got, want) < 2e-3, (shapes, B)


def test_fused_norm_matches_separate_launches():
    """The decode step with the residual add + RMSNorm inside the q|k|v and
    gate|up launches against the same step with the norms as launches of
    their own (the fused entry points must really run: no fallback; gate|up
    takes the SwiGLU launch for B <= 2; for 3 <= B <= 8 every Linear runs on
    the matrix-core kernel, the norms folded into q|k|v and gate|up, the
    SwiGLU product into gate|up (eptq_llama_linear_swiglu) and the residual
    adds into o and down)."""
    from eptq_amd.llama import LlamaConfig, build_synthetic
    import eptq_amd.llama as LL
    print("synthetic llama: fused norm vs separate launches", flush=True)
    calls, swiglu, mc = [], [], []
    real, real_sw, real_llin = LL.norm_linear, LL.norm_swiglu, LL.QuantLlama._llin
    real_llsw = LL.QuantLlama._llin_swiglu
    LL.norm_linear = lambda *a, **k: (calls.append(1), real(*a, **k))[1]
    LL.norm_swiglu = lambda *a, **k: (swiglu.append(1), real_sw(*a, **k))[1]
    LL.QuantLlama._llin = lambda self, mod, x, norm_w=None, resid=None: (
        mc.append("norm" if norm_w is not None else "resid" if resid is not None else "plain"),
        real_llin(self, mod, x, norm_w=norm_w, resid=resid))[1]
    LL.QuantLlama._llin_swiglu = lambda self, mod, x, norm_w: (mc.append("swiglu"), real_llsw(self, mod, x, norm_w))[1]
    for kv, B in ((4, 1), (2, 3), (4, 8)):
        cfg = LlamaConfig(hidden=512, ffn=1024, layers=2, heads=4, kv_heads=kv, vocab=256)
        model = build_synthetic(cfg, device="cuda", seed=13 + B)
        model.alloc_cache(B, 64, "cuda")
        prompt = torch.randint(0, cfg.vocab, (B, 12), device="cuda", generator=torch.Generator("cuda").manual_seed(B))
        with torch.no_grad():
            model.forward_tokens(prompt, torch.arange(12, device="cuda"))
            kc0 = [k.clone() for k in model.kc]
            vc0 = [v.clone() for v in model.vc]
            tok = torch.randint(0, cfg.vocab, (B, 1), device="cuda")
            pos = torch.tensor([12], device="cuda")
            model.fused_ops = False
            ref = model.decode_tokens(tok, pos).float()
            kref = [k[:, :, 12].clone() for k in model.kc]
            for i in range(cfg.layers):
                model.kc[i].copy_(kc0[i])
                model.vc[i].copy_(vc0[i])
            model.fused_ops = True
            got = model.decode_tokens(tok, pos).float()
        assert rel_l2(got.cpu().numpy(), ref.cpu().numpy()) < 2e-3, (kv, B)
        for i in range(cfg.layers):
            assert rel_l2(model.kc[i][:, :, 12].float().cpu().numpy(), kref[i].float().cpu().numpy()) < 2e-3
        if B <= 2:
            assert len(swiglu) == cfg.layers and len(calls) == cfg.layers and not mc, "fused path for every norm"
        else:
            assert not swiglu and not calls, B
            assert mc.count("norm") == cfg.layers and mc.count("swiglu") == cfg.layers, mc
            assert mc.count("resid") == 2 * cfg.layers, mc
        calls.clear()
        swiglu.clear()
        mc.clear()
    LL.norm_linear, LL.norm_swiglu, LL.QuantLlama._llin = real, real_sw, real_llin
    LL.QuantLlama._llin_swiglu = real_llsw


def test_split_attention_matches_single_workgroup():
    """Decode attention with positions split over workgroups (partials
    combined by the last one) against one workgroup per head, at several
    positions including empty splits, for MHA and GQA."""
    from eptq_amd.kernels import _lib
    lib = _lib.load()
    print("decode attention: split vs single workgroup", flush=True)
    gen = torch.Generator("cuda").manual_seed(5)
    D, L = 128, 1024
    for B, H, Hk in ((1, 32, 32), (2, 8, 2), (3, 4, 4)):
        kc = (torch.randn((B, Hk, L, D), generator=gen, device="cuda") * 0.5).half()
        vc = torch.randn((B, Hk, L, D), generator=gen, device="cuda").half()
        inv = 1.0 / (10000.0 ** (torch.arange(0, D, 2, device="cuda").float() / D))
        f = torch.outer(torch.arange(L, device="cuda").float(), inv)
        emb = torch.cat((f, f), dim=-1)
        cos, sin = emb.cos().contiguous(), emb.sin().contiguous()
        work = torch.zeros(lib.eptq_llama_attn_work_bytes(B, H), dtype=torch.uint8, device="cuda")
        s = torch.cuda.current_stream().cuda_stream
        for p in (0, 5, 17, 300, 1023):
            qkv = torch.randn((B, (H + 2 * Hk) * D), generator=gen, device="cuda").half()
            pos = torch.tensor([p], device="cuda")
            outs, caches = [], []
            for w in (None, work.data_ptr()):
                k2, v2 = kc.clone(), vc.clone()
                out = torch.empty((B, H * D), dtype=torch.float16, device="cuda")
                rc = lib.eptq_llama_rope_attn(qkv.data_ptr(), pos.data_ptr(), cos.data_ptr(), sin.data_ptr(),
                                              k2.data_ptr(), v2.data_ptr(), out.data_ptr(), B, H, Hk, D, L, w, s)
                assert rc == 0
                outs.append(out.float().cpu().numpy())
                caches.append((k2, v2))
            assert rel_l2(outs[1], outs[0]) < 2e-3, (B, H, Hk, p)
            assert torch.equal(caches[0][0], caches[1][0]) and torch.equal(caches[0][1], caches[1][1])
        cnt = work[lib.eptq_llama_attn_work_bytes(B, H) - 4 * B * H:].view(torch.int32)
        assert int(cnt.abs().sum()) == 0, "counters are left at zero"


def test_graph_decoder_refuses_after_model_retargeted():
    """A second GraphDecoder on the same model takes over its caches and
    workspaces; the first then raises instead of launching (its captured
    graph addresses buffers the model no longer uses)."""
    from eptq_amd.llama import GraphDecoder, LlamaConfig, build_synthetic
    print("GraphDecoder: stale decoder refuses to run", flush=True)
    cfg = LlamaConfig(hidden=512, ffn=1024, layers=1, heads=4, kv_heads=4, vocab=256)
    model = build_synthetic(cfg, device="cuda", seed=5)
    prompt = torch.randint(0, cfg.vocab, (2, 8), device="cuda", generator=torch.Generator("cuda").manual_seed(5))
    d1 = GraphDecoder(model, 2, 32, device="cuda")
    d1.prefill(prompt)
    d1.capture()
    d1.step()
    torch.cuda.synchronize()
    d2 = GraphDecoder(model, 2, 32, device="cuda")
    for call in (d1.step, d1.capture, lambda: d1.prefill(prompt)):
        with pytest.raises(RuntimeError, match="newer GraphDecoder"):
            call()
    d2.prefill(prompt)
    d2.step()
    torch.cuda.synchronize()
