"""GPU: benchmark configuration 4 at its real size — the synthetic
Llama-2-7B (32 layers, hidden 4096, FFN 11008, 32 heads, vocab 32000, every
decoder Linear a synthetic E8-D4 layer at radius 1.75 with 0.2% critical
blocks), 128-token random prompt, greedy decode at batch 1 and 8.

* Two layers' GPU weights (``k_dequant``) are uint16-equal to the oracle's
  ``dequantize_layer``.
* The first decode step's logits match a dense reference: the same network
  with every matmul and the attention in fp32 over those exact weights
  (activations rounded to fp16 where the model's modules output fp16, as the
  reference's own reconstruct path runs the model in fp16), within 1e-2
  relative L2.
* Eight greedy steps replayed from the captured HIP graph give the tokens
  of eight eager steps.
* Past the attention kernel's 256-row chunks: prompts of 254 and 510 tokens,
  three greedy steps, then the logits at position 257 (two chunks) and 513
  (three chunks) against the same dense reference.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu

PROMPT = 128


@pytest.fixture(scope="module")
def llama7b():
    from eptq_amd.llama import LLAMA2_7B, build_synthetic
    print("building synthetic Llama-2-7B (224 E8-D4 layers)", flush=True)
    model = build_synthetic(LLAMA2_7B, device="cuda", seed=4000, percmask=0.002)
    torch.cuda.synchronize()
    print("built", flush=True)
    return model


def _rms(x16, w, eps):
    xf = x16.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps) * w.float()).half()


def _rope(x, cos, sin):
    d = x.shape[-1] // 2
    return x * cos + torch.cat((-x[..., d:], x[..., :d]), dim=-1) * sin


@torch.no_grad()
def _dense_last_logits(model, ids):
    """Logits at the last position of ids (B, T), fp32 matmuls and attention
    over the GPU-dequantized weights."""
    cfg = model.cfg
    B, T = ids.shape
    H, Hk, D = cfg.heads, cfg.kv_heads, cfg.head_dim
    x = model.embed_tokens.weight[ids]                       # (B, T, hidden) fp16
    pos = torch.arange(T, device=ids.device).float()
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, D, 2, device=ids.device).float() / D))
    f = torch.outer(pos, inv)
    emb = torch.cat((f, f), dim=-1)
    cos, sin = emb.cos()[None, None], emb.sin()[None, None]
    causal = torch.full((T, T), float("-inf"), device=ids.device).triu(1)

    def lin(mod, a):
        W = torch.cat([p.dequantize() for p in (mod.parts if hasattr(mod, "parts") else [mod])]).float()
        return torch.matmul(a.float(), W.t()).half()

    for layer in model.layers:
        h = _rms(x, layer.input_layernorm.weight, cfg.eps)
        qkv = lin(layer.qkv_proj, h)
        q, k, v = qkv.split([H * D, Hk * D, Hk * D], dim=-1)
        q = _rope(q.reshape(B, T, H, D).transpose(1, 2).float(), cos, sin).half().float()
        k = _rope(k.reshape(B, T, Hk, D).transpose(1, 2).float(), cos, sin).half().float()
        v = v.reshape(B, T, Hk, D).transpose(1, 2).float()
        if Hk != H:
            k = k.repeat_interleave(H // Hk, dim=1)
            v = v.repeat_interleave(H // Hk, dim=1)
        s = torch.matmul(q, k.transpose(-1, -2).contiguous()) / math.sqrt(D) + causal
        o = torch.matmul(torch.softmax(s, dim=-1), v).half()
        o = o.transpose(1, 2).reshape(B, T, H * D)
        x = x + lin(layer.o_proj, o)
        h = _rms(x, layer.post_attention_layernorm.weight, cfg.eps)
        gu = lin(layer.gate_up_proj, h).float()
        a = (torch.nn.functional.silu(gu[..., :cfg.ffn]) * gu[..., cfg.ffn:]).half()
        x = x + lin(layer.down_proj, a)
    h = _rms(x[:, -1], model.norm.weight, cfg.eps)
    return torch.matmul(h.float(), model.lm_head.weight.float().t())


def test_llama7b_weights_bit_exact(llama7b):
    print("config 4: two layers' GPU W vs the oracle", flush=True)
    for mod in (llama7b.layers[0].qkv_proj.parts[0], llama7b.layers[31].down_proj):
        W = mod.dequantize().cpu().numpy()
        ref = dequantize_layer(mod.Q.cpu().numpy(), mod.g.cpu().numpy(), mod.h.cpu().numpy(),
                               mod.O_vals.cpu().numpy(), mod._table_f32.cpu().numpy(), "e8_d4")
        assert np.array_equal(W.view(np.uint16), ref.view(np.uint16))


@pytest.mark.parametrize("B", [1, 8])
def test_llama7b_decode(llama7b, B):
    from eptq_amd.llama import GraphDecoder
    print(f"config 4 at B={B}: prefill {PROMPT} tokens", flush=True)
    dec = GraphDecoder(llama7b, B, PROMPT + 16, device="cuda")
    gen = torch.Generator("cuda").manual_seed(100 + B)
    prompt = torch.randint(0, llama7b.cfg.vocab, (B, PROMPT), device="cuda", generator=gen)
    t1 = dec.prefill(prompt).clone()
    with torch.no_grad():
        logits = llama7b.decode_next(dec.tok, dec.pos).float()
    torch.cuda.synchronize()
    print(f"config 4 at B={B}: dense fp32 reference", flush=True)
    want = _dense_last_logits(llama7b, torch.cat([prompt, t1], dim=1))
    err = rel_l2(logits.cpu().numpy(), want.cpu().numpy())
    print(f"config 4 at B={B}: step-1 logits rel_l2 {err:.3e}", flush=True)
    assert err <= 1e-2

    print(f"config 4 at B={B}: 8 eager steps vs 8 graph replays", flush=True)
    eager = []
    dec.tok.copy_(t1)
    dec.pos.fill_(PROMPT)
    for _ in range(8):
        dec.step()
        eager.append(dec.tok.clone())
    dec.tok.copy_(t1)
    dec.pos.fill_(PROMPT)
    dec.capture()
    for i in range(8):
        dec.step()
        torch.cuda.synchronize()
        assert torch.equal(dec.tok, eager[i]), f"step {i}"
    assert int(dec.pos.item()) == PROMPT + 8
    dec.graph = None


@pytest.mark.parametrize("P", [254, 510])
def test_llama7b_decode_past_chunks(llama7b, P):
    from eptq_amd.llama import GraphDecoder
    print(f"config 4 at B=1: prefill {P} tokens, 3 steps, logits at {P + 3}", flush=True)
    dec = GraphDecoder(llama7b, 1, P + 8, device="cuda")
    gen = torch.Generator("cuda").manual_seed(300 + P)
    prompt = torch.randint(0, llama7b.cfg.vocab, (1, P), device="cuda", generator=gen)
    toks = [dec.prefill(prompt).clone()]
    for _ in range(3):
        dec.step()
        toks.append(dec.tok.clone())
    assert int(dec.pos.item()) == P + 3
    with torch.no_grad():
        logits = llama7b.decode_next(dec.tok, dec.pos).float()
    torch.cuda.synchronize()
    want = _dense_last_logits(llama7b, torch.cat([prompt] + toks, dim=1))
    err = rel_l2(logits.cpu().numpy(), want.cpu().numpy())
    print(f"config 4 at B=1, position {P + 3}: logits rel_l2 {err:.3e}", flush=True)
    assert err <= 1e-2
