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


def test_llama_graph_decode_matches_eager():
    from eptq_amd.llama import GraphDecoder, LlamaConfig, build_synthetic
    print("synthetic llama: graph vs eager decode", flush=True)
    cfg = LlamaConfig(hidden=256, ffn=512, layers=2, heads=4, kv_heads=4, vocab=512)
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
