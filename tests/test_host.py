"""Host-side logic on the CPU: the on-disk format, the quantizer loaders, the
drop-in ``EPTQLinear`` construction and the model loader, the synthetic
generators and the bench's one-GPU contract.  Forward passes need the GPU (no
CPU fallback exists: calling one on CPU tensors must raise)."""

from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from eptq_amd.config import QuantizedLayerData
from eptq_amd.handlers import LlamaHandler, ModelHandler, OPTHandler, get_model_handler_by_type
from eptq_amd.kernels.linear import EPTQLinear, QuantizedLinear
from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.quantizers.e8_d4 import e8d4_raw_codes
from eptq_amd.reconstruct import load_quantizer, load_quantized_layer, save_quantizer
from eptq_amd.synthetic import make_layer, make_x, write_quantized_model
from oracle.dequant import build_csr

ROOT = Path(__file__).resolve().parent.parent


# ------------------------------------------------------------ format -------

def test_layer_data_roundtrip(tmp_path):
    qd = make_layer(64, 40, seed=1, percmask=0.05, bias=True, qb_size=16, chosen_r=1.8)
    qd.save(tmp_path / "l.pt")
    back = QuantizedLayerData.load(tmp_path / "l.pt")
    for k in ("Q", "g", "h", "O", "bias", "S_group"):
        assert torch.equal(getattr(back, k), getattr(qd, k)), k
    assert back.chosen_r == 1.8 and back.out_features == 64 and back.in_features == 40


def test_layer_data_optional_keys_absent(tmp_path):
    qd = make_layer(16, 8, seed=2, percmask=0.0)
    torch.save({"Q": qd.Q, "g": qd.g, "h": qd.h, "O": qd.O}, tmp_path / "old.pt")
    back = load_quantized_layer(tmp_path, "old")
    assert back.bias is None and back.chosen_r is None and back.S_group is None


def test_synthetic_layer_properties():
    qd = make_layer(256, 512, seed=3, percmask=0.002, bias=True, qb_size=128)
    M, N = 32, 512
    assert qd.Q.dtype == torch.int16 and qd.Q.shape == (M, N)
    nnz = round(0.002 * M * N)
    assert int((qd.Q == 32767).sum()) == nnz == qd.O.shape[0]
    assert qd.O.shape == (nnz, 8) and qd.g.dtype == torch.float16 and qd.S_group.shape == (2, N)
    assert (qd.g > 0).all() and (qd.h > 0).all()
    again = make_layer(256, 512, seed=3, percmask=0.002, bias=True, qb_size=128)
    assert torch.equal(again.Q, qd.Q) and torch.equal(again.O, qd.O)
    assert make_x(2, 512, seed=5).shape == (2, 512)
    with pytest.raises(ValueError):
        make_layer(12, 8, seed=0, percmask=0.0)
    with pytest.raises(ValueError):
        make_layer(64, 8, seed=0, percmask=0.0, qb_size=12)


# ------------------------------------------------------------ quantizers ---

@pytest.mark.parametrize("qtype", ["e8_d4", "e8_lattice"])
def test_load_quantizer_new_format(tmp_path, qtype):
    q = E8D4Quantizer(radius=1.75) if qtype == "e8_d4" else E8LatticeQuantizer(radius=1.6)
    save_quantizer(q, tmp_path, qtype)
    back = load_quantizer(tmp_path, device="cpu")
    assert type(back) is type(q) and back._radius == q._radius
    assert torch.equal(back.flat_table(), q.flat_table())
    back.set_radius(2.0)   # raw codes kept: exact raw / r
    raw = back._raw_codes if qtype == "e8_d4" else back._raw_points
    assert torch.equal(back.flat_table(), (raw / 2.0).reshape(back.flat_table().shape))


def test_load_quantizer_mid_and_old_formats(tmp_path):
    raw = torch.from_numpy(e8d4_raw_codes())
    torch.save({"quantizer_type": "e8_d4", "codebook": raw / 1.7, "saved_radius": 1.7}, tmp_path / "quantizer.pt")
    q = load_quantizer(tmp_path, device="cpu")
    assert q._radius == 1.7 and torch.equal(q.codes, raw / 1.7)
    torch.save({"quantizer_type": "e8_d4", "codebook": raw / 1.9}, tmp_path / "quantizer.pt")
    (tmp_path / "quant_config.json").write_text(json.dumps({"codebook_radius": 1.9}))
    q = load_quantizer(tmp_path, device="cpu")
    assert q._radius == 1.9
    q.set_radius(1.8)      # no raw codes: in-place rescale by r_old / r_new
    assert torch.allclose(q.codes, raw / 1.8, rtol=1e-6)
    torch.save({"quantizer_type": "nope", "codebook": raw}, tmp_path / "quantizer.pt")
    with pytest.raises(ValueError):
        load_quantizer(tmp_path, device="cpu")


def test_warp_codebook_identity_at_alpha_one():
    q = E8D4Quantizer(radius=1.75)
    before = q.codes.clone()
    q.warp_codebook(1.0)
    assert torch.allclose(q.codes, before, rtol=1e-6, atol=0)


def test_quantizer_dequant_matches_table_layout():
    q = E8D4Quantizer(radius=1.75)
    u = torch.tensor([[0x0000, 0x7FFF], [0xC0FF, 0x4321]], dtype=torch.int64)
    W = q.dequant(u, 1.0)
    t = q.flat_table()
    for m in range(2):
        for n in range(2):
            v = int(u[m, n])
            want = torch.cat([t[((v >> 14) & 3) * 128 + ((v >> 7) & 127)], t[((v >> 14) & 3) * 128 + (v & 127)]])
            assert torch.equal(W[8 * m:8 * m + 8, n], want)


# ------------------------------------------------------------ EPTQLinear ---

def test_eptqlinear_builds_csr_and_shared_tables():
    qd = make_layer(64, 48, seed=4, percmask=0.05, bias=True)
    q = E8D4Quantizer(radius=1.75)
    lin = EPTQLinear.from_quantized_data(qd, q, "e8_d4")
    cols, rp = build_csr(qd.Q.numpy())
    assert lin.O_col.tolist() == cols.tolist() and lin.O_row_ptr.tolist() == rp.tolist()
    assert lin.in_features == 48 and lin.out_features == 64 and QuantizedLinear is EPTQLinear
    assert lin._codebook.dtype == torch.float16 and lin._codebook.shape == (512, 4)
    assert torch.equal(lin._table_f32, q.flat_table())
    assert "Q" in lin.state_dict() and "_codebook" not in lin.state_dict()
    lin2 = EPTQLinear.from_quantized_data(make_layer(64, 48, seed=5, percmask=0.0), q, "e8_d4")
    assert lin2._table_f32 is lin._table_f32       # one table per (quantizer, radius)


def test_eptqlinear_honours_chosen_r():
    q = E8D4Quantizer(radius=1.75)
    qd = make_layer(32, 16, seed=6, percmask=0.0, chosen_r=1.9)
    lin = EPTQLinear.from_quantized_data(qd, q, "e8_d4")
    assert torch.equal(lin._table_f32, (q._raw_codes / 1.9).reshape(512, 4))
    assert q._radius == 1.75 and torch.equal(q.codes, q._raw_codes / 1.75)


def test_eptqlinear_rejects_bad_inputs():
    q = E8D4Quantizer(radius=1.75)
    qd = make_layer(32, 16, seed=7, percmask=0.1)
    bad = QuantizedLayerData(Q=qd.Q, g=qd.g, h=qd.h, O=qd.O[:-1])
    with pytest.raises(ValueError, match="inconsistent"):
        EPTQLinear.from_quantized_data(bad, q, "e8_d4")
    with pytest.raises(ValueError):
        EPTQLinear.from_quantized_data(qd, q, "e8_q")
    with pytest.raises(ValueError):
        EPTQLinear.from_quantized_data(QuantizedLayerData(Q=qd.Q.int(), g=qd.g, h=qd.h, O=qd.O), q, "e8_d4")


def test_forward_has_no_cpu_fallback():
    lin = EPTQLinear.from_quantized_data(make_layer(32, 16, seed=8, percmask=0.0),
                                         E8D4Quantizer(radius=1.75), "e8_d4")
    with pytest.raises(RuntimeError, match="HIP"):
        lin(torch.zeros(1, 16, dtype=torch.float16))


def test_custom_ops_registered_with_fake_impls():
    import eptq_amd.kernels  # noqa: F401  (registers the ops)
    from torch._subclasses.fake_tensor import FakeTensorMode
    for name in ("e8_forward", "e8d4_forward", "e8_forward_grouped", "e8d4_forward_grouped",
                 "e8_dequant", "e8d4_dequant"):
        assert hasattr(torch.ops.eptq, name)
    with FakeTensorMode():
        Q = torch.empty(4, 64, dtype=torch.int16)
        y = torch.ops.eptq.e8d4_forward(Q, torch.empty(512, 4, dtype=torch.float16),
                                        torch.empty(32, dtype=torch.float16), torch.empty(64, dtype=torch.float16),
                                        torch.empty(3, 64, dtype=torch.float16), torch.empty(0, 8, dtype=torch.float16),
                                        torch.empty(0, dtype=torch.int32), torch.empty(5, dtype=torch.int32),
                                        torch.empty(0, dtype=torch.float16))
        assert y.shape == (3, 32)


# ------------------------------------------------------------ model loader ---

def _tiny_tokenizer():
    from tokenizers import Tokenizer, models, pre_tokenizers
    from transformers import PreTrainedTokenizerFast
    vocab = {f"t{i}": i for i in range(120)}
    vocab["<unk>"] = 120
    tok = Tokenizer(models.WordLevel(vocab=vocab, unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.Whitespace()
    return PreTrainedTokenizerFast(tokenizer_object=tok, unk_token="<unk>")


@pytest.fixture(scope="module")
def tiny_dir(tmp_path_factory):
    from transformers import LlamaConfig
    d = tmp_path_factory.mktemp("qmodel")
    cfg = LlamaConfig(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    write_quantized_model(d, cfg, percmask=0.02, seed=3, tokenizer=_tiny_tokenizer())
    return d


def test_load_quantized_model_swaps_every_decoder_linear(tiny_dir):
    from eptq_amd.kernels.patch import load_quantized_model
    model, tok = load_quantized_model(str(tiny_dir), device="cpu")
    handler = LlamaHandler()
    layers = handler.get_layers(model)
    assert len(layers) == 2
    for lid, layer in enumerate(layers):
        lins = {n: m for n, m in layer.named_modules() if isinstance(m, EPTQLinear)}
        assert set(lins) == {"self_attn.q_proj", "self_attn.k_proj", "self_attn.v_proj", "self_attn.o_proj",
                             "mlp.gate_proj", "mlp.up_proj", "mlp.down_proj"}
        assert not any(isinstance(m, torch.nn.Linear) for m in layer.modules())
        qd = load_quantized_layer(tiny_dir / f"layer_{lid}", "self_attn.k_proj")
        assert torch.equal(lins["self_attn.k_proj"].Q, qd.Q) and lins["self_attn.k_proj"].out_features == 32
    assert not any(p.is_meta for p in model.parameters())
    glob = torch.load(tiny_dir / "non_quantized_params.pt", weights_only=True)
    assert torch.equal(model.lm_head.weight.data, glob["lm_head.weight"])
    assert tok("t1 t2")["input_ids"] == [1, 2]


def test_handlers():
    assert isinstance(get_model_handler_by_type("llama"), LlamaHandler)
    assert isinstance(get_model_handler_by_type("opt"), OPTHandler)
    with pytest.raises(ValueError):
        get_model_handler_by_type("gpt2")

    class OPTForCausalLM(torch.nn.Module):
        pass
    assert ModelHandler.detect_model_type(OPTForCausalLM()) == "opt"


# ------------------------------------------------------------ bench ---------

def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True,
                       text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_bench_algorithmic_bytes():
    sys.path.insert(0, str(ROOT))
    from bench import algo_bytes
    # Q 2MN + CSR 20·nnz + 4(M+1) + g 2·out + h 2·in + x 2·B·in + y 2·B·out
    assert algo_bytes(4096, 4096, 1, 0) == 2 * 512 * 4096 + 4 * 513 + 2 * 4096 * 2 + 2 * 4096 * 2
    assert algo_bytes(64, 32, 2, 3, bias=True, n_groups=2) - algo_bytes(64, 32, 2, 3) == 2 * 64 + 2 * 2 * 32
