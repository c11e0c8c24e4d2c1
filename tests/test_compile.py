"""torch.compile traces the drop-in modules with no graph break (CPU).

The reference registers its kernels as custom ops "so torch.compile sees these
as first-class ops (no graph break)" (``kernels/__init__.py:44-47``) and
publishes its decode numbers under ``torch.compile(..., fullgraph=True)``
(``bench_decode.py:146-149``).  Here the modules are moved to the ``meta``
device, where every ``eptq::`` op runs its fake implementation, and compiled
with ``fullgraph=True`` (which raises on any graph break): single E8-D4, E8
and S_group layers, the multi-layer module, and a whole tiny Llama from
``load_quantized_model``.  The captured graphs must hold the ``eptq::`` ops
and nothing that touches ctypes.  The same compiled path runs on the GPU in
``tests/test_gpu_compile.py``.
"""

from __future__ import annotations

import pytest
import torch
from torch._dynamo.backends.common import aot_autograd

import eptq_amd.kernels  # noqa: F401  (registers the eptq:: ops)
from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.synthetic import make_layer


def _recording_backend(graphs):
    def fw(gm, example_inputs):
        graphs.append(gm)
        return gm
    return aot_autograd(fw_compiler=fw)


def _eptq_targets(gm):
    out = []
    for n in gm.graph.nodes:
        t = n.target
        if n.op == "call_function" and "auto_functionalized" in str(t):
            t = n.args[0]
        if n.op == "call_function" and "eptq" in str(t):
            out.append(str(t))
    return out


def _compile_and_run(mod, x):
    graphs = []
    torch._dynamo.reset()
    c = torch.compile(mod, fullgraph=True, backend=_recording_backend(graphs))
    y = c(x)
    assert len(graphs) == 1, f"{len(graphs)} graphs: a graph break"
    return y, graphs[0]


@pytest.mark.parametrize("kind,groups", [("e8_d4", False), ("e8_d4", True), ("e8_lattice", False),
                                         ("e8_lattice", True)])
def test_single_linear_compiles_fullgraph(kind, groups):
    q = E8D4Quantizer(radius=1.75) if kind == "e8_d4" else E8LatticeQuantizer(radius=1.6)
    qd = make_layer(64, 128, seed=11, percmask=0.01, bias=True, qb_size=32 if groups else None)
    lin = EPTQLinear.from_quantized_data(qd, q, kind).to("meta")
    for dt in (torch.float16, torch.bfloat16, torch.float32):
        x = torch.empty(2, 3, 128, dtype=dt, device="meta")
        y, gm = _compile_and_run(lin, x)
        assert y.shape == (2, 3, 64) and y.dtype == dt and y.device.type == "meta"
        want = "eptq.e8d4_forward_multi" if kind == "e8_d4" else (
            "eptq.e8_forward_grouped" if groups else "eptq.e8_forward")
        assert any(want in t for t in _eptq_targets(gm)), _eptq_targets(gm)


def test_multi_linear_compiles_fullgraph_with_and_without_workspace():
    q = E8D4Quantizer(radius=1.75)
    lins = [EPTQLinear.from_quantized_data(make_layer(o, 128, seed=20 + o, percmask=0.01), q, "e8_d4")
            for o in (64, 32, 32)]
    mod = EPTQMultiLinear(lins).to("meta")
    x = torch.empty(8, 128, dtype=torch.float16, device="meta")
    y, gm = _compile_and_run(mod, x)
    assert y.shape == (8, 128)
    assert _eptq_targets(gm) == ["eptq.e8d4_forward_multi.default"]
    # An attached workspace is a graph input the op mutates.
    mod._work = torch.empty(1024, dtype=torch.uint8, device="meta")
    y, gm = _compile_and_run(mod, x)
    assert y.shape == (8, 128)
    assert _eptq_targets(gm) == ["eptq.e8d4_forward_multi.default"]


def test_eager_forward_calls_only_registered_ops(monkeypatch):
    """The module forward reaches the library only through torch.ops.eptq.*:
    with the ctypes entry points replaced by a raising stub, the meta-device
    forward (fake implementations) still runs."""
    from eptq_amd.kernels import _lib

    def boom(*a, **k):
        raise AssertionError("ctypes path reached from the module forward")
    monkeypatch.setattr(_lib, "load", boom)
    q = E8D4Quantizer(radius=1.75)
    lin = EPTQLinear.from_quantized_data(make_layer(64, 128, seed=3, percmask=0.01), q, "e8_d4").to("meta")
    assert lin(torch.empty(5, 128, dtype=torch.float16, device="meta")).shape == (5, 64)


def test_tiny_llama_from_loader_compiles_fullgraph(tmp_path):
    from transformers import LlamaConfig
    from eptq_amd.kernels.patch import load_quantized_model
    from eptq_amd.synthetic import write_quantized_model
    from test_host import _tiny_tokenizer
    cfg = LlamaConfig(vocab_size=128, hidden_size=64, intermediate_size=128, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    write_quantized_model(tmp_path, cfg, percmask=0.02, seed=3, tokenizer=_tiny_tokenizer())
    model, _ = load_quantized_model(str(tmp_path), device="cpu")
    model = model.to("meta")
    ids = torch.zeros(1, 8, dtype=torch.long, device="meta")

    class Logits(torch.nn.Module):
        def __init__(self, m):
            super().__init__()
            self.m = m

        def forward(self, ids):
            return self.m(ids, use_cache=False).logits

    with torch.no_grad():
        y, gm = _compile_and_run(Logits(model), ids)
    assert y.shape == (1, 8, 128)
    # 2 layers x (q, k, v, o, gate, up, down), one op each.
    assert len(_eptq_targets(gm)) == 14, _eptq_targets(gm)
