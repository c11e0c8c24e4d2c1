"""GPU: the drop-in modules under torch.compile and under graph capture.

The reference's decode numbers are measured with the model compiled
(``bench_decode.py:146-149``) and its ops registered so that torch.compile
"sees these as first-class ops (no graph break) and can wrap them in CUDA
graphs" (``kernels/__init__.py:44-47``).  Checks:

* a tiny Llama from ``load_quantized_model`` compiled with
  ``fullgraph=True`` (``aot_eager``, and the ``cudagraphs`` backend, which
  replays the compiled forward as a captured graph) gives the eager logits
  and stays within the 2e-2 bar of a dense fp32 model over the oracle's W —
  at 8 tokens (the vector decode kernel), 16 (the matrix-core kernel with the
  stream's split-K workspace looked up inside the op) and 40 (16-row slices);
* eager modules captured into two ``torch.cuda.graph``s in a row on the
  default capture stream (no workspace exists for that stream, so none is
  made during the capture, and the captured launches are the unsplit
  kernel's), the second replayed first with eager work between replays:
  every replay bit-identical to the unsplit call and within rounding of the
  eager split-K result; and modules with an attached workspace, captured and
  replayed, bit-identical to eager, with the split-K counters back at zero.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def tiny_model(tmp_path_factory):
    from transformers import LlamaConfig
    from eptq_amd.kernels.patch import load_quantized_model
    from eptq_amd.synthetic import write_quantized_model
    from test_host import _tiny_tokenizer
    d = tmp_path_factory.mktemp("qmodel_compile")
    cfg = LlamaConfig(vocab_size=128, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=64)
    write_quantized_model(d, cfg, percmask=0.02, seed=21, tokenizer=_tiny_tokenizer())
    model, _ = load_quantized_model(str(d), device="cuda")
    return d, model


class _Logits(torch.nn.Module):
    def __init__(self, m):
        super().__init__()
        self.m = m

    def forward(self, ids):
        return self.m(ids, use_cache=False).logits


def _dense_reference(d, model):
    from transformers import AutoConfig, AutoModelForCausalLM
    ref = AutoModelForCausalLM.from_config(AutoConfig.from_pretrained(d)).float().eval()
    sd = {}
    for name, mod in model.named_modules():
        if isinstance(mod, EPTQLinear):
            W = dequantize_layer(mod.Q.cpu().numpy(), mod.g.cpu().numpy(), mod.h.cpu().numpy(),
                                 mod.O_vals.cpu().numpy(), mod._table_f32.cpu().numpy(), mod.quantizer_type)
            sd[name + ".weight"] = torch.from_numpy(W.astype(np.float32))
    for name, p in model.named_parameters():
        sd[name] = p.detach().float().cpu()
    ref.load_state_dict(sd, strict=False)
    return ref


@pytest.mark.parametrize("backend", ["aot_eager", "cudagraphs"])
def test_compiled_tiny_llama_matches_eager_and_oracle(tiny_model, backend):
    d, model = tiny_model
    ref = _dense_reference(d, model)
    gen = torch.Generator().manual_seed(3)
    torch._dynamo.reset()
    wrapped = _Logits(model)
    compiled = torch.compile(wrapped, fullgraph=True, backend=backend)
    for shape in ((1, 8), (2, 8), (1, 40)):
        print(f"compiled tiny llama ({backend}), ids {shape}", flush=True)
        ids = torch.randint(0, 128, shape, generator=gen)
        with torch.no_grad():
            eager = wrapped(ids.cuda()).float()
            for rep in range(3):
                got = compiled(ids.cuda()).float()
                torch.cuda.synchronize()
                err = rel_l2(got.cpu().numpy(), eager.cpu().numpy())
                print(f"  replay {rep}: rel-L2 vs eager {err:.2e}, bit-equal {torch.equal(got, eager)}")
                assert err <= 1e-3, (shape, rep, err)
            want = ref(ids).logits.numpy()
        assert rel_l2(got.cpu().numpy(), want) <= 2e-2, shape


def _layers():
    from eptq_amd.quantizers import E8D4Quantizer
    from eptq_amd.synthetic import make_layer
    q = E8D4Quantizer(radius=1.75)
    single = EPTQLinear.from_quantized_data(make_layer(512, 1024, seed=31, percmask=0.002, bias=True), q,
                                            "e8_d4").cuda()
    multi = EPTQMultiLinear([EPTQLinear.from_quantized_data(make_layer(o, 1024, seed=40 + o, percmask=0.002), q,
                                                            "e8_d4").cuda() for o in (512, 128, 128)])
    return single, multi


def test_two_graphs_on_the_default_capture_stream():
    """ADVICE case: the first module call of a stream happens under capture."""
    print("torch.cuda.graph x2 on the default capture stream, second replayed first", flush=True)
    single, multi = _layers()
    x = torch.randn(8, 1024, generator=torch.Generator().manual_seed(1)).half().cuda()
    with torch.no_grad():
        want_s, want_m = single(x), multi(x)
    torch.cuda.synchronize()
    g1, g2 = torch.cuda.CUDAGraph(), torch.cuda.CUDAGraph()
    with torch.no_grad():
        with torch.cuda.graph(g1):
            ys = single(x)
        with torch.cuda.graph(g2):
            ym = multi(x)
    # The captures ran the unsplit kernel (no workspace is made during a
    # capture), the eager calls the split-K form of the stream's workspace:
    # the same sums in another order, so equal to rounding; every replay is
    # bit-identical to the first.
    first = None
    for rep in range(4):
        g2.replay()
        torch.cuda.synchronize()
        with torch.no_grad():
            assert torch.equal(multi(x), want_m)   # eager work between replays
        g1.replay()
        torch.cuda.synchronize()
        if first is None:
            first = (ys.clone(), ym.clone())
            assert rel_l2(ys.float().cpu().numpy(), want_s.float().cpu().numpy()) <= 1e-3
            assert rel_l2(ym.float().cpu().numpy(), want_m.float().cpu().numpy()) <= 1e-3
        assert torch.equal(ys, first[0]) and torch.equal(ym, first[1]), rep
    from eptq_amd.kernels import linear_forward_multi
    layers = [dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr, bias=l.bias,
                   S_group=l.S_group) for l in multi.parts]
    assert torch.equal(linear_forward_multi(layers, multi.parts[0]._codebook, x, work=None), first[1])


def test_graph_with_attached_workspace_matches_eager():
    from eptq_amd.kernels import decode_workspace
    print("torch.cuda.graph with an attached split-K workspace", flush=True)
    single, multi = _layers()
    ws = decode_workspace("cuda")
    single._work = ws
    multi._work = ws
    x = torch.randn(12, 1024, generator=torch.Generator().manual_seed(2)).half().cuda()
    with torch.no_grad():
        want_s, want_m = single(x), multi(x)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(g):
        ys = single(x)
        ym = multi(x)
    for rep in range(4):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(ys, want_s) and torch.equal(ym, want_m), rep
    counters = ws[:4 * 64].view(torch.int32)
    assert int(counters.abs().sum()) == 0, "split-K counters return to zero"
