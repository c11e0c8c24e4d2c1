"""GPU: batch-1 chains of dependent E8-D4 Linears in one launch (``eptq_amd.chain``).

Every stage's output is checked against the oracle (``oracle/chain.py``:
the stage input formed from the GPU's own source output — slice, SwiGLU,
RMSNorm — then the fp32 reconstruct + matmul of every layer) within the
1e-2 relative-L2 bar, so an error is pinned to its stage.  Also: repeated
runs and a HIP-graph replay of a run are bit-identical to the first run (the
run number advances; nothing is reset), and a wait forced to expire from the
host (a zero spin bound) sets the error word, every workgroup leaves, and
the next run after clearing it is exact again.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.chain import SLICE, SWIGLU, DecodeChain, llama_stages
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.chain import stage_input, stage_ref
from oracle.matvec import rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2
NAMES = ("q", "k", "v", "o", "gate", "up", "down")


def _stack(hidden, ffn, n_layers, p, seed, kv=None, bias=False):
    q = E8D4Quantizer(radius=1.75)
    kvo = kv or hidden
    layers, raw, norms = [], [], []
    for i in range(n_layers):
        shapes = dict(q=(hidden, hidden), k=(kvo, hidden), v=(kvo, hidden), o=(hidden, hidden),
                      gate=(ffn, hidden), up=(ffn, hidden), down=(hidden, ffn))
        qd = {k: make_layer(o, n, seed=seed + 10 * i + j, percmask=p, bias=bias and k in ("q", "o", "down"))
              for j, (k, (o, n)) in enumerate(shapes.items())}
        layers.append({k: EPTQLinear.from_quantized_data(v, q, "e8_d4").cuda() for k, v in qd.items()})
        raw.append({k: layer_np(v) for k, v in qd.items()})
        g = torch.Generator().manual_seed(seed + i)
        norms.append(tuple((1 + 0.1 * torch.randn(hidden, generator=g)).half().cuda() for _ in range(2)))
    return layers, raw, norms


def _raw_stages(raw):
    out = []
    for R in raw:
        out += [[R["q"], R["k"], R["v"]], [R["o"]], [R["gate"], R["up"]], [R["down"]]]
    return out


def _check(chain, stages, raw_stages, x0):
    tab = table("e8_d4", 1.75)
    worst = 0.0
    for s, st in enumerate(stages):
        src = x0.cpu().numpy() if st["src"] < 0 else chain.y[st["src"]].cpu().numpy()
        nw = st.get("norm_weight")
        x = stage_input(src, st.get("src_col", 0), st["layers"][0].in_features, st.get("act", SLICE),
                        None if nw is None else nw.cpu().numpy(), st.get("eps", 1e-5))
        want = stage_ref(x, raw_stages[s], tab)
        got = chain.y[s].float().cpu().numpy()
        assert np.isfinite(got).all(), s
        err = rel_l2(got, want)
        worst = max(worst, err)
        assert err <= TOL, (s, err)
    return worst


def test_small_llama_chain_matches_oracle_and_repeats_exactly():
    print("chain: 3-layer llama stack hidden 512 ffn 1024 (12 stages), norms and biases", flush=True)
    layers, raw, norms = _stack(512, 1024, 3, p=0.01, seed=300, kv=256, bias=True)
    stages = llama_stages(layers, norms)
    chain = DecodeChain(stages)
    x0 = make_x(1, 512, seed=9)[0].cuda()
    chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 0
    print(f"  worst stage rel-L2 {_check(chain, stages, _raw_stages(raw), x0):.2e}")
    first = [y.clone() for y in chain.y]
    for rep in range(3):
        chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 0
    assert all(torch.equal(a, b) for a, b in zip(first, chain.y))
    # A captured run replays bit-identically (the run number lives on the device).
    for y in chain.y:
        y.zero_()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            chain.run(x0)
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert all(torch.equal(a, b) for a, b in zip(first, chain.y)), rep
    assert chain.error() == 0


def test_chain_slices_and_offsets():
    """Stages reading inner slices of earlier outputs (not only the leading
    columns), a stage fed by the chain input twice, SwiGLU without a norm."""
    print("chain: slice offsets, SwiGLU, two x-sourced stages", flush=True)
    q = E8D4Quantizer(radius=1.75)
    # (out, in, seed) of each stage's layers.
    spec = [[(256, 384, 1), (512, 384, 2)],    # 0: x -> 768 outputs
            [(384, 256, 3)],                   # 1: stage 0 columns [512, 768)
            [(128, 384, 4), (64, 384, 5)],     # 2: x again -> 192 outputs
            [(96, 64, 7)],                     # 3: SwiGLU(stage 2 [64, 128), [128, 192))
            [(256, 192, 6)]]                   # 4: stage 1 columns [128, 320)
    src = [(-1, 0, SLICE), (0, 512, SLICE), (-1, 0, SLICE), (2, 64, SWIGLU), (1, 128, SLICE)]
    qds = [[make_layer(o, n, seed=sd, percmask=0.02) for o, n, sd in st] for st in spec]
    stages = [dict(layers=[EPTQLinear.from_quantized_data(d, q, "e8_d4").cuda() for d in ds], src=a, src_col=c, act=t)
              for ds, (a, c, t) in zip(qds, src)]
    raw = [[layer_np(d) for d in ds] for ds in qds]
    chain = DecodeChain(stages)
    x0 = make_x(1, 384, seed=4)[0].cuda()
    chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 0
    _check(chain, stages, raw, x0)


def test_llama2_7b_layer_chain_matches_oracle():
    print("chain: one Llama-2-7B decoder layer (4 stages), norms, 0.1% critical blocks", flush=True)
    layers, raw, norms = _stack(4096, 11008, 1, p=0.001, seed=700)
    stages = llama_stages(layers, norms)
    chain = DecodeChain(stages)
    x0 = make_x(1, 4096, seed=11)[0].cuda()
    chain.run(x0)
    chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 0
    print(f"  worst stage rel-L2 {_check(chain, stages, _raw_stages(raw), x0):.2e}")


def test_expired_wait_sets_the_error_word_and_clears():
    print("chain: zero spin bound -> error word; cleared -> exact again", flush=True)
    layers, raw, norms = _stack(512, 1024, 2, p=0.01, seed=900, kv=256)
    stages = llama_stages(layers, norms)
    chain = DecodeChain(stages)
    x0 = make_x(1, 512, seed=2)[0].cuda()
    spin = chain.plan.spin_ticks
    chain.plan.spin_ticks = 0
    chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 1
    chain.plan.spin_ticks = spin
    chain.run(x0)          # the error word is sticky: this run leaves at once
    torch.cuda.synchronize()
    assert chain.error(clear=True) == 1
    assert chain.error() == 0
    chain.run(x0)
    torch.cuda.synchronize()
    assert chain.error() == 0
    _check(chain, stages, _raw_stages(raw), x0)


def test_host_operands_are_refused_before_any_launch():
    """A module whose codebook never left the host (EPTQLinear built from
    host data and not moved) is refused by the wrapper, and the C ABI refuses
    a host pointer among the operands with EPTQ_EINVAL — a persistent launch
    reading one would fault."""
    import ctypes
    from eptq_amd.chain import ChainPlan, ChainStage, _lib_chain
    from eptq_amd.kernels import _lib
    print("chain: host operands refused", flush=True)
    q = E8D4Quantizer(radius=1.75)
    lin = EPTQLinear.from_quantized_data(make_layer(256, 256, seed=3, percmask=0.01), q, "e8_d4")
    for name in ("Q", "g", "h", "O_vals", "O_col", "O_row_ptr"):
        setattr(lin, name, getattr(lin, name).cuda())
    assert lin._codebook.device.type == "cpu"
    with pytest.raises(ValueError, match="_codebook"):
        DecodeChain([dict(layers=[lin], src=-1)])
    lib = _lib_chain()
    la = (_lib.EptqLayer * 1)(_lib.EptqLayer(lin.Q.data_ptr(), lin.g.data_ptr(), lin.h.data_ptr(),
                                             lin.O_vals.data_ptr(), lin.O_col.data_ptr(), lin.O_row_ptr.data_ptr(),
                                             None, None, 0, 32, 0))
    y = torch.empty(256, dtype=torch.float16, device="cuda")
    st = (ChainStage * 1)(ChainStage(1, ctypes.cast(la, ctypes.c_void_p), 256, -1, 0, 256, SLICE, None, 1e-5,
                                     y.data_ptr()))
    nbytes = int(lib.eptq_e8d4_chain_work_bytes(st, 1))
    work = torch.empty(nbytes + 256, dtype=torch.uint8, device="cuda")
    wp = (work.data_ptr() + 255) & ~255
    plan = ChainPlan()
    host_codes = lin._codebook.contiguous()
    s = torch.cuda.current_stream().cuda_stream
    rc = lib.eptq_e8d4_chain_plan(st, 1, host_codes.data_ptr(), wp, nbytes, ctypes.byref(plan), s)
    assert rc == _lib.EPTQ_EINVAL and "device memory" in lib.eptq_last_error().decode()
    dev_codes = host_codes.cuda()
    host_g = lin.g.cpu()
    la[0].g = host_g.data_ptr()
    rc = lib.eptq_e8d4_chain_plan(st, 1, dev_codes.data_ptr(), wp, nbytes, ctypes.byref(plan), s)
    assert rc == _lib.EPTQ_EINVAL and "layer 0" in lib.eptq_last_error().decode()
    la[0].g = lin.g.data_ptr()
    assert lib.eptq_e8d4_chain_plan(st, 1, dev_codes.data_ptr(), wp, nbytes, ctypes.byref(plan), s) == 0
