"""GPU: the persistent decode chain (``eptq_e8d4_chain_*``) against the
one-launch-per-stage path.

A chain of decoder stages (q|k|v, o, gate|up, down per transformer layer) in
which every stage reads an earlier stage's output, as a decode step does.
Each stage's output must match the multi-layer launch applied to the same
input (the chain's own input of that stage) within the fp16-accumulation
tolerance, the first stage must match the oracle (fp32 reconstruct +
matmul), repeated runs and HIP-graph replays must reproduce the first run
bit for bit, and no stage wait may time out.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels import DecodeChain, linear_forward_multi
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.dequant import dequantize_layer
from oracle.matvec import rel_l2

pytestmark = pytest.mark.gpu


def _layers(shapes, seed, percmask=0.002, qb=None):
    q = E8D4Quantizer(radius=1.75)
    out = []
    for k, (o, i) in enumerate(shapes):
        lin = EPTQLinear.from_quantized_data(make_layer(o, i, seed=seed + 17 * k, percmask=percmask,
                                                        qb_size=qb), q, "e8_d4").cuda()
        out.append(lin)
    return out


def _ld(lin):
    return dict(Q=lin.Q, g=lin.g, h=lin.h, O_vals=lin.O_vals, O_col=lin.O_col, O_row_ptr=lin.O_row_ptr,
                bias=lin.bias, S_group=lin.S_group)


def _decoder_chain(hidden, ffn, n_layers, heads_kv_dim=None, seed=0, qb=None):
    """Stages of n_layers decoder layers; returns (stages, linears per stage, x0)."""
    kv = hidden if heads_kv_dim is None else heads_kv_dim
    x0 = make_x(1, hidden, seed=seed + 1).cuda()
    stages, lins = [], []
    prev = x0
    for layer in range(n_layers):
        s = seed + 1000 * layer
        for shapes, n_in in ((((hidden, hidden), (kv, hidden), (kv, hidden)), hidden),
                             (((hidden, hidden),), hidden),
                             (((ffn, hidden), (ffn, hidden)), ffn),
                             (((hidden, ffn),), hidden)):
            ls = _layers(shapes, s, qb=qb)
            s += 100
            width = sum(o for o, _ in shapes)
            y = torch.empty((1, width), dtype=torch.float16, device="cuda")
            x = prev[:, :shapes[0][1]]
            stages.append(dict(layers=[_ld(l) for l in ls], x=x, y=y, wait=True))
            lins.append(ls)
            prev = y
            del n_in
    return stages, lins, x0


def _check_stages(stages, lins, tol):
    for i, (S, ls) in enumerate(zip(stages, lins)):
        x = S["x"].contiguous()
        want = linear_forward_multi([_ld(l) for l in ls], ls[0]._codebook, x).float().cpu().numpy()
        got = S["y"].float().cpu().numpy()
        assert np.isfinite(got).all(), f"stage {i}"
        assert rel_l2(got, want) < tol, (i, rel_l2(got, want))


@pytest.mark.parametrize("hidden,ffn,kv,n_layers,qb", [
    (512, 1376, None, 2, None),      # small: every layer fits in one row group per workgroup
    (4096, 11008, None, 1, None),    # Llama-2-7B decoder layer
    (1024, 3584, 256, 2, 128),       # GQA k/v, S_group (Llama-3 style, scaled down)
])
def test_chain_matches_stage_by_stage(hidden, ffn, kv, n_layers, qb):
    print(f"decode chain: hidden={hidden} ffn={ffn} kv={kv} layers={n_layers} qb={qb}", flush=True)
    stages, lins, x0 = _decoder_chain(hidden, ffn, n_layers, heads_kv_dim=kv, seed=hidden + n_layers, qb=qb)
    chain = DecodeChain(stages, lins[0][0]._codebook)
    assert chain.grid >= 256
    chain.run()
    chain.check()
    _check_stages(stages, lins, 2e-3)
    first = [S["y"].clone() for S in stages]
    # The first stage against the oracle.
    l0 = lins[0]
    W = np.concatenate([dequantize_layer(l.Q.cpu().numpy(), l.g.cpu().numpy(), l.h.cpu().numpy(),
                                         l.O_vals.cpu().numpy(), l._table_f32.cpu().numpy(), "e8_d4",
                                         S_group=None if l.S_group is None else l.S_group.cpu().numpy())
                        for l in l0], axis=0).astype(np.float64)
    ref = x0.double().cpu().numpy() @ W.T
    assert rel_l2(stages[0]["y"].double().cpu().numpy(), ref) < 1e-2
    # Repeated runs (the epoch advances) reproduce the first run exactly.
    for _ in range(3):
        for S in stages:
            S["y"].zero_()
        chain.run()
        chain.check()
        for i, S in enumerate(stages):
            assert torch.equal(S["y"], first[i]), f"rerun stage {i}"
    chain.close()


def test_chain_in_a_graph_replays_exactly():
    print("decode chain: HIP graph replays", flush=True)
    stages, lins, x0 = _decoder_chain(1024, 2816, 2, seed=3)
    chain = DecodeChain(stages, lins[0][0]._codebook)
    chain.run()
    chain.check()
    want = [S["y"].clone() for S in stages]
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            chain.run()
    torch.cuda.current_stream().wait_stream(s)
    for rep in range(4):
        for S in stages:
            S["y"].zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        chain.check()
        for i, S in enumerate(stages):
            assert torch.equal(S["y"], want[i]), (rep, i)
        # eager work between replays
        chain.run()
        chain.check()
    chain.close()


def test_chain_new_input_changes_every_stage():
    """The stages really read their predecessors: a new x0 (written in place)
    changes the output of every stage, and matches stage-by-stage again."""
    print("decode chain: new input", flush=True)
    stages, lins, x0 = _decoder_chain(512, 1024, 2, seed=7)
    chain = DecodeChain(stages, lins[0][0]._codebook)
    chain.run()
    chain.check()
    before = [S["y"].clone() for S in stages]
    x0.copy_(make_x(1, 512, seed=99).cuda())
    chain.run()
    chain.check()
    for i, S in enumerate(stages):
        assert not torch.equal(S["y"], before[i]), i
    _check_stages(stages, lins, 2e-3)
    chain.close()
