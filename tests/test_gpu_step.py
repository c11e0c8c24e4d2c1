"""GPU parity of the batch-1 decode-step engine (``eptq_step_*``): one
persistent launch running dependent E8-D4 stages.

Each stage's output is checked against the fp32 reconstruct + matmul oracle
applied to the stage's actual input (the engine's own fp16 output of the
stage it reads, RMSNorm'd where the stage asks for it), within 1e-2 relative
L2, and against the single-launch multi-layer kernel on the same input.  The
chain covers multi-layer stages (q|k|v-like widths), RMSNorm inputs, a column
offset, an input width whose last 64-chunk segment is partial, rows with more
than 64 critical blocks, a stage with fewer rows than compute units, and a
stage with several rows per compute unit.  Reruns and HIP-graph replays give
bit-identical outputs, every output word carries the run's flag, and the
plain copy equals the flagged output.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from eptq_amd.kernels import DecodeStep, linear_forward_multi
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def _lin(out, inp, seed, p=0.002, bias=False):
    q = E8D4Quantizer(radius=1.75)
    qd = make_layer(out, inp, seed=seed, percmask=p, bias=bias)
    return EPTQLinear.from_quantized_data(qd, q, "e8_d4").cuda(), qd


def _layer_dict(l):
    return dict(Q=l.Q, g=l.g, h=l.h, O_vals=l.O_vals, O_col=l.O_col, O_row_ptr=l.O_row_ptr, bias=l.bias)


def _rmsnorm16(x16, w16, eps):
    xf = x16.float()
    inv = torch.rsqrt(xf.pow(2).mean() + eps)
    return (xf * inv * w16.float()).half()


def make_chain():
    torch.manual_seed(0)
    L = {}
    # name: (out, in, seed, percmask, bias)
    specs = {
        "q": (512, 512, 1, 0.002, False), "k": (256, 512, 2, 0.002, False), "v": (256, 512, 3, 0.002, True),
        "o": (512, 512, 4, 0.002, False),
        "gate": (4096, 512, 5, 0.002, False), "up": (4096, 512, 6, 0.002, False),
        "down": (512, 4096, 7, 0.002, False),
        "odd": (1024, 776, 8, 0.002, True),      # 97 chunks: one full and one partial segment
        "dense": (64, 512, 9, 0.15, False),       # ~77 critical blocks per row, 8 rows in all
    }
    for name, (o, i, sd, p, b) in specs.items():
        L[name] = _lin(o, i, sd, p, b)
    x0 = make_x(1, 512, seed=10).cuda()
    nw1 = (1.0 + 0.1 * torch.randn(512)).half().cuda()
    nw2 = (1.0 + 0.1 * torch.randn(512)).half().cuda()
    y_last = torch.empty((1, 64), dtype=torch.float16, device="cuda")
    stages = [
        dict(layers=[L["q"][0], L["k"][0], L["v"][0]], N=512, x=x0, norm_w=nw1, eps=1e-5),   # 0
        dict(layers=[L["o"][0]], N=512, src=0, col=0),                                      # 1
        dict(layers=[L["gate"][0], L["up"][0]], N=512, src=1, col=0, norm_w=nw2, eps=1e-5),  # 2
        dict(layers=[L["down"][0]], N=4096, src=2, col=4096),                               # 3 (the up half)
        dict(layers=[L["odd"][0]], N=776, src=2, col=8),                                    # 4
        dict(layers=[L["dense"][0]], N=512, src=3, col=0, y=y_last),                        # 5
    ]
    for S in stages:
        S["layers"] = [_layer_dict(l) for l in S["layers"]]
    codes = L["q"][0]._codebook
    plan = DecodeStep(stages, codes)
    return plan, stages, L, x0


@pytest.fixture(scope="module")
def chain():
    return make_chain()


def _check_stage(plan, stages, s, L):
    S = stages[s]
    if S.get("src", -1) < 0:
        x = S["x"]
    else:
        x = plan.output(S["src"])[:, S["col"]:S["col"] + S["N"]].contiguous()
    if S.get("norm_w") is not None:
        x = _rmsnorm16(x, S["norm_w"], S["eps"])
    got = plan.output(s).float().cpu().numpy()
    # Single-launch kernel on the same input.
    codes = plan._codes
    same = linear_forward_multi(S["layers"], codes, x).float().cpu().numpy()
    # fp32 oracle per layer.
    refs = []
    for Ld in S["layers"]:
        Q = Ld["Q"].cpu().numpy()
        refs.append(linear_ref(x.float().cpu().numpy(), Q, Ld["g"].cpu().numpy(), Ld["h"].cpu().numpy(),
                               Ld["O_vals"].cpu().numpy(), table("e8_d4", 1.75), "e8_d4",
                               None if Ld["bias"] is None else Ld["bias"].cpu().numpy()))
    ref = np.concatenate(refs, axis=1)
    e_ref, e_same = rel_l2(got, ref), rel_l2(got, same)
    print(f"  stage {s}: rel_l2 vs oracle {e_ref:.2e}, vs single-launch kernel {e_same:.2e}", flush=True)
    assert np.isfinite(got).all()
    assert e_ref <= TOL and e_same <= 2e-3, s


def test_step_chain_matches_oracle(chain):
    plan, stages, L, _ = chain
    print("decode-step engine: 6-stage chain", flush=True)
    plan.run()
    plan.status()
    for s in range(len(stages)):
        _check_stage(plan, stages, s, L)
    # The plain copy equals the flagged output; flags are the run's.
    assert torch.equal(stages[5]["y"], plan.output(5).cuda())
    for s in range(len(stages)):
        f = plan.flags(s)
        assert bool((f == f[0]).all()) and int(f[0]) != 0


def test_step_reruns_and_graph_replays_bit_identical(chain):
    plan, stages, L, x0 = chain
    print("decode-step engine: reruns and graph replays", flush=True)
    plan.run()
    plan.status()
    first = [plan.output(s) for s in range(len(stages))]
    f0 = int(plan.flags(0)[0])
    plan.run()
    plan.status()
    assert int(plan.flags(0)[0]) == f0 + 1024
    for s in range(len(stages)):
        assert torch.equal(plan.output(s), first[s]), s
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        plan.run()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    with torch.cuda.graph(g):
        plan.run()
    for r in range(3):
        g.replay()
        torch.cuda.synchronize()
        _ = torch.randn(1000, device="cuda").sum()   # unrelated eager work between replays
        for s in range(len(stages)):
            assert torch.equal(plan.output(s), first[s]), (r, s)
    plan.status()
    del g


def test_step_input_change_propagates(chain):
    """A new plain input gives the outputs of the new input (the plan reads x
    at run time, not at init)."""
    plan, stages, L, x0 = chain
    print("decode-step engine: new input", flush=True)
    saved = x0.clone()
    x0.copy_(make_x(1, 512, seed=77).cuda())
    plan.run()
    plan.status()
    for s in range(len(stages)):
        _check_stage(plan, stages, s, L)
    x0.copy_(saved)


def test_step_rejects_bad_plans():
    from eptq_amd.kernels import EptqError
    l, _ = _lin(256, 512, 20)
    d = _layer_dict(l)
    x = make_x(1, 512, seed=1).cuda()
    codes = l._codebook
    bad = [
        [dict(layers=[d] * 4, N=512, x=x)],                              # four layers
        [dict(layers=[d], N=512, src=0, col=0)],                         # reads itself
        [dict(layers=[d], N=512, x=x), dict(layers=[d], N=512, src=0, col=2)],   # col not a multiple of 4
        [dict(layers=[d], N=512, x=x), dict(layers=[d], N=512, src=0, col=1800)],  # past the output
    ]
    for stages in bad:
        with pytest.raises(EptqError):
            DecodeStep(stages, codes)
