"""The drop-in module's split-K workspace per (device, stream).

``EPTQLinear`` / ``EPTQMultiLinear`` without an attached workspace use the
current stream's own (``stream_workspace``), so batches of 5..128 rows take
the split-K form of the matrix-core decode.  Checks: one workspace per
stream (the same tensor on repeated calls, different tensors on different
streams), module calls interleaved on two streams stay within the 1e-2
relative-L2 bar of the fp32 oracle and are bit-identical to the same calls
made one stream at a time, and repeats are bit-identical.
"""

import pytest
import torch

from eptq_amd.kernels import stream_workspace
from eptq_amd.kernels.linear import EPTQLinear, EPTQMultiLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.synthetic import make_layer, make_x
from oracle.matvec import linear_ref, rel_l2

from _util import layer_np, table

pytestmark = pytest.mark.gpu

TOL = 1e-2


def test_one_workspace_per_stream():
    print("stream_workspace: identity per stream", flush=True)
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    with torch.cuda.stream(s1):
        a = stream_workspace("cuda")
        a2 = stream_workspace("cuda")
    with torch.cuda.stream(s2):
        b = stream_workspace("cuda")
    assert a is a2 and a.data_ptr() != b.data_ptr()
    torch.cuda.synchronize()
    assert int(a.count_nonzero()) == 0 and int(b.count_nonzero()) == 0


@pytest.mark.parametrize("B", [8, 16, 40])
def test_modules_on_two_streams(B):
    print(f"two streams, B={B}: 1024x2048 and q|k|v 1024+256+256 x 2048", flush=True)
    q = E8D4Quantizer(radius=1.75)
    qa = make_layer(1024, 2048, seed=51, percmask=0.002, bias=True)
    qkv = [make_layer(o, 2048, seed=60 + k, percmask=0.002) for k, o in enumerate((1024, 256, 256))]
    ma = EPTQLinear.from_quantized_data(qa, q, "e8_d4").cuda()
    mb = EPTQMultiLinear([EPTQLinear.from_quantized_data(d, q, "e8_d4").cuda() for d in qkv])
    xa = make_x(B, 2048, seed=70).cuda()
    xb = make_x(B, 2048, seed=71).cuda()
    with torch.no_grad():
        ya0 = ma(xa)
        yb0 = mb(xb)
    torch.cuda.synchronize()
    ref_a = linear_ref(xa.float().cpu().numpy(), *(layer_np(qa)[k] for k in ("Q", "g", "h", "O")),
                       table("e8_d4", 1.75), "e8_d4", layer_np(qa)["bias"])
    assert rel_l2(ya0.float().cpu().numpy(), ref_a) <= TOL
    import numpy as np
    ref_b = np.concatenate([linear_ref(xb.float().cpu().numpy(), n["Q"], n["g"], n["h"], n["O"],
                                       table("e8_d4", 1.75), "e8_d4") for n in map(layer_np, qkv)], axis=1)
    assert rel_l2(yb0.float().cpu().numpy(), ref_b) <= TOL
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    s1.wait_stream(torch.cuda.current_stream())
    s2.wait_stream(torch.cuda.current_stream())
    outs = []
    with torch.no_grad():
        for _ in range(20):
            with torch.cuda.stream(s1):
                ya = ma(xa)
            with torch.cuda.stream(s2):
                yb = mb(xb)
            outs.append((ya, yb))
    torch.cuda.synchronize()
    for ya, yb in outs:
        assert torch.equal(ya, ya0) and torch.equal(yb, yb0)
