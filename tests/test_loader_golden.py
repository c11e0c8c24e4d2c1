"""CPU: the loader's per-layer tables against the reference's own loader.

``tests/golden/loader_<format>.npz`` hold what the reference's
``load_quantizer`` (``reconstruct.py:39-90``) and ``dequantize_layer``
(``algorithms/eptq.py:406-471``) produced for a ``quantizer.pt`` of each
on-disk format and a sequence of layers with assorted ``chosen_r``, decoded in
order with one quantizer object: the table as loaded, the fp32 table each
layer was decoded with, and each layer's fp16 W.  Building ``EPTQLinear``
layers in the same order must give the same tables bit for bit (the radius
switches rescale a raw-less table in place and drop a warp, and earlier
layers' tables must not change afterwards), and the oracle's dequantization
with those tables must give the reference's W.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from eptq_amd.config import QuantizedLayerData
from eptq_amd.kernels.linear import EPTQLinear
from eptq_amd.quantizers import E8D4Quantizer
from eptq_amd.quantizers.e8_d4 import e8d4_raw_codes
from eptq_amd.reconstruct import load_quantizer
from oracle.dequant import dequantize_layer

GOLDEN = Path(__file__).resolve().parent / "golden"


def _write_quantizer(d: Path, fmt: str, radius: float, alpha: float) -> None:
    """The quantizer.pt the golden file was made from (same bytes of table)."""
    raw = torch.from_numpy(e8d4_raw_codes())
    if fmt == "warp":
        data = {"quantizer_type": "e8_d4", "raw_codes": raw, "radius": radius, "warp_alpha": alpha}
    elif fmt == "old":
        data = {"quantizer_type": "e8_d4", "codebook": raw / radius}
        (d / "quant_config.json").write_text(json.dumps({"codebook_radius": radius}))
    else:
        data = {"quantizer_type": "e8_d4", "codebook": raw / 1.875, "saved_radius": radius}
    torch.save(data, d / "quantizer.pt")


def _layers(z):
    out = []
    for i, cr in enumerate(z["chosen_r"]):
        O = z["O"][z["O_off"][i]:z["O_off"][i + 1]]
        out.append(QuantizedLayerData(Q=torch.from_numpy(z["Q"][i]), g=torch.from_numpy(z["g"][i]),
                                      h=torch.from_numpy(z["h"][i]), O=torch.from_numpy(O),
                                      chosen_r=None if np.isnan(cr) else float(cr)))
    return out


@pytest.mark.parametrize("fmt", ["warp", "old", "mid"])
def test_layer_tables_match_reference_loader(tmp_path, fmt):
    z = np.load(GOLDEN / f"loader_{fmt}.npz")
    _write_quantizer(tmp_path, fmt, float(z["radius"]), float(z["warp_alpha"]))
    q = load_quantizer(tmp_path, device="cpu")
    assert np.array_equal(q.codes.numpy().view(np.uint32), z["loaded"].view(np.uint32))
    lins = []
    for i, qd in enumerate(_layers(z)):
        lin = EPTQLinear.from_quantized_data(qd, q, "e8_d4")
        lins.append(lin)
        want = z["tables"][i].reshape(512, 4)
        assert np.array_equal(lin._table_f32.numpy().view(np.uint32), want.view(np.uint32)), f"layer {i}"
        assert torch.equal(lin._codebook, lin._table_f32.half())
        W = dequantize_layer(qd.Q.numpy(), qd.g.numpy(), qd.h.numpy(), qd.O.numpy(), lin._table_f32.numpy(),
                             "e8_d4")
        assert np.array_equal(W.view(np.uint16), z["W"][i].view(np.uint16)), f"layer {i}"
    # Loading later layers leaves every earlier layer's table as it was.
    for i, lin in enumerate(lins):
        assert np.array_equal(lin._table_f32.numpy().view(np.uint32),
                              z["tables"][i].reshape(512, 4).view(np.uint32)), f"layer {i} changed"


def test_legacy_tables_survive_later_loads():
    """A raw-less table rescaled in place by later layers' chosen_r: the
    tables already handed to layers are private copies."""
    raw = torch.from_numpy(e8d4_raw_codes())
    q = E8D4Quantizer(codebook=(raw / 1.75).clone())
    q._radius = 1.75
    first = EPTQLinear.from_quantized_data(
        QuantizedLayerData(Q=torch.zeros(2, 8, dtype=torch.int16), g=torch.ones(16, dtype=torch.float16),
                           h=torch.ones(8, dtype=torch.float16), O=torch.zeros(0, 8, dtype=torch.float16)),
        q, "e8_d4")
    snap = first._table_f32.clone()
    for cr in (1.9, 1.6, 2.0, 1.7, 1.95):
        EPTQLinear.from_quantized_data(
            QuantizedLayerData(Q=torch.zeros(2, 8, dtype=torch.int16), g=torch.ones(16, dtype=torch.float16),
                               h=torch.ones(8, dtype=torch.float16), O=torch.zeros(0, 8, dtype=torch.float16),
                               chosen_r=cr), q, "e8_d4")
    assert torch.equal(first._table_f32, snap)
    assert first._table_f32.data_ptr() != q.codes.data_ptr()


def test_warp_properties():
    """warp_codebook(α) (quantizers/e8_d4.py:282-298): directions kept, the
    largest point fixed, every norm mapped to (‖c‖/max)^α·max."""
    for alpha in (0.7, 1.3, 2.0):
        q = E8D4Quantizer(radius=1.75)
        before = q.codes.reshape(-1, 4).double()
        q.warp_codebook(alpha)
        after = q.codes.reshape(-1, 4).double()
        nb, na = before.norm(dim=1), after.norm(dim=1)
        mx = nb.max()
        nz = nb > 1e-8
        assert torch.all(na[~nz] == 0)
        cos = (before[nz] * after[nz]).sum(1) / (nb[nz] * na[nz])
        assert torch.all(cos > 1 - 1e-6)
        want = (nb[nz] / mx) ** alpha * mx
        assert torch.allclose(na[nz], want, rtol=1e-5)
        top = int(torch.argmax(nb))
        assert torch.allclose(after[top], before[top], rtol=1e-6)
