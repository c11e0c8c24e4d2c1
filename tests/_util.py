"""Shared helpers for the test-suite: seeded layers as numpy + torch views."""

import numpy as np
import torch

from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from eptq_amd.synthetic import make_layer, make_x

_TABLES = {}


def table(kind, radius):
    key = (kind, radius)
    if key not in _TABLES:
        q = E8D4Quantizer(radius=radius) if kind == "e8_d4" else E8LatticeQuantizer(radius=radius)
        _TABLES[key] = q.flat_table().numpy()
    return _TABLES[key]


def layer_np(qd):
    """QuantizedLayerData -> dict of numpy arrays (oracle inputs)."""
    return dict(Q=qd.Q.numpy(), g=qd.g.numpy(), h=qd.h.numpy(), O=qd.O.numpy(),
                S_group=None if qd.S_group is None else qd.S_group.numpy(),
                bias=None if qd.bias is None else qd.bias.numpy())


def csr_dev(Q, device="cuda"):
    mask = Q == 32767
    rows, cols = mask.nonzero(as_tuple=True)
    counts = torch.bincount(rows, minlength=Q.shape[0])
    rp = torch.cat([torch.zeros(1, dtype=torch.int32), counts.cumsum(0).to(torch.int32)])
    return cols.to(torch.int32).to(device), rp.to(device)
