#!/usr/bin/env python3
"""Write the golden fixtures of this directory from the reference implementation.

Development-container tool (the reference tree is not available where the
tests run).  It imports the reference package read-only from
``$EPTQ_REFERENCE_DIR`` (default ``/root/reference``) under the package name
``eptq`` (its modules use package-relative imports), runs on the CPU, and
stores inputs and outputs as plain ``.npz`` arrays (no pickles):

* ``e8d4_table_r1.75.npz`` — ``E8D4Quantizer(radius=1.75).codes`` (fp32, 4x128x4).
* ``e8_table_r1.6.npz`` — sha256 of ``E8LatticeQuantizer(radius=1.6).points``
  (fp32, 65535x8) plus its first and last 64 rows and the rows around each
  shell boundary.
* ``dequant_<case>.npz`` — a small seeded layer (``Q, g, h, O`` and optional
  ``S_group``, ``chosen_r``) and ``algorithms/eptq.py:dequantize_layer``'s
  fp16 W for it.  These pin the operation order and rounding of the
  reference's dequantization (which no closed form fixes).
* ``loader_<format>.npz`` — a ``quantizer.pt`` of the given on-disk format
  (``warp``: new format with ``warp_alpha`` 1.3; ``old``: a pre-divided table
  whose radius comes from ``quant_config.json``; ``mid``: a pre-divided table
  with ``saved_radius``) loaded by the reference's ``load_quantizer``, then a
  sequence of small layers with assorted ``chosen_r`` dequantized in order by
  its ``dequantize_layer`` with that one quantizer object: the table as loaded,
  the fp32 table each layer was decoded with (recorded inside the reference's
  own ``dequant`` call) and each layer's W.  These pin the warp bits and the
  per-layer radius switches, which rescale a raw-less table in place and drop
  a warp.

Inputs come from ``eptq_amd.synthetic.make_layer`` with fixed seeds.
Usage: ``python tests/golden/make_golden.py``.
"""

from __future__ import annotations

import hashlib
import importlib.util
import os
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parent.parent
sys.path.insert(0, str(REPO))

from eptq_amd.synthetic import make_layer  # noqa: E402

# (name, kind, out, in, seed, percmask, qb_size, chosen_r, g_scale)
CASES = [
    ("e8d4_basic", "e8_d4", 32, 64, 11, 0.05, None, None, 1.0),
    ("e8d4_groups", "e8_d4", 64, 48, 12, 0.04, 16, None, 1.0),
    ("e8d4_chosen_r", "e8_d4", 32, 40, 13, 0.03, None, 1.9, 1.0),
    ("e8d4_tiny_g", "e8_d4", 32, 64, 14, 0.02, None, None, 1e-3),
    ("e8_basic", "e8_lattice", 32, 64, 15, 0.05, None, None, 1.0),
    ("e8_groups", "e8_lattice", 64, 32, 16, 0.05, 32, None, 1.0),
]


# (format, radius on disk, warp_alpha, chosen_r of each layer in load order)
LOADER_CASES = [
    ("warp", 1.75, 1.3, [None, 1.75, 1.9, None, 1.6]),
    ("old", 1.75, 1.0, [1.9, None, 1.6, 1.9, 2.0, None]),
    ("mid", 1.75, 1.0, [None, 1.9, 1.9, 1.75, 2.1]),
]


def loader_case(ref, alg, recon, fmt, radius, alpha, chosen):
    import json
    import tempfile
    raw = ref.E8D4Quantizer(device="cpu", radius=1.0)._raw_codes.float()
    with tempfile.TemporaryDirectory() as d:
        d = Path(d)
        if fmt == "warp":
            data = {"quantizer_type": "e8_d4", "raw_codes": raw, "radius": radius, "warp_alpha": alpha}
        elif fmt == "old":
            data = {"quantizer_type": "e8_d4", "codebook": raw / radius}
            (d / "quant_config.json").write_text(json.dumps({"codebook_radius": radius}))
        else:
            data = {"quantizer_type": "e8_d4", "codebook": raw / 1.875, "saved_radius": radius}
        torch.save(data, d / "quantizer.pt")
        q = recon.load_quantizer(d, device="cpu")
    loaded = q.codes.float().clone().numpy()
    seen = []
    orig = type(q).dequant

    def spy(self, *a, **k):
        if not seen or seen[-1][0] != len(Ws):
            seen.append((len(Ws), self.codes.float().clone().numpy()))
        return orig(self, *a, **k)

    Ws, layers = [], []
    type(q).dequant = spy
    try:
        for i, cr in enumerate(chosen):
            qd = make_layer(16, 24, seed=40 + i, percmask=0.05, chosen_r=cr)
            rqd = ref.QuantizedLayerData(Q=qd.Q.clone(), g=qd.g.clone(), h=qd.h.clone(), O=qd.O.clone(),
                                         bias=None, chosen_r=cr, S_group=None)
            Ws.append(alg.dequantize_layer(rqd, q).numpy())
            layers.append(qd)
    finally:
        type(q).dequant = orig
    arrays = dict(format=np.asarray(fmt), radius=np.float64(radius), warp_alpha=np.float64(alpha),
                  chosen_r=np.asarray([np.nan if c is None else c for c in chosen], dtype=np.float64),
                  loaded=loaded, tables=np.stack([s[1] for s in seen]), W=np.stack(Ws),
                  Q=np.stack([l.Q.numpy() for l in layers]), g=np.stack([l.g.numpy() for l in layers]),
                  h=np.stack([l.h.numpy() for l in layers]))
    # Layers differ in their critical-block count: O is stored flat with offsets.
    arrays["O"] = np.concatenate([l.O.numpy() for l in layers])
    arrays["O_off"] = np.cumsum([0] + [int(l.O.shape[0]) for l in layers])
    np.savez(HERE / f"loader_{fmt}.npz", **arrays)
    print(f"loader_{fmt}: {len(chosen)} layers")


def import_reference(ref_dir: Path):
    spec = importlib.util.spec_from_file_location(
        "eptq", ref_dir / "__init__.py", submodule_search_locations=[str(ref_dir)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules["eptq"] = mod
    spec.loader.exec_module(mod)
    import eptq.algorithms.eptq as alg  # noqa: E402
    return mod, alg


def main() -> None:
    ref_dir = Path(os.environ.get("EPTQ_REFERENCE_DIR", "/root/reference"))
    ref, alg = import_reference(ref_dir)
    import eptq.reconstruct as recon  # noqa: E402

    for case in LOADER_CASES:
        loader_case(ref, alg, recon, *case)

    d4 = ref.E8D4Quantizer(device="cpu", radius=1.75)
    np.savez(HERE / "e8d4_table_r1.75.npz", codes=d4.codes.float().numpy())

    e8 = ref.E8LatticeQuantizer(device="cpu", radius=1.6)
    e8.remove_last()          # quantize.py:178-181 drops the last of 65,536 points
    pts = e8.points.float().contiguous().numpy()
    sizes = [1, 240, 2160, 6720, 17520, 30240]
    bounds = np.cumsum(sizes)
    near = np.unique(np.concatenate([np.arange(b - 2, b + 2) for b in bounds]))
    np.savez(HERE / "e8_table_r1.6.npz",
             sha256=np.frombuffer(hashlib.sha256(pts.tobytes()).digest(), dtype=np.uint8),
             shape=np.asarray(pts.shape), head=pts[:64], tail=pts[-64:],
             boundary_index=near, boundary_rows=pts[near])

    for name, kind, out, inp, seed, p, qb, chosen_r, g_scale in CASES:
        qd = make_layer(out, inp, seed=seed, percmask=p, qb_size=qb, chosen_r=chosen_r)
        if g_scale != 1.0:
            qd.g = (qd.g.float() * g_scale).half()
        rq = ref.E8D4Quantizer(device="cpu", radius=1.75) if kind == "e8_d4" else \
            ref.E8LatticeQuantizer(device="cpu", radius=1.6)
        if kind == "e8_lattice":
            rq.remove_last()
        rqd = ref.QuantizedLayerData(Q=qd.Q.clone(), g=qd.g.clone(), h=qd.h.clone(), O=qd.O.clone(),
                                     bias=None, chosen_r=chosen_r,
                                     S_group=None if qd.S_group is None else qd.S_group.clone())
        W = alg.dequantize_layer(rqd, rq)
        arrays = dict(Q=qd.Q.numpy(), g=qd.g.numpy(), h=qd.h.numpy(), O=qd.O.numpy(),
                      W=W.numpy(), radius=np.float64(1.75 if kind == "e8_d4" else 1.6))
        if qd.S_group is not None:
            arrays["S_group"] = qd.S_group.numpy()
        if chosen_r is not None:
            arrays["chosen_r"] = np.float64(chosen_r)
        np.savez(HERE / f"dequant_{name}.npz", kind=np.asarray(kind), **arrays)
        print(f"{name}: W {tuple(W.shape)} nnz {qd.O.shape[0]}")


if __name__ == "__main__":
    main()
