"""The oracle (and the HIP path) against golden vectors from the reference itself.

``tests/golden/*.npz`` were written by ``tests/golden/make_golden.py`` from the
reference's own ``E8D4Quantizer``/``E8LatticeQuantizer`` tables and
``algorithms/eptq.py:dequantize_layer`` on seeded layers (CPU).  They pin what
no closed form fixes: the order and rounding of the dequantization
(``(v·S)·g·h`` in fp32, then one fp16 rounding), the critical-block overwrite
and the CPU table bits.  The mutation tests show that plausible mistakes in
that order are caught by these fixtures.
"""

from __future__ import annotations

import functools
import hashlib
from pathlib import Path

import numpy as np
import pytest
import torch

from eptq_amd.quantizers import E8D4Quantizer, E8LatticeQuantizer
from oracle.codebooks import e8_raw_points_shells, e8d4_raw_codes_heap, scale_table
from oracle.dequant import (_decode_blocks, dequantize_layer, dequantize_layer_torch_loop,
                            dequantize_scalar)
from oracle.matvec import rel_l2

GOLDEN = Path(__file__).resolve().parent / "golden"
CASES = sorted(p.stem[len("dequant_"):] for p in GOLDEN.glob("dequant_*.npz"))


def load_case(name):
    z = np.load(GOLDEN / f"dequant_{name}.npz")
    d = {k: z[k] for k in z.files}
    d["kind"] = str(d["kind"])
    return d


@functools.lru_cache(maxsize=None)
def _raw(kind):
    return e8d4_raw_codes_heap() if kind == "e8_d4" else e8_raw_points_shells()


def table_for(d):
    r = float(d["chosen_r"]) if "chosen_r" in d else float(d["radius"])
    if d["kind"] == "e8_d4":
        return scale_table(_raw("e8_d4"), r).reshape(512, 4)
    return scale_table(_raw("e8_lattice"), r)


def as_bits(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def test_fixtures_present():
    assert len(CASES) >= 6
    assert (GOLDEN / "e8d4_table_r1.75.npz").exists() and (GOLDEN / "e8_table_r1.6.npz").exists()


def test_e8d4_table_matches_reference():
    ref = np.load(GOLDEN / "e8d4_table_r1.75.npz")["codes"]
    assert np.array_equal(scale_table(_raw("e8_d4"), 1.75), ref)
    assert np.array_equal(E8D4Quantizer(radius=1.75).codes.numpy(), ref)


def test_e8_table_matches_reference():
    z = np.load(GOLDEN / "e8_table_r1.6.npz")
    mine = scale_table(_raw("e8_lattice"), 1.6)
    assert tuple(z["shape"]) == mine.shape
    assert hashlib.sha256(mine.tobytes()).digest() == z["sha256"].tobytes()
    assert np.array_equal(mine[:64], z["head"]) and np.array_equal(mine[-64:], z["tail"])
    assert np.array_equal(mine[z["boundary_index"]], z["boundary_rows"])
    pkg = E8LatticeQuantizer(radius=1.6).flat_table().numpy()
    assert hashlib.sha256(pkg.tobytes()).digest() == z["sha256"].tobytes()


@pytest.mark.parametrize("name", CASES)
def test_oracle_dequant_bit_exact_vs_reference(name):
    d = load_case(name)
    W = dequantize_layer(d["Q"], d["g"], d["h"], d["O"], table_for(d), d["kind"], d.get("S_group"))
    assert np.array_equal(as_bits(W), as_bits(d["W"]))


@pytest.mark.parametrize("name", CASES)
def test_scalar_bruteforce_bit_exact_vs_reference(name):
    d = load_case(name)
    W = dequantize_scalar(d["Q"], d["g"], d["h"], d["O"], table_for(d), d["kind"], d.get("S_group"))
    assert np.array_equal(as_bits(W), as_bits(d["W"]))


@pytest.mark.parametrize("name", CASES)
def test_cpu_baseline_port_bit_exact_vs_reference(name):
    d = load_case(name)
    W = dequantize_layer_torch_loop(d["Q"], d["g"], d["h"], d["O"], table_for(d), d["kind"],
                                    d.get("S_group"))
    assert np.array_equal(as_bits(W.numpy()), as_bits(d["W"]))


# --------------------------------------------------------------------------
# Mutations planted in the oracle: each must disagree with the reference.
# --------------------------------------------------------------------------

def _mutant(d, variant):
    Q = np.asarray(d["Q"], dtype=np.int16)
    M, N = Q.shape
    u = Q.astype(np.int32) + 32768
    mask = u == 65535
    u = np.where(mask, 0, u)
    tab = table_for(d)
    if variant == "swap_halves" and d["kind"] == "e8_d4":
        blk = _decode_blocks(u, tab, "e8_d4")
        blk = np.concatenate([blk[..., 4:], blk[..., :4]], axis=-1)
    else:
        blk = _decode_blocks(u, tab, d["kind"])
    W = np.ascontiguousarray(blk.transpose(0, 2, 1)).reshape(8 * M, N).astype(np.float32)
    S = d.get("S_group")
    if S is not None:
        W = W * np.repeat(S.astype(np.float32), (8 * M) // S.shape[0], axis=0)
    if d["O"].size:
        mi, ni = np.nonzero(mask)
        if variant == "column_major_markers":
            order = np.lexsort((mi, ni))
            mi, ni = mi[order], ni[order]
        Wv = W.reshape(M, 8, N)
        O = d["O"].astype(np.float32)
        if variant == "o_times_s" and S is not None:
            O = O * S.astype(np.float32)[(8 * mi) // ((8 * M) // S.shape[0]), ni][:, None]
        Wv[mi, :, ni] = O
    g = d["g"].astype(np.float32)
    h = d["h"].astype(np.float32)
    if variant == "gh_first":
        W = W * (g[:, None] * h[None, :])
    else:
        W = (W * g[:, None]) * h[None, :]
    return W.astype(np.float16)


@pytest.mark.parametrize("variant,cases", [
    ("gh_first", [c for c in CASES]),
    ("swap_halves", [c for c in CASES if c.startswith("e8d4")]),
    ("column_major_markers", [c for c in CASES]),
    ("o_times_s", [c for c in CASES if "groups" in c]),
])
def test_planted_mistakes_are_caught(variant, cases):
    caught = [not np.array_equal(as_bits(_mutant(load_case(c), variant)), as_bits(load_case(c)["W"]))
              for c in cases]
    assert any(caught), f"mutation {variant} not detected by any golden case"


def test_unmutated_reconstruction_agrees():
    # The mutant builder with no mutation is the oracle itself.
    for c in CASES:
        d = load_case(c)
        assert np.array_equal(as_bits(_mutant(d, "none")), as_bits(d["W"]))


# --------------------------------------------------------------------------
# GPU: the HIP dequant and Linear against the same fixtures.
# --------------------------------------------------------------------------

def _dev_layer(d, dev):
    from tests._util import csr_dev
    Q = torch.from_numpy(d["Q"]).to(dev)
    O_col, O_row_ptr = csr_dev(torch.from_numpy(d["Q"]), dev)
    return dict(Q=Q, g=torch.from_numpy(d["g"]).to(dev), h=torch.from_numpy(d["h"]).to(dev),
                O=torch.from_numpy(d["O"]).to(dev).reshape(-1, 8), O_col=O_col, O_row_ptr=O_row_ptr,
                S=None if "S_group" not in d else torch.from_numpy(d["S_group"]).to(dev))


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
def test_gpu_dequant_bit_exact_vs_reference(name):
    from eptq_amd.kernels import dequant
    d = load_case(name)
    dev = torch.device("cuda:0")
    L = _dev_layer(d, dev)
    tab = torch.from_numpy(table_for(d)).to(dev).contiguous()
    W = dequant(d["kind"], L["Q"], tab, L["g"], L["h"], L["O"], L["O_col"], L["O_row_ptr"], L["S"])
    assert np.array_equal(W.cpu().numpy().view(np.uint16), as_bits(d["W"]))


@pytest.mark.gpu
@pytest.mark.parametrize("name", CASES)
@pytest.mark.parametrize("B", [1, 3, 8, 40])
def test_gpu_linear_vs_reference_weights(name, B):
    from eptq_amd.kernels import linear_forward
    d = load_case(name)
    dev = torch.device("cuda:0")
    L = _dev_layer(d, dev)
    N = d["Q"].shape[1]
    x = torch.from_numpy(np.random.default_rng(B).standard_normal((B, N)).astype(np.float16)).to(dev)
    codes = torch.from_numpy(table_for(d)).half().to(dev)
    y = linear_forward(d["kind"], L["Q"], codes, L["g"], L["h"], x, L["O"], L["O_col"],
                       L["O_row_ptr"], None, L["S"])
    ref = x.cpu().float().numpy() @ d["W"].astype(np.float32).T
    assert rel_l2(y.cpu().float().numpy(), ref) <= 1e-2
