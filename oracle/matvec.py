"""Oracle for the fused quantized Linear: y = x · Wᵀ + bias.

Test infrastructure only (see ``oracle/__init__.py``).

* :func:`linear_ref` — the north-star reference: the oracle's bit-exact fp16 W
  (``algorithms/eptq.py:406-471``), then an fp32 matmul and bias
  (``benchmark_inference.py:82-85`` with fp32 accumulation).
* :func:`fused_ref64` — the fused math of ``test_e8_cuda.py:23-53`` /
  ``csrc/eptq_kernels.cu:196-290`` in float64 without rounding W to fp16:
  ``y[b, 8m+k] = g·(Σ_n v_k(m,n)·h_n·x_bn + Σ_CSR O_k·h_c·x_bc) + bias``.
* :func:`rel_l2` — the acceptance metric (≤ 1e-2).
"""

from __future__ import annotations

import numpy as np

from .dequant import _decode_blocks, dequantize_layer


def linear_ref(x, Q, g, h, O, table, kind, bias=None, S_group=None) -> np.ndarray:
    """fp32 reconstruct + matmul: (B, N) x -> (B, 8M) float32."""
    W = dequantize_layer(Q, g, h, O, table, kind, S_group).astype(np.float32)
    y = np.asarray(x).astype(np.float32) @ W.T
    if bias is not None and np.asarray(bias).size > 0:
        y = y + np.asarray(bias).astype(np.float32)[None, :]
    return y.astype(np.float32)


def fused_ref64(x, Q, g, h, O, table, kind, bias=None, S_group=None) -> np.ndarray:
    """float64 evaluation of the fused decode math (no fp16 rounding of W)."""
    Q = np.asarray(Q, dtype=np.int16)
    M, N = Q.shape
    u = Q.astype(np.int32) + 32768
    mask = u == 65535
    blk = _decode_blocks(np.where(mask, 0, u), np.asarray(table, dtype=np.float32), kind)
    blk = blk.astype(np.float64)
    blk[mask] = 0.0
    V = blk.transpose(0, 2, 1).reshape(8 * M, N)
    if S_group is not None:
        S = np.asarray(S_group).astype(np.float64)
        V = V * np.repeat(S, (8 * M) // S.shape[0], axis=0)
    O = np.asarray(O).astype(np.float64)
    if O.size > 0:
        mi, ni = np.nonzero(mask)
        Vv = V.reshape(M, 8, N)
        Vv[mi, :, ni] = O
    xh = np.asarray(x).astype(np.float64) * np.asarray(h).astype(np.float64)[None, :]
    y = (xh @ V.T) * np.asarray(g).astype(np.float64)[None, :]
    if bias is not None and np.asarray(bias).size > 0:
        y = y + np.asarray(bias).astype(np.float64)[None, :]
    return y


def rel_l2(y, ref) -> float:
    y = np.asarray(y, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    den = np.linalg.norm(ref)
    return float(np.linalg.norm(y - ref) / (den if den > 0 else 1.0))
