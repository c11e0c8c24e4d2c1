"""Oracle of one stage of a batch-1 Linear chain (``include/eptq_chain.h``).

Test infrastructure only (see ``oracle/__init__.py``).  The chain has no
counterpart in the reference; each stage is the reference's quantized Linear
(``linear_ref``: ``dequantize_layer`` W, ``algorithms/eptq.py:406-471``, then an
fp32 product) applied to an input formed from an earlier stage's output:

* SLICE:  in = src[src_col : src_col + N]
* SWIGLU: in = fp16(silu(a) * b), a = src[src_col : +N], b = src[src_col + N : +N],
  silu and the product in float32 (the roundings of a separate SiLU-multiply
  kernel: an fp32 product, then fp16);
* with an RMSNorm weight w: in <- in * w / sqrt(mean(in^2) + eps), in float64
  (the chain applies the scalar to the fp32 sums of the Linear).

Pinned by known answers in ``tests/test_oracle_chain.py`` (SwiGLU of zero
gates is zero, of large gates is the up values; the RMSNorm of a constant
vector is w; slices are identity) and by ``linear_ref``'s own pinning.
"""

from __future__ import annotations

import numpy as np

from .matvec import linear_ref

SLICE, SWIGLU = 0, 1


def stage_input(src, src_col: int, N: int, act: int, norm_weight=None, eps: float = 1e-5) -> np.ndarray:
    """(N,) float64 input of a stage from its source vector ``src`` (fp16)."""
    src = np.asarray(src, dtype=np.float16)
    a = src[src_col:src_col + N].astype(np.float32)
    if act == SWIGLU:
        b = src[src_col + N:src_col + 2 * N].astype(np.float32)
        x = (a / (np.float32(1.0) + np.exp(-a)) * b).astype(np.float32).astype(np.float16)
    else:
        x = a
    x = np.asarray(x, dtype=np.float64)
    if norm_weight is not None:
        w = np.asarray(norm_weight, dtype=np.float16).astype(np.float64)
        x = x * w / np.sqrt(np.mean(x * x) + eps)
    return x


def stage_ref(x, layers, table) -> np.ndarray:
    """Stage outputs side by side: each layer's ``linear_ref`` on ``x``
    (``layers``: dicts of numpy Q, g, h, O and optional bias)."""
    x = np.asarray(x, dtype=np.float64)[None, :]
    return np.concatenate([linear_ref(x, L["Q"], L["g"], L["h"], L["O"], table, "e8_d4", L.get("bias"))[0]
                           for L in layers])
