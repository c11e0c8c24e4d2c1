"""Oracle dequantizer: ``dequantize_layer`` (``algorithms/eptq.py:406-471``) on the CPU.

Test infrastructure only (see ``oracle/__init__.py``).

Definition restated (per element, all arithmetic IEEE fp32, RNE):

1. ``u = Q + 32768``; ``u == 65535`` marks a critical block; those are decoded
   as index 0 and later overwritten (``:421-427``).
2. ``v = table(u)`` — E8-D4: rows 0..3 ``codes[t, i]``, rows 4..7
   ``codes[t, j]`` (``quantizers/e8_d4.py:237-255``); E8: ``points[u]``.
3. With ``S_group`` (n_groups, N): ``v *= fp32(S[row // qb, n])`` where
   ``qb = out_features // n_groups`` (``:440-449``).
4. Critical blocks: ``v[8m:8m+8, n] = fp32(O[i])`` with ``i`` the row-major
   rank of (m, n) among the markers; O is not multiplied by S (``:461-466``).
5. ``W = (v · fp32(g)[:, None]) · fp32(h)[None, :]`` then ``.half()`` (``:469-471``).
"""

from __future__ import annotations

import numpy as np


def _decode_blocks(u: np.ndarray, table: np.ndarray, kind: str) -> np.ndarray:
    """(M, N) indices -> (M, N, 8) fp32 block vectors."""
    if kind == "e8_d4":
        t = table.reshape(512, 4)
        a1 = t[(((u >> 14) & 3) << 7) | ((u >> 7) & 127)]
        a2 = t[(((u >> 14) & 3) << 7) | (u & 127)]
        return np.concatenate([a1, a2], axis=-1)
    if kind == "e8_lattice":
        return table.reshape(-1, 8)[u]
    raise ValueError(kind)


def dequantize_layer(Q, g, h, O, table, kind, S_group=None) -> np.ndarray:
    """fp16 W of shape (8M, N), bit-exact definition (vectorized restatement)."""
    Q = np.asarray(Q, dtype=np.int16)
    M, N = Q.shape
    u = Q.astype(np.int32) + 32768
    mask = u == 65535
    u = np.where(mask, 0, u)
    blk = _decode_blocks(u, np.asarray(table, dtype=np.float32), kind)   # (M, N, 8)
    W = np.ascontiguousarray(blk.transpose(0, 2, 1)).reshape(8 * M, N)
    if S_group is not None:
        S = np.asarray(S_group).astype(np.float32)
        qb = (8 * M) // S.shape[0]
        W = (W * np.repeat(S, qb, axis=0)).astype(np.float32)
    O = np.asarray(O)
    if O.size > 0:
        mi, ni = np.nonzero(mask)          # row-major order
        Wv = W.reshape(M, 8, N)
        Wv[mi, :, ni] = O.astype(np.float32)
    gf = np.asarray(g).astype(np.float32)
    hf = np.asarray(h).astype(np.float32)
    W = (W * gf[:, None]).astype(np.float32)
    W = (W * hf[None, :]).astype(np.float32)
    return W.astype(np.float16)


def dequantize_scalar(Q, g, h, O, table, kind, S_group=None) -> np.ndarray:
    """Element-by-element brute force of the same definition (tiny inputs only)."""
    Q = np.asarray(Q, dtype=np.int16)
    M, N = Q.shape
    tab = np.asarray(table, dtype=np.float32)
    tab = tab.reshape(512, 4) if kind == "e8_d4" else tab.reshape(-1, 8)
    out = np.zeros((8 * M, N), dtype=np.float16)
    rank = 0
    o_of = {}
    for m in range(M):
        for n in range(N):
            if int(Q[m, n]) + 32768 == 65535:
                o_of[(m, n)] = rank
                rank += 1
    qb = None
    if S_group is not None:
        qb = (8 * M) // np.asarray(S_group).shape[0]
    for m in range(M):
        for n in range(N):
            u = int(Q[m, n]) + 32768
            for k in range(8):
                row = 8 * m + k
                if (m, n) in o_of:
                    v = np.float32(np.asarray(O)[o_of[(m, n)], k])
                else:
                    if kind == "e8_d4":
                        t, i, j = (u >> 14) & 3, (u >> 7) & 127, u & 127
                        v = tab[t * 128 + (i if k < 4 else j), k % 4]
                    else:
                        v = tab[u, k]
                    if qb is not None:
                        v = np.float32(v * np.float32(np.asarray(S_group)[row // qb, n]))
                w = np.float32(np.float32(v * np.float32(np.asarray(g)[row])) * np.float32(np.asarray(h)[n]))
                out[row, n] = np.float16(w)
    return out


def build_csr(Q):
    """CSR of the critical blocks, as ``kernels/linear.py:122-139`` builds it:
    ``O_col`` (nnz,) int32 in row-major marker order, ``O_row_ptr`` (M+1,) int32."""
    Q = np.asarray(Q, dtype=np.int16)
    M = Q.shape[0]
    rows, cols = np.nonzero(Q == 32767)
    counts = np.bincount(rows, minlength=M)
    row_ptr = np.concatenate([[0], np.cumsum(counts)]).astype(np.int32)
    return cols.astype(np.int32), row_ptr


def dequantize_layer_torch_loop(Q, g, h, O, table, kind, S_group=None):
    """The reference's CPU data flow, restated with torch on the CPU: the
    per-column Python loop of ``algorithms/eptq.py:440-453`` (one advanced-index
    decode per column), the row-major ``nonzero`` overwrite and the fp32 scale.
    Used as the timed CPU baseline (kind "port"); same bits as
    :func:`dequantize_layer`."""
    import torch
    Qt = torch.as_tensor(np.asarray(Q)).int() + 32768
    mask = Qt == 65535
    Qt[mask] = 0
    tab = torch.as_tensor(np.asarray(table, dtype=np.float32))
    if kind == "e8_d4":
        codes = tab.reshape(4, 128, 4)

        def dq(col):
            t = (col >> 14) & 3
            i = (col >> 7) & 0x7F
            j = col & 0x7F
            a1 = codes[t.T, i.T]
            a2 = codes[t.T, j.T]
            return torch.stack((a1, a2), dim=-2).reshape(j.shape[-1], -1).T * 1.0
    else:
        pts = tab.reshape(-1, 8)

        def dq(col):
            return pts[col.T.long()].reshape(col.shape[1], -1).T * 1.0
    out_features = Qt.shape[0] * 8
    N = Qt.shape[1]
    W = torch.zeros((out_features, N), dtype=torch.float32)
    if S_group is not None:
        S = torch.as_tensor(np.asarray(S_group)).float()
        qb = out_features // S.shape[0]
        for j in range(N):
            W[:, j:j + 1] = dq(Qt[:, j:j + 1]) * S[:, j].repeat_interleave(qb).unsqueeze(1)
    else:
        for j in range(N):
            W[:, j:j + 1] = dq(Qt[:, j:j + 1])
    Wv = W.view(-1, 8, N)
    Ot = torch.as_tensor(np.asarray(O))
    if Ot.numel() > 0:
        i0, i1 = mask.nonzero(as_tuple=True)
        Wv[i0, :, i1] = Ot.float()
    W = W * torch.as_tensor(np.asarray(g)).float()[:, None] * torch.as_tensor(np.asarray(h)).float()[None, :]
    return W.half()
