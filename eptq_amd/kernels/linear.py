"""``EPTQLinear`` (alias ``QuantizedLinear``): a quantized ``nn.Linear`` on gfx950 kernels.

Drop-in for the reference's ``kernels/linear.py:20-219``: same constructor
signature, same ``from_quantized_data(quant_data, codebook, quantizer_type)``,
same buffer names (``Q, g, h, O_vals, O_col, O_row_ptr, bias``), the same
shared non-buffer codebook moved by ``_apply``, and ``forward`` mapping
(..., in) -> (..., out) in the input dtype.

Differences, all towards the reference's own reconstruct semantics:

* ``codebook`` may be a loaded quantizer (``reconstruct.load_quantizer``) as
  well as a table tensor; with a quantizer, a layer's ``chosen_r`` selects the
  table ``raw / chosen_r`` exactly as ``dequantize_layer`` does
  (``algorithms/eptq.py:432-457``) — the reference kernel path ignores it.
* ``S_group`` layers stay compressed and run the fused grouped kernel instead
  of a materialized fp16 W (``kernels/linear.py:97-120,158-164``).
* every batch size runs a hand-written HIP kernel of this library: the decode
  matvec for ≤16 rows, 16-row slices of the matrix-core decode up to 128 rows,
  the prefill GEMM that decodes weight tiles into LDS above (the reference's
  ``csrc/eptq_kernels.cu:520-537`` route), and from 2048 fp16 tokens (256
  for S_group layers or bf16 x, 64 for E8 layers) the two-pass prefill: each weight
  decoded once into a transient fp16 W (freed on return), then this
  library's W-streaming GEMM.  No library GEMM runs.  ``EPTQ_CUDA_DECODE`` / ``EPTQ_FORCE_TRITON`` are
  accepted and ignored.
* ``dequantize()`` returns the bit-exact fp16 W of ``dequantize_layer`` from the
  GPU (needs the fp32 table, kept alongside the fp16 kernel table).
"""

from __future__ import annotations

import hashlib
import weakref
from typing import Optional, Tuple

import torch
import torch.nn as nn

from . import dequant as _dequant  # noqa: F401  (also registers the eptq:: ops)

_KINDS = ("e8_lattice", "e8_d4")

# Layers whose tables carry the same bits share one fp32 and one fp16 tensor:
# (device, kind, sha256 of the fp32 bits) -> (fp32 table, fp16 table).  The
# entries are private snapshots (never views of a quantizer's codes), so no
# later radius change of the quantizer can alter a table already handed out;
# they are dropped once no layer holds them.
_SHARED: "weakref.WeakValueDictionary[Tuple, torch.Tensor]" = weakref.WeakValueDictionary()
_SHARED16: "weakref.WeakValueDictionary[Tuple, torch.Tensor]" = weakref.WeakValueDictionary()


def _share(tab: torch.Tensor, quantizer_type: str) -> Tuple[torch.Tensor, torch.Tensor]:
    tab = tab.detach().float().contiguous()
    digest = hashlib.sha256(tab.cpu().numpy().tobytes()).hexdigest()
    key = (str(tab.device), quantizer_type, tuple(tab.shape), digest)
    t32 = _SHARED.get(key)
    if t32 is None:
        t32 = tab.clone()
        _SHARED[key] = t32
    t16 = _SHARED16.get(key)
    if t16 is None:
        t16 = t32.to(torch.float16)
        _SHARED16[key] = t16
    return t32, t16


def _table_for(codebook, quantizer_type: str, chosen_r: Optional[float]) -> Tuple[torch.Tensor, torch.Tensor]:
    """(fp32, fp16) kernel-layout tables of one layer.

    With a quantizer, the layer's table is what ``dequantize_layer`` decodes
    with (``algorithms/eptq.py:430-457``): the quantizer is switched to the
    layer's ``chosen_r`` when that differs from its radius, the table is read,
    and the radius is switched back — on the quantizer object itself, so a
    legacy table (no raw codes: ``set_radius`` rescales in place) drifts from
    layer to layer exactly as it does when the reference reconstructs the
    layers in the same order, and a warped table loses its warp at the first
    such switch as the reference's does (``quantizers/e8_d4.py:90-102``).
    The table handed to the layer is a copy taken at that point."""
    if isinstance(codebook, torch.Tensor):
        t = codebook.float()
        t = t.reshape(512, 4) if quantizer_type == "e8_d4" else t.reshape(-1, 8)
        return _share(t, quantizer_type)
    q = codebook
    saved_r = q._radius
    swap = chosen_r is not None and chosen_r != saved_r
    if swap:
        q.set_radius(chosen_r)
    try:
        tab = q.flat_table().clone()
    finally:
        if swap:
            q.set_radius(saved_r)
    return _share(tab, quantizer_type)


class EPTQLinear(nn.Module):
    """Quantized Linear: Q (M, N) int16 indices + g/h scales + CSR outliers."""

    def __init__(self, Q: torch.Tensor, codebook: torch.Tensor, g: torch.Tensor,
                 h: torch.Tensor, O_vals: torch.Tensor, O_col: torch.Tensor,
                 O_row_ptr: torch.Tensor, bias: Optional[torch.Tensor], quantizer_type: str,
                 S_group: Optional[torch.Tensor] = None,
                 table_f32: Optional[torch.Tensor] = None):
        super().__init__()
        # Decode workspace of E8-D4 calls (``decode_workspace``): the
        # matrix-core kernel splits the columns of layers with few row tiles
        # over several workgroups through it.  None = the current stream's
        # own (``stream_workspace``; none, i.e. the unsplit kernel, while a
        # graph is being captured); calls sharing one must not overlap in
        # time.
        self._work: Optional[torch.Tensor] = None
        if quantizer_type not in _KINDS:
            raise ValueError(f"unknown quantizer_type {quantizer_type!r}")
        self.in_features = int(Q.shape[1])
        self.out_features = int(Q.shape[0]) * 8
        self.quantizer_type = quantizer_type
        self.register_buffer("Q", Q.contiguous())
        self.register_buffer("g", g.contiguous())
        self.register_buffer("h", h.contiguous())
        self.register_buffer("O_vals", O_vals.contiguous())
        self.register_buffer("O_col", O_col.contiguous())
        self.register_buffer("O_row_ptr", O_row_ptr.contiguous())
        self.register_buffer("bias", bias.contiguous() if bias is not None else None)
        self.register_buffer("S_group", S_group.contiguous() if S_group is not None else None)
        # Shared tables — not buffers, so they are not duplicated in state_dict.
        self._codebook = codebook
        self._table_f32 = table_f32 if table_f32 is not None else codebook.float()

    def _apply(self, fn, *args, **kwargs):
        super()._apply(fn, *args, **kwargs)
        self._codebook = fn(self._codebook)
        self._table_f32 = fn(self._table_f32)
        return self

    @classmethod
    def from_quantized_data(cls, quant_data, codebook, quantizer_type: str) -> "EPTQLinear":
        """Build from a ``QuantizedLayerData`` (``kernels/linear.py:83-152``).

        ``codebook``: the shared table tensor (E8-D4 (4,128,4)/(512,4), E8
        (65535, 8); fp16 or fp32, already divided by the radius) or a loaded
        quantizer, which also honours the layer's ``chosen_r``.
        """
        if quantizer_type not in _KINDS:
            raise ValueError(f"unknown quantizer_type {quantizer_type!r}")
        Q = quant_data.Q
        if Q.dtype != torch.int16:
            raise ValueError(f"Q must be int16, got {Q.dtype}")
        M = Q.shape[0]
        tab32, cb16 = _table_for(codebook, quantizer_type, quant_data.chosen_r)

        # Critical blocks — nonzero() on row-major Q is in row-major order.
        mask = Q == 32767
        O_row, O_col = mask.nonzero(as_tuple=True)
        n_masked = int(O_row.shape[0])
        if int(quant_data.O.shape[0]) != n_masked:
            raise ValueError(f"layer data is inconsistent: Q marks {n_masked} critical blocks "
                             f"(entries equal to 32767) but O holds {quant_data.O.shape[0]} rows")
        counts = torch.bincount(O_row.long(), minlength=M)
        O_row_ptr = torch.cat([torch.zeros(1, dtype=torch.int32, device=O_row.device),
                               counts.cumsum(0).to(torch.int32)])
        S = quant_data.S_group
        if S is not None:
            S = S.to(torch.float16)
        return cls(Q=Q, codebook=cb16, g=quant_data.g.to(torch.float16),
                   h=quant_data.h.to(torch.float16),
                   O_vals=quant_data.O.to(torch.float16).reshape(-1, 8),
                   O_col=O_col.to(torch.int32), O_row_ptr=O_row_ptr,
                   bias=quant_data.bias.to(torch.float16) if quant_data.bias is not None else None,
                   quantizer_type=quantizer_type, S_group=S, table_f32=tab32)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # Only registered ops below (reference kernels/linear.py:177-208), so
        # torch.compile traces the call without a graph break.
        shape = x.shape
        out_dtype = x.dtype
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype not in (torch.float16, torch.bfloat16):
            x2 = x2.half()
        x2 = x2.contiguous()
        if self.quantizer_type == "e8_d4":
            y = torch.ops.eptq.e8d4_forward_multi([self.Q], self._codebook, [self.g], [self.h], x2,
                                                  [self.O_vals], [self.O_col], [self.O_row_ptr],
                                                  [self.bias], [self.S_group], self._work)
        else:
            bias = self.bias if self.bias is not None else x2.new_empty(0, dtype=torch.float16)
            if self.S_group is None:
                y = torch.ops.eptq.e8_forward(self.Q, self._codebook, self.g, self.h, x2, self.O_vals,
                                              self.O_col, self.O_row_ptr, bias)
            else:
                y = torch.ops.eptq.e8_forward_grouped(self.Q, self._codebook, self.g, self.h, x2,
                                                      self.O_vals, self.O_col, self.O_row_ptr, bias,
                                                      self.S_group)
        if y.dtype != out_dtype:
            y = y.to(out_dtype)
        return y.reshape(*shape[:-1], self.out_features)

    @torch.no_grad()
    def dequantize(self) -> torch.Tensor:
        """fp16 W (out, in), bit-exact with ``dequantize_layer`` on the same table."""
        return _dequant(self.quantizer_type, self.Q, self._table_f32, self.g, self.h,
                        self.O_vals, self.O_col, self.O_row_ptr, self.S_group)

    def extra_repr(self) -> str:
        return (f"in={self.in_features}, out={self.out_features}, "
                f"quantizer={self.quantizer_type}, n_masked={self.O_col.shape[0]}"
                + (f", groups={self.S_group.shape[0]}" if self.S_group is not None else ""))


QuantizedLinear = EPTQLinear


class EPTQMultiLinear(nn.Module):
    """Several E8-D4 ``EPTQLinear`` layers applied to the same input, outputs
    side by side (e.g. q|k|v or gate|up): one kernel launch per call where the
    decode kernel takes them all.  Each layer keeps its own scales and
    critical blocks; no weights are merged."""

    def __init__(self, linears):
        super().__init__()
        self._work: Optional[torch.Tensor] = None   # as EPTQLinear._work
        ls = list(linears)
        if not ls or any(l.quantizer_type != "e8_d4" for l in ls):
            raise ValueError("EPTQMultiLinear takes one or more E8-D4 layers")
        if len({l.in_features for l in ls}) != 1 or any(not torch.equal(l._table_f32, ls[0]._table_f32)
                                                        for l in ls[1:]):
            raise ValueError("layers must share in_features and the codebook table")
        self.parts = nn.ModuleList(ls)
        self.in_features = ls[0].in_features
        self.out_features = sum(l.out_features for l in ls)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape, out_dtype = x.shape, x.dtype
        x2 = x.reshape(-1, self.in_features)
        if x2.dtype not in (torch.float16, torch.bfloat16):
            x2 = x2.half()
        x2 = x2.contiguous()
        ps = list(self.parts)
        y = torch.ops.eptq.e8d4_forward_multi([l.Q for l in ps], ps[0]._codebook, [l.g for l in ps],
                                              [l.h for l in ps], x2, [l.O_vals for l in ps],
                                              [l.O_col for l in ps], [l.O_row_ptr for l in ps],
                                              [l.bias for l in ps], [l.S_group for l in ps], self._work)
        if y.dtype != out_dtype:
            y = y.to(out_dtype)
        return y.reshape(*shape[:-1], self.out_features)
