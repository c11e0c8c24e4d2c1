"""EPTQ HIP kernels as ``torch.library`` custom ops.

Drop-in for the reference's ``kernels/__init__.py:50-91``: the ops
``eptq::e8_forward`` and ``eptq::e8d4_forward`` keep their names, argument
order and meaning ``(Q, codebook, g, h, x, O_vals, O_col, O_row_ptr, bias)``
(an empty ``bias`` means no bias) and have fake implementations for
``torch.compile``.  They run the gfx950 kernels of ``libeptq_hip.so`` through
its C ABI on the current HIP stream; there is no CPU or PyTorch fallback.

Additions over the reference: fp32 tables are accepted (the kernels convert),
bf16 activations give bf16 outputs, ``*_grouped`` variants take ``S_group``
(the reference materializes an fp16 W instead, ``kernels/linear.py:97-120``),
``eptq::e8d4_dequant`` / ``eptq::e8_dequant`` produce the bit-exact fp16 W of
``dequantize_layer`` (``algorithms/eptq.py:406-471``) on the GPU, and
``eptq::e8d4_forward_multi`` runs several E8-D4 layers that share x (q|k|v,
gate|up) in one launch with a split-K workspace.  ``EPTQLinear.forward`` and
``EPTQMultiLinear.forward`` call only these registered ops, so, as in the
reference (``kernels/__init__.py:44-47``), ``torch.compile(fullgraph=True)``
sees each quantized Linear as one op with no graph break.
"""

from __future__ import annotations


import threading
from typing import List, Optional

import torch

from . import _lib
from ._lib import EPTQ_BF16, EPTQ_F16, EPTQ_F32, EptqError

__all__ = ["e8_forward", "e8d4_forward", "e8_forward_grouped", "e8d4_forward_grouped",
           "e8d4_forward_multi", "e8_dequant", "e8d4_dequant", "EptqError", "linear_forward",
           "linear_forward_multi", "dequant", "decode_workspace", "stream_workspace"]


def _ptr(t: Optional[torch.Tensor]):
    if t is None or t.numel() == 0:
        return None
    return t.data_ptr()


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


def _check_layer(kind, Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group):
    _require(Q.is_cuda, "Q must be a CUDA (HIP) tensor")
    dev = Q.device
    _require(Q.dtype == torch.int16 and Q.dim() == 2 and Q.is_contiguous(),
             "Q must be a contiguous 2-D int16 tensor")
    M, N = Q.shape
    for name, t, dt in (("g", g, torch.float16), ("h", h, torch.float16),
                        ("O_vals", O_vals, torch.float16), ("O_col", O_col, torch.int32),
                        ("O_row_ptr", O_row_ptr, torch.int32)):
        _require(t.device == dev, f"{name} must be on {dev}")
        _require(t.dtype == dt, f"{name} must be {dt}, got {t.dtype}")
        _require(t.is_contiguous(), f"{name} must be contiguous")
    _require(g.numel() == 8 * M, f"g must have {8 * M} elements")
    _require(h.numel() == N, f"h must have {N} elements")
    _require(O_row_ptr.numel() == M + 1, f"O_row_ptr must have {M + 1} elements")
    _require(O_vals.numel() == 8 * O_col.numel(), "O_vals must be (nnz, 8) with nnz = len(O_col)")
    _require(codes.device == dev and codes.is_contiguous(), "codebook must be contiguous on the layer's device")
    _require(codes.dtype in (torch.float16, torch.float32), "codebook must be fp16 or fp32")
    rows = 512 if kind == "e8_d4" else 65535
    _require(codes.numel() == rows * (4 if kind == "e8_d4" else 8),
             f"{kind} codebook must have {rows} rows")
    n_groups = 0
    if S_group is not None:
        _require(S_group.device == dev and S_group.dtype == torch.float16 and S_group.is_contiguous(),
                 "S_group must be a contiguous fp16 tensor on the layer's device")
        _require(S_group.dim() == 2 and S_group.shape[1] == N, "S_group must be (n_groups, in_features)")
        n_groups = int(S_group.shape[0])
    return M, N, n_groups


def linear_forward(kind: str, Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias=None,
                   S_group=None, two_pass: bool = False) -> torch.Tensor:
    """Run the fused quantized Linear on ``x`` (B, N) -> (B, 8M), dtype of x.
    ``two_pass`` (what the module's ops pass): from ``_two_pass_min`` tokens
    (2048 for E8-D4, 256 with S_group or bf16 x, 64 for E8) and 64-multiple
    shapes, the two-pass prefill instead of the fused C-ABI kernel."""
    M, N, n_groups = _check_layer(kind, Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group)
    _require(x.device == Q.device, "x must be on the layer's device")
    _require(x.dim() == 2 and x.shape[1] == N, f"x must be (B, {N})")
    _require(x.dtype in (torch.float16, torch.bfloat16), "x must be fp16 or bf16")
    _require(x.is_contiguous(), "x must be contiguous")
    if bias is not None and bias.numel() > 0:
        _require(bias.device == Q.device and bias.dtype == torch.float16 and bias.numel() == 8 * M
                 and bias.is_contiguous(), "bias must be a contiguous fp16 (out_features,) tensor")
    B = int(x.shape[0])
    y = torch.empty((B, 8 * M), dtype=x.dtype, device=x.device)
    if B == 0:
        return y
    lib = _lib.load()
    layer = dict(Q=Q, g=g, h=h, O_vals=O_vals, O_col=O_col, O_row_ptr=O_row_ptr, bias=bias, S_group=S_group)
    if two_pass and B >= _two_pass_min(kind, [layer], x) and _two_pass_ok([layer], x, N):
        _two_pass_into(lib, [layer], codes, x, y, kind)
        return y
    fn = lib.eptq_e8d4_forward if kind == "e8_d4" else lib.eptq_e8_forward
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream().cuda_stream
        rc = fn(_ptr(Q), _ptr(codes), EPTQ_F32 if codes.dtype == torch.float32 else EPTQ_F16,
                _ptr(g), _ptr(h), _ptr(x), EPTQ_BF16 if x.dtype == torch.bfloat16 else EPTQ_F16,
                _ptr(O_vals), _ptr(O_col), _ptr(O_row_ptr), _ptr(bias), _ptr(S_group), n_groups,
                M, N, B, _ptr(y), stream)
    _lib.check(rc, fn.__name__)
    return y


def decode_workspace(device) -> torch.Tensor:
    """A zero-filled workspace for ``linear_forward_multi(..., work=)`` on
    ``device`` (``eptq_e8d4_work_bytes`` bytes)."""
    with torch.cuda.device(device):
        n = int(_lib.load().eptq_e8d4_work_bytes())
    return torch.zeros(n, dtype=torch.uint8, device=device)


# One split-K workspace per (device, stream): launches on one stream run one
# after another, so modules that share their stream's workspace never overlap
# on it.  Created on first eager use, zero-filled before that stream uses it.
_STREAM_WORK: dict = {}


def stream_workspace(device) -> Optional[torch.Tensor]:
    """The decode workspace of the current stream on ``device`` (see
    ``decode_workspace``), created on first eager use.

    While the current stream is capturing a graph this returns None (the
    unsplit kernel, same results): a workspace made during a capture would
    come from that graph's private pool with its zero fill recorded, not run,
    and graphs captured on one stream may later replay concurrently on
    different streams.  A caller that wants split-K inside a captured graph
    attaches its own workspace (``EPTQLinear._work = decode_workspace(dev)``),
    which that graph's replays then must not share with concurrent work."""
    device = torch.device(device)
    if torch.cuda.is_current_stream_capturing():
        return None
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    w = _STREAM_WORK.get(key)
    if w is None:
        w = _workspace_outside_graph_pools(device, stream)
        _STREAM_WORK[key] = w
    return w


def _workspace_outside_graph_pools(device, stream) -> torch.Tensor:
    """``decode_workspace`` allocated and zero-filled by a helper thread on a
    stream of its own, then ordered before ``stream``.  The calling thread
    may be routing its allocations into a graph's private memory pool
    (torch.compile's cudagraph warm-up runs do, per thread), where a buffer
    kept alive across calls does not belong."""
    box = {}

    def run():
        try:
            with torch.cuda.device(device):
                side = torch.cuda.Stream(device)
                side.wait_stream(stream)
                with torch.cuda.stream(side):
                    box["w"] = decode_workspace(device)
                    box["ev"] = side.record_event()
        except BaseException as e:  # re-raised in the caller
            box["err"] = e

    t = threading.Thread(target=run, name="eptq-workspace")
    t.start()
    t.join()
    if "err" in box:
        raise box["err"]
    stream.wait_event(box["ev"])
    return box["w"]


# Token counts from which the module's forwards run the two-pass prefill
# (every weight decoded once into a transient fp16 W, then eptq_f16_gemm).
# E8-D4: measured 1.09-1.36x the fused kernel at 2048 tokens on the six
# Llama-2-7B / 13B projection shapes, mixed at 1024 (0.85-1.11x: the fused
# kernel splits K over idle CUs there), slower at 512.  E8-D4 with S_group
# (whose fused path is the older grouped GEMM): 1.2-1.8x from 256 tokens on
# 4096x4096, 11008x4096 and 4096x11008.  E8 (whose fused GEMM gathers from a
# 1 MB table): 2x from 64 tokens on 4096x4096, 1.3-2.5x at 256-2048 tokens on
# 4096x4096 and 11008x4096, level on 3072x768.  E8-D4 with bf16 x (whose
# fused path decodes into registers): 1.2-2.1x from 256 tokens on 4096x4096,
# 11008x4096, 4096x11008 and 14336x4096.
TWO_PASS_MIN_TOKENS = 2048
TWO_PASS_MIN_TOKENS_GROUPED = 256
TWO_PASS_MIN_TOKENS_BF16 = 256
TWO_PASS_MIN_TOKENS_E8 = 64


def _two_pass_min(kind: str, layers, x) -> int:
    if kind != "e8_d4":
        return TWO_PASS_MIN_TOKENS_E8
    if x.dtype == torch.bfloat16:
        return TWO_PASS_MIN_TOKENS_BF16
    return TWO_PASS_MIN_TOKENS_GROUPED if all(L.get("S_group") is not None for L in layers) else TWO_PASS_MIN_TOKENS


def _two_pass_ok(layers, x, N) -> bool:
    # bf16 x goes through eptq_bf16_rows_to_f16 (rows up to 16384 columns).
    return ((x.dtype == torch.float16 or (x.dtype == torch.bfloat16 and N <= 16384)) and N % 64 == 0
            and all((8 * int(L["Q"].shape[0])) % 64 == 0 for L in layers))


def _two_pass_into(lib, layers, codes, x, y, kind: str = "e8_d4") -> None:
    """y[:, layer columns] = x · W_lᵀ + bias_l with each layer's W decoded once
    (``eptq_e8d4_dequant`` / ``eptq_e8_dequant``, S_group included, into one
    transient buffer sized for the largest layer, reused layer after layer on
    the stream) and multiplied by ``eptq_f16_gemm_rows``.  The table is the
    kernels' (fp16, widened to fp32): the same table values the fused kernel
    multiplies.  bf16 x is first taken to fp16 row by row with a power-of-two
    scale (``eptq_bf16_rows_to_f16``) that the GEMM restores at its bf16
    output."""
    N = int(x.shape[1])
    B, ldy = int(x.shape[0]), int(y.shape[1])
    tab = codes if codes.dtype == torch.float32 else codes.float()
    F_max = max(8 * int(L["Q"].shape[0]) for L in layers)
    wbuf = torch.empty(F_max * N, dtype=torch.float16, device=x.device)
    deq = lib.eptq_e8d4_dequant if kind == "e8_d4" else lib.eptq_e8_dequant
    off = 0
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream().cuda_stream
        xg, rs = x, None
        if x.dtype == torch.bfloat16:
            xg = torch.empty((B, N), dtype=torch.float16, device=x.device)
            rs = torch.empty(B, dtype=torch.float32, device=x.device)
            _lib.check(lib.eptq_bf16_rows_to_f16(_ptr(x), N, B, _ptr(xg), _ptr(rs), stream), "eptq_bf16_rows_to_f16")
        y_dtype = EPTQ_BF16 if y.dtype == torch.bfloat16 else EPTQ_F16
        for L in layers:
            M = int(L["Q"].shape[0])
            S = L.get("S_group")
            n_groups = 0 if S is None else int(S.shape[0])
            rc = deq(_ptr(L["Q"]), _ptr(tab), _ptr(L["g"]), _ptr(L["h"]), _ptr(L["O_vals"]), _ptr(L["O_col"]),
                     _ptr(L["O_row_ptr"]), _ptr(S), n_groups, M, N, _ptr(wbuf), stream)
            _lib.check(rc, deq.__name__)
            rc = lib.eptq_f16_gemm_rows(_ptr(wbuf), _ptr(xg), _ptr(L.get("bias")), 8 * M, N, B, _ptr(rs),
                                        _ptr(y) + 2 * off, y_dtype, ldy, stream)
            _lib.check(rc, "eptq_f16_gemm_rows")
            off += 8 * M


def linear_forward_multi(layers, codes, x, work: Optional[torch.Tensor] = None,
                         two_pass: bool = False) -> torch.Tensor:
    """E8-D4 layers sharing ``x`` (B, N) -> (B, Σ out) with the layers' outputs
    side by side, in one decode launch when the kernel takes them all.
    ``layers``: dicts with Q, g, h, O_vals, O_col, O_row_ptr and optional
    bias, S_group (the EPTQLinear buffers).  ``two_pass`` (what the
    module's op passes): from ``_two_pass_min`` fp16 tokens (64-multiple
    shapes) the two-pass prefill (``_two_pass_into``) instead of the fused
    C-ABI launch.  ``work``: optional workspace from
    ``decode_workspace`` (lets batches of 3..16 split the columns of layers
    with few row tiles over several workgroups); calls sharing one must not
    overlap in time."""
    _require(len(layers) > 0, "no layers")
    _require(x.dim() == 2 and x.dtype in (torch.float16, torch.bfloat16) and x.is_contiguous(),
             "x must be a contiguous 2-D fp16/bf16 tensor")
    N = int(x.shape[1])
    arr = (_lib.EptqLayer * len(layers))()
    off = 0
    keep = []
    for i, L in enumerate(layers):
        M, n2, n_groups = _check_layer("e8_d4", L["Q"], codes, L["g"], L["h"], L["O_vals"], L["O_col"],
                                       L["O_row_ptr"], L.get("S_group"))
        _require(n2 == N and L["Q"].device == x.device, "layers must take x's in_features on x's device")
        b = L.get("bias")
        arr[i] = _lib.EptqLayer(_ptr(L["Q"]), _ptr(L["g"]), _ptr(L["h"]), _ptr(L["O_vals"]), _ptr(L["O_col"]),
                                _ptr(L["O_row_ptr"]), _ptr(b), _ptr(L.get("S_group")), n_groups, M, off)
        off += 8 * M
        keep.append(L)
    B = int(x.shape[0])
    y = torch.empty((B, off), dtype=x.dtype, device=x.device)
    if B == 0:
        return y
    lib = _lib.load()
    if two_pass and B >= _two_pass_min("e8_d4", keep, x) and _two_pass_ok(keep, x, N):
        _two_pass_into(lib, keep, codes, x, y)
        return y
    with torch.cuda.device(x.device):
        stream = torch.cuda.current_stream().cuda_stream
        rc = lib.eptq_e8d4_forward_multi(len(layers), arr, _ptr(codes),
                                         EPTQ_F32 if codes.dtype == torch.float32 else EPTQ_F16, _ptr(x),
                                         EPTQ_BF16 if x.dtype == torch.bfloat16 else EPTQ_F16, N, B,
                                         _ptr(y), off, _ptr(work), 0 if work is None else work.numel(),
                                         stream)
    _lib.check(rc, "eptq_e8d4_forward_multi")
    return y


def dequant(kind: str, Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group=None,
            out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Bit-exact fp16 W (8M, N) on the GPU; ``codes`` must be the fp32 table.
    ``out``: a contiguous fp16 (8M, N) tensor on Q's device to write W into."""
    M, N, n_groups = _check_layer(kind, Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group)
    _require(codes.dtype == torch.float32, "dequant needs the fp32 table for bit-exact W")
    if out is None:
        W = torch.empty((8 * M, N), dtype=torch.float16, device=Q.device)
    else:
        _require(out.dtype == torch.float16 and tuple(out.shape) == (8 * M, N) and out.is_contiguous()
                 and out.device == Q.device, "out must be a contiguous fp16 (8M, N) tensor on Q's device")
        W = out
    lib = _lib.load()
    fn = lib.eptq_e8d4_dequant if kind == "e8_d4" else lib.eptq_e8_dequant
    with torch.cuda.device(Q.device):
        stream = torch.cuda.current_stream().cuda_stream
        rc = fn(_ptr(Q), _ptr(codes), _ptr(g), _ptr(h), _ptr(O_vals), _ptr(O_col),
                _ptr(O_row_ptr), _ptr(S_group), n_groups, M, N, _ptr(W), stream)
    _lib.check(rc, fn.__name__)
    return W


def f16_gemm(W: torch.Tensor, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y (T, F) = x (T, N) · Wᵀ + bias for fp16 W (F, N): the second pass of
    the two-pass prefill (``eptq_f16_gemm``).  Raises EptqError (code 2)
    where the kernel does not take the shape (F, N multiples of 64)."""
    _require(W.dtype == torch.float16 and x.dtype == torch.float16 and W.is_contiguous() and x.is_contiguous()
             and W.dim() == 2 and x.dim() == 2 and W.shape[1] == x.shape[1] and W.device == x.device,
             "W (F, N) and x (T, N) must be contiguous fp16 on one device")
    _require(bias is None or (bias.dtype == torch.float16 and bias.is_contiguous() and bias.numel() == W.shape[0]),
             "bias must be a contiguous fp16 (F,) tensor")
    F, N = int(W.shape[0]), int(W.shape[1])
    T = int(x.shape[0])
    y = torch.empty((T, F), dtype=torch.float16, device=x.device)
    with torch.cuda.device(x.device):
        rc = _lib.load().eptq_f16_gemm(_ptr(W), _ptr(x), _ptr(bias), F, N, T, _ptr(y), F,
                                       torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "eptq_f16_gemm")
    return y


# ---------------------------------------------------------------------------
# torch.library registration (names and signatures of kernels/__init__.py:50-91)
# ---------------------------------------------------------------------------

@torch.library.custom_op("eptq::e8_forward", mutates_args=())
def e8_forward(Q: torch.Tensor, codebook: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
               x: torch.Tensor, O_vals: torch.Tensor, O_col: torch.Tensor,
               O_row_ptr: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    return linear_forward("e8_lattice", Q, codebook, g, h, x, O_vals, O_col, O_row_ptr, bias, two_pass=True)


@e8_forward.register_fake
def _e8_forward_fake(Q, codebook, g, h, x, O_vals, O_col, O_row_ptr, bias):
    return x.new_empty(x.shape[0], Q.shape[0] * 8)


@torch.library.custom_op("eptq::e8d4_forward", mutates_args=())
def e8d4_forward(Q: torch.Tensor, codes: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
                 x: torch.Tensor, O_vals: torch.Tensor, O_col: torch.Tensor,
                 O_row_ptr: torch.Tensor, bias: torch.Tensor) -> torch.Tensor:
    return linear_forward("e8_d4", Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias, two_pass=True)


@e8d4_forward.register_fake
def _e8d4_forward_fake(Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias):
    return x.new_empty(x.shape[0], Q.shape[0] * 8)


@torch.library.custom_op("eptq::e8_forward_grouped", mutates_args=())
def e8_forward_grouped(Q: torch.Tensor, codebook: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
                       x: torch.Tensor, O_vals: torch.Tensor, O_col: torch.Tensor,
                       O_row_ptr: torch.Tensor, bias: torch.Tensor,
                       S_group: torch.Tensor) -> torch.Tensor:
    return linear_forward("e8_lattice", Q, codebook, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group,
                          two_pass=True)


@e8_forward_grouped.register_fake
def _e8_forward_grouped_fake(Q, codebook, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group):
    return x.new_empty(x.shape[0], Q.shape[0] * 8)


@torch.library.custom_op("eptq::e8d4_forward_grouped", mutates_args=())
def e8d4_forward_grouped(Q: torch.Tensor, codes: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
                         x: torch.Tensor, O_vals: torch.Tensor, O_col: torch.Tensor,
                         O_row_ptr: torch.Tensor, bias: torch.Tensor,
                         S_group: torch.Tensor) -> torch.Tensor:
    return linear_forward("e8_d4", Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group, two_pass=True)


@e8d4_forward_grouped.register_fake
def _e8d4_forward_grouped_fake(Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group):
    return x.new_empty(x.shape[0], Q.shape[0] * 8)


@torch.library.custom_op("eptq::e8d4_dequant", mutates_args=())
def e8d4_dequant(Q: torch.Tensor, codes: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
                 O_vals: torch.Tensor, O_col: torch.Tensor, O_row_ptr: torch.Tensor,
                 S_group: Optional[torch.Tensor] = None) -> torch.Tensor:
    return dequant("e8_d4", Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group)


@e8d4_dequant.register_fake
def _e8d4_dequant_fake(Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group=None):
    return Q.new_empty(Q.shape[0] * 8, Q.shape[1], dtype=torch.float16)


@torch.library.custom_op("eptq::e8_dequant", mutates_args=())
def e8_dequant(Q: torch.Tensor, codes: torch.Tensor, g: torch.Tensor, h: torch.Tensor,
               O_vals: torch.Tensor, O_col: torch.Tensor, O_row_ptr: torch.Tensor,
               S_group: Optional[torch.Tensor] = None) -> torch.Tensor:
    return dequant("e8_lattice", Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group)


@e8_dequant.register_fake
def _e8_dequant_fake(Q, codes, g, h, O_vals, O_col, O_row_ptr, S_group=None):
    return Q.new_empty(Q.shape[0] * 8, Q.shape[1], dtype=torch.float16)


@torch.library.custom_op("eptq::e8d4_forward_multi", mutates_args=("work",))
def e8d4_forward_multi(Q: List[torch.Tensor], codes: torch.Tensor, g: List[torch.Tensor],
                       h: List[torch.Tensor], x: torch.Tensor, O_vals: List[torch.Tensor],
                       O_col: List[torch.Tensor], O_row_ptr: List[torch.Tensor],
                       bias: List[Optional[torch.Tensor]], S_group: List[Optional[torch.Tensor]],
                       work: Optional[torch.Tensor]) -> torch.Tensor:
    """E8-D4 layers sharing ``x`` (B, N) -> (B, Σ 8·M_l), outputs side by side
    (``linear_forward_multi``); the op ``EPTQLinear`` / ``EPTQMultiLinear``
    call for E8-D4 layers.  No counterpart in the reference, whose module
    calls ``eptq::e8d4_forward`` per projection (``kernels/linear.py:177-208``).

    ``work`` (required, may be None; a mutated argument with a default
    trips torch's in-place bookkeeping): a ``decode_workspace`` tensor
    (declared mutated: the split-K parts write their partial sums there; the
    counters return to zero), or None for the current stream's own (``stream_workspace``), which the op
    looks up when it runs, like a BLAS library's internal workspace."""
    layers = [dict(Q=Q[i], g=g[i], h=h[i], O_vals=O_vals[i], O_col=O_col[i], O_row_ptr=O_row_ptr[i],
                   bias=bias[i], S_group=S_group[i]) for i in range(len(Q))]
    if work is None and x.is_cuda:
        work = stream_workspace(x.device)
    return linear_forward_multi(layers, codes, x, work=work, two_pass=True)


@e8d4_forward_multi.register_fake
def _e8d4_forward_multi_fake(Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group, work):
    n = len(Q)
    torch._check(n > 0 and all(len(t) == n for t in (g, h, O_vals, O_col, O_row_ptr, bias, S_group)),
                 lambda: "every per-layer list must have one entry per layer")
    return x.new_empty(x.shape[0], sum(q.shape[0] * 8 for q in Q))
