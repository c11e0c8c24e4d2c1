"""Batch-1 chains of dependent E8-D4 Linears in one launch (``include/eptq_chain.h``).

No counterpart in the reference, whose decode step launches one
``EPTQLinear`` per projection (``kernels/linear.py:154-212``, timed by
``bench_decode.py:50-71``).  A ``DecodeChain`` runs a fixed sequence of
stages — each one or more E8-D4 layers sharing an input vector — where every
stage's input is a slice of the chain input or of an earlier stage's output,
optionally through SwiGLU and an RMSNorm, as one persistent HIP launch.

``llama_chain`` builds the chain of a Llama decoder stack without attention
and residuals (per layer: RMSNorm -> q|k|v; the q slice -> o; RMSNorm ->
gate|up; SwiGLU -> down; the next layer's RMSNorm reads down's output), the
dependency structure of a decode step's Linears.
"""

from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import torch

from .kernels import _lib
from .kernels.linear import EPTQLinear

SLICE, SWIGLU = 0, 1

_P, _I, _F, _LL = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_longlong


class ChainStage(ctypes.Structure):
    """``eptq_chain_stage`` of include/eptq_chain.h."""
    _fields_ = [("n_layers", _I), ("layers", _P), ("out_features", _I), ("src", _I), ("src_col", _I),
                ("N", _I), ("act", _I), ("norm_weight", _P), ("eps", _F), ("y", _P)]


class ChainPlan(ctypes.Structure):
    """``eptq_chain_plan`` of include/eptq_chain.h."""
    _fields_ = [("codes", _P), ("n_stages", _I), ("grid", _I), ("lds_bytes", _I), ("copies", _I),
                ("slot_bytes", _I), ("csc_offset", _I), ("pad", _I), ("spin_ticks", _LL), ("work_bytes", _LL)]


CHAIN_SIGNATURES = {
    "eptq_e8d4_chain_work_bytes": ([_P, _I], _LL),
    "eptq_e8d4_chain_plan": ([_P, _I, _P, _P, _LL, _P, _P], _I),
    "eptq_e8d4_chain_run": ([_P, _P, _P, _P], _I),
    "eptq_e8d4_chain_error": ([_P, _I, _P, _P], _I),
}


def _lib_chain():
    lib = _lib.load()
    for name, (args, res) in CHAIN_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None or t.numel() == 0 else t.data_ptr()


class DecodeChain:
    """A planned chain on one device.

    ``stages``: dicts with ``layers`` (E8-D4 ``EPTQLinear``s sharing the input,
    outputs side by side), ``src`` (-1: the chain input, else an earlier
    stage), ``src_col`` (first source column), ``act`` (``SLICE`` or
    ``SWIGLU``), optional ``norm_weight`` (fp16, in_features) and ``eps``.
    Stage outputs are ``self.y[s]`` (fp16, out_features), rewritten by every
    ``run``."""

    def __init__(self, stages: Sequence[dict], device="cuda"):
        lib = _lib_chain()
        self.device = torch.device(device)
        if self.device.index is None:
            self.device = torch.device(self.device.type, torch.cuda.current_device())
        n = len(stages)
        if n == 0:
            raise ValueError("a chain needs at least one stage")
        codes = stages[0]["layers"][0]._codebook
        self._keep = []
        self.y: List[torch.Tensor] = []
        arr = (ChainStage * n)()
        for s, st in enumerate(stages):
            lins = list(st["layers"])
            if any(not isinstance(l, EPTQLinear) or l.quantizer_type != "e8_d4" for l in lins):
                raise ValueError(f"stage {s}: chain stages take E8-D4 EPTQLinear layers")
            for l in lins:
                for name in ("Q", "g", "h", "O_vals", "O_col", "O_row_ptr", "bias", "_codebook"):
                    t = getattr(l, name)
                    if t is not None and t.device != self.device:
                        raise ValueError(f"stage {s}: {name} of a layer is on {t.device}, not on the chain's "
                                         f"device {self.device} (move the modules with .to(device))")
            if any(not torch.equal(l._codebook, codes) for l in lins):
                raise ValueError(f"stage {s}: every layer of a chain must share the codebook table")
            la = (_lib.EptqLayer * len(lins))()
            off = 0
            for i, l in enumerate(lins):
                la[i] = _lib.EptqLayer(_ptr(l.Q), _ptr(l.g), _ptr(l.h), _ptr(l.O_vals), _ptr(l.O_col),
                                       _ptr(l.O_row_ptr), _ptr(l.bias), None, 0, int(l.Q.shape[0]), off)
                off += l.out_features
            y = torch.empty(off, dtype=torch.float16, device=self.device)
            nw = st.get("norm_weight")
            if nw is not None:
                nw = nw.to(device=self.device, dtype=torch.float16).contiguous()
            self._keep += [la, nw, lins]
            self.y.append(y)
            arr[s] = ChainStage(len(lins), ctypes.cast(la, _P), off, int(st.get("src", -1)), int(st.get("src_col", 0)),
                                lins[0].in_features, int(st.get("act", SLICE)), _ptr(nw), float(st.get("eps", 1e-5)),
                                y.data_ptr())
        self._stages = arr
        with torch.cuda.device(self.device):
            nbytes = int(lib.eptq_e8d4_chain_work_bytes(arr, n))
            if nbytes <= 0:
                raise _lib.EptqError("eptq_e8d4_chain_work_bytes: " + lib.eptq_last_error().decode(), 2)
            self.work = torch.empty(nbytes + 256, dtype=torch.uint8, device=self.device)
            self._work_ptr = (self.work.data_ptr() + 255) & ~255
            self.plan = ChainPlan()
            rc = lib.eptq_e8d4_chain_plan(arr, n, codes.data_ptr(), self._work_ptr, nbytes, ctypes.byref(self.plan),
                                          torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(rc, "eptq_e8d4_chain_plan")
        self.codes = codes
        self.n_stages = n

    def run(self, x: torch.Tensor) -> None:
        """One pass of every stage on the current stream (asynchronous)."""
        if x.device != self.device or x.dtype != torch.float16 or not x.is_contiguous():
            raise ValueError("x must be a contiguous fp16 tensor on the chain's device")
        rc = _lib_chain().eptq_e8d4_chain_run(ctypes.byref(self.plan), self._work_ptr, x.data_ptr(),
                                              torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(rc, "eptq_e8d4_chain_run")

    def error(self, clear: bool = False) -> int:
        """The workspace's error word (synchronizes the current stream)."""
        err = ctypes.c_int(0)
        rc = _lib_chain().eptq_e8d4_chain_error(self._work_ptr, int(clear), ctypes.byref(err),
                                                torch.cuda.current_stream(self.device).cuda_stream)
        _lib.check(rc, "eptq_e8d4_chain_error")
        return err.value


def llama_stages(layers, norm_weights=None, eps: float = 1e-5) -> List[dict]:
    """Stages of a Llama decoder stack's Linears as a dependency chain.

    ``layers``: per decoder layer a dict with EPTQLinear ``q, k, v, o, gate,
    up, down``.  ``norm_weights``: per layer (input_norm, post_norm) fp16
    vectors, or None for no RMSNorm.  Stage 4l: q|k|v reading the chain input
    (l = 0) or the previous layer's down output; 4l+1: o reading the q slice;
    4l+2: gate|up reading o; 4l+3: down reading SwiGLU(gate, up)."""
    stages = []
    for i, L in enumerate(layers):
        nw = norm_weights[i] if norm_weights is not None else (None, None)
        stages.append(dict(layers=[L["q"], L["k"], L["v"]], src=-1 if i == 0 else 4 * i - 1, src_col=0,
                           act=SLICE, norm_weight=nw[0], eps=eps))
        stages.append(dict(layers=[L["o"]], src=4 * i, src_col=0, act=SLICE))
        stages.append(dict(layers=[L["gate"], L["up"]], src=4 * i + 1, src_col=0, act=SLICE, norm_weight=nw[1],
                           eps=eps))
        stages.append(dict(layers=[L["down"]], src=4 * i + 2, src_col=0, act=SWIGLU))
    return stages
