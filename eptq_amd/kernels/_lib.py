"""ctypes binding of the C ABI in ``include/eptq_hip.h`` (``libeptq_hip.so``).

The shared library is built in-tree by ``__graft_entry__.build()`` (or
``python -m eptq_amd.build``) into ``eptq_amd/_lib/``.  There is no fallback:
if the library is missing or fails to load, every op raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent.parent / "_lib" / "libeptq_hip.so"

EPTQ_OK, EPTQ_EINVAL, EPTQ_EUNSUPPORTED, EPTQ_EHIP, EPTQ_ETIMEOUT = 0, 1, 2, 3, 4
EPTQ_F16, EPTQ_F32, EPTQ_BF16 = 0, 1, 2

# Every symbol the header declares, with its ctypes signature.
_P, _I = ctypes.c_void_p, ctypes.c_int
SIGNATURES = {
    "eptq_abi_version": ([], _I),
    "eptq_last_error": ([], ctypes.c_char_p),
    "eptq_e8d4_forward": ([_P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P], _I),
    "eptq_e8_forward": ([_P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P], _I),
    "eptq_e8d4_forward_multi": ([_I, _P, _P, _I, _P, _I, _I, _I, _P, _I, _P, ctypes.c_longlong, _P], _I),
    "eptq_e8d4_work_bytes": ([], ctypes.c_longlong),
    "eptq_e8d4_forward_multi_noalloc": ([_I, _P, _P, _I, _P, _I, _I, _I, _P, _I, _P], _I),
    "eptq_e8d4_dequant": ([_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P], _I),
    "eptq_e8_dequant": ([_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P], _I),
    "eptq_f16_gemm": ([_P, _P, _P, _I, _I, _I, _P, _I, _P], _I),
    "eptq_f16_gemm_rows": ([_P, _P, _P, _I, _I, _I, _P, _P, _I, _I, _P], _I),
    "eptq_bf16_rows_to_f16": ([_P, _I, _I, _P, _P, _P], _I),
}

class EptqLayer(ctypes.Structure):
    """``eptq_layer`` of include/eptq_hip.h."""
    _fields_ = [("Q", _P), ("g", _P), ("h", _P), ("O_vals", _P), ("O_col", _P), ("O_row_ptr", _P),
                ("bias", _P), ("S_group", _P), ("n_groups", _I), ("M", _I), ("y_offset", ctypes.c_longlong)]


# Fused decode-step operators of the Llama harness (include/eptq_llama.h).
_F = ctypes.c_float
LLAMA_SIGNATURES = {
    "eptq_llama_rmsnorm": ([_P, _P, _P, _P, _I, _I, _F, _P], _I),
    "eptq_llama_rope_attn": ([_P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _P, _P], _I),
    "eptq_llama_attn_work_bytes": ([_I, _I], ctypes.c_longlong),
    "eptq_llama_silu_mul": ([_P, _P, _I, _I, _P], _I),
    "eptq_llama_norm_linear": ([_I, _P, _P, _P, _P, _P, _F, _P, _I, _I, _P, _I, _P], _I),
    "eptq_llama_norm_swiglu": ([_P, _P, _P, _P, _P, _F, _P, _I, _I, _P, _P], _I),
    "eptq_llama_linear": ([_I, _P, _P, _P, _I, _I, _P, _F, _P, _P, _I, _P, ctypes.c_longlong, _P], _I),
    "eptq_llama_linear_swiglu": ([_P, _P, _P, _I, _I, _P, _F, _P, _P, _P, ctypes.c_longlong, _P], _I),
    "eptq_llama_lm_head_work_bytes": ([_I], ctypes.c_longlong),
    "eptq_llama_lm_head_argmax": ([_P, _P, _P, _F, _P, _I, _I, _I, _P, _P, _P, _P, _P], _I),
}

_lib = None


class EptqError(RuntimeError):
    """A C-ABI call returned an error code (``code``: EPTQ_*; 0 if none)."""

    def __init__(self, msg: str, code: int = 0):
        super().__init__(msg)
        self.code = code


def load(path: os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and return the library with argtypes set."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise EptqError(
            f"EPTQ HIP library not built: {p} is missing "
            "(run __graft_entry__.build() or `python -m eptq_amd.build`)")
    lib = ctypes.CDLL(str(p))
    for name, (args, res) in {**SIGNATURES, **LLAMA_SIGNATURES}.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    if path is None:
        _lib = lib
    return lib


def check(rc: int, what: str) -> None:
    if rc != EPTQ_OK:
        msg = load().eptq_last_error().decode(errors="replace")
        raise EptqError(f"{what} failed (code {rc}): {msg}", rc)


def forward_into(kind: str, Q, codes, g, h, x, O_vals, O_col, O_row_ptr, bias, S_group,
                 y, stream: int) -> None:
    """Launch the fused Linear writing into a preallocated ``y`` (no allocation,
    no validation beyond the C ABI's own checks) — for graph capture and
    benchmarks.  Arguments are torch tensors; ``stream`` a raw hipStream_t."""
    lib = load()
    fn = lib.eptq_e8d4_forward if kind == "e8_d4" else lib.eptq_e8_forward

    def p(t):
        return None if t is None or t.numel() == 0 else t.data_ptr()

    n_groups = 0 if S_group is None else int(S_group.shape[0])
    codes_dt = EPTQ_F32 if codes.element_size() == 4 else EPTQ_F16
    x_dt = EPTQ_BF16 if str(x.dtype) == "torch.bfloat16" else EPTQ_F16
    rc = fn(p(Q), p(codes), codes_dt, p(g), p(h), p(x), x_dt, p(O_vals), p(O_col),
            p(O_row_ptr), p(bias), p(S_group), n_groups, int(Q.shape[0]), int(Q.shape[1]),
            int(x.shape[0]), p(y), stream)
    check(rc, fn.__name__)
