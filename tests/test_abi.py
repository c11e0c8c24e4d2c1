"""The C ABI boundary on the CPU: the library loads, exports every symbol that
``include/eptq_hip.h`` declares with the ctypes signatures the Python side
binds, and rejects invalid arguments with the documented codes before touching
the GPU (no compute calls here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from eptq_amd.kernels import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "eptq_hip.h"


def header_functions(path=HEADER):
    text = re.sub(r"/\*.*?\*/", "", path.read_text(), flags=re.S)
    return re.findall(r"^\s*(?:const\s+)?(?:long\s+)?\w+\s*\*?\s*(eptq_\w+)\s*\(", text, flags=re.M)


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        pytest.skip("libeptq_hip.so not built (run __graft_entry__.build())")
    return _lib.load()


def test_header_declares_the_bound_functions():
    names = header_functions()
    assert len(names) == len(set(names))
    assert set(names) == set(_lib.SIGNATURES)
    llama = header_functions(HEADER.parent / "eptq_llama.h")
    assert set(llama) == set(_lib.LLAMA_SIGNATURES)


def test_every_declared_symbol_is_exported(lib):
    for name in header_functions() + header_functions(HEADER.parent / "eptq_llama.h"):
        assert hasattr(lib, name), name
        assert isinstance(getattr(lib, name), ctypes._CFuncPtr)


def test_abi_version(lib):
    assert lib.eptq_abi_version() == 3
    assert lib.eptq_last_error() is not None


def _fwd_args(**over):
    a = dict(Q=16, codes=16, codes_dtype=_lib.EPTQ_F16, g=16, h=16, x=16, x_dtype=_lib.EPTQ_F16,
             O_vals=None, O_col=None, O_row_ptr=16, bias=None, S_group=None, n_groups=0,
             M=4, N=64, B=1, y=16, stream=None)
    a.update(over)
    return list(a.values())


@pytest.mark.parametrize("fn", ["eptq_e8d4_forward", "eptq_e8_forward"])
@pytest.mark.parametrize("over,code,msg", [
    (dict(Q=None), _lib.EPTQ_EINVAL, "null"),
    (dict(O_row_ptr=None), _lib.EPTQ_EINVAL, "null"),
    (dict(M=0), _lib.EPTQ_EINVAL, "positive"),
    (dict(N=-8), _lib.EPTQ_EINVAL, "positive"),
    (dict(B=-1), _lib.EPTQ_EINVAL, "B=-1"),
    (dict(x=None), _lib.EPTQ_EINVAL, "null x/y"),
    (dict(O_vals=16), _lib.EPTQ_EINVAL, "both"),
    (dict(codes_dtype=7), _lib.EPTQ_EINVAL, "codes_dtype"),
    (dict(x_dtype=_lib.EPTQ_F32), _lib.EPTQ_EINVAL, "x_dtype"),
    (dict(N=60), _lib.EPTQ_EUNSUPPORTED, "multiple of 8"),
    (dict(Q=18), _lib.EPTQ_EUNSUPPORTED, "aligned"),
    (dict(S_group=16, n_groups=3), _lib.EPTQ_EINVAL, "divide"),
    (dict(S_group=16, n_groups=8), _lib.EPTQ_EUNSUPPORTED, "multiple of 8"),
])
def test_forward_rejects_invalid_arguments(lib, fn, over, code, msg):
    rc = getattr(lib, fn)(*_fwd_args(**over))
    assert rc == code
    assert msg in lib.eptq_last_error().decode()
    assert fn in lib.eptq_last_error().decode()


def test_forward_empty_batch_is_a_no_op(lib):
    assert lib.eptq_e8d4_forward(*_fwd_args(B=0, x=None, y=None)) == _lib.EPTQ_OK


@pytest.mark.parametrize("fn", ["eptq_e8d4_dequant", "eptq_e8_dequant"])
def test_dequant_rejects_invalid_arguments(lib, fn):
    f = getattr(lib, fn)
    ok = dict(Q=16, codes=16, g=16, h=16, O_vals=None, O_col=None, O_row_ptr=16, S_group=None,
              n_groups=0, M=4, N=64, W=16, stream=None)
    rc = f(*{**ok, "W": None}.values())
    assert rc == _lib.EPTQ_EINVAL and "null W" in lib.eptq_last_error().decode()
    rc = f(*{**ok, "codes": 24}.values())
    assert rc == _lib.EPTQ_EUNSUPPORTED and "aligned" in lib.eptq_last_error().decode()
    rc = f(*{**ok, "W": 20}.values())
    assert rc == _lib.EPTQ_EUNSUPPORTED and "8-byte" in lib.eptq_last_error().decode()


def test_f16_gemm_rejects_invalid_arguments(lib):
    # (W, x, bias, F, N, T, y, ldy, stream); no argument here reaches a launch.
    f = lib.eptq_f16_gemm
    W, x, y = 1 << 20, 1 << 24, 1 << 28
    assert f(W, x, None, 128, 64, 0, y, 128, None) == _lib.EPTQ_OK          # empty batch: no-op
    assert f(None, x, None, 128, 64, 4, y, 128, None) == _lib.EPTQ_EINVAL
    assert "null" in lib.eptq_last_error().decode()
    assert f(W, x, None, 0, 64, 4, y, 128, None) == _lib.EPTQ_EINVAL
    assert f(W, x, None, 128, 64, 4, y, 64, None) == _lib.EPTQ_EINVAL       # ldy < F
    assert f(W, x, None, 128, 64, 4, x + 64, 128, None) == _lib.EPTQ_EINVAL  # y inside x
    assert "overlaps" in lib.eptq_last_error().decode()
    assert f(W, x, None, 100, 64, 4, y, 128, None) == _lib.EPTQ_EUNSUPPORTED  # F not a multiple of 64
    assert "multiples" in lib.eptq_last_error().decode()
    # y a column slice whose last row ends right where x starts: no overlap
    # (F = 100 then stops it before any launch, with the shape error).
    T, F, ldy = 4, 100, 256
    assert f(W, y + ((T - 1) * ldy + F) * 2, None, F, 64, T, y, ldy, None) == _lib.EPTQ_EUNSUPPORTED
    assert f(W, y + ((T - 1) * ldy + F) * 2 - 2, None, F, 64, T, y, ldy, None) == _lib.EPTQ_EINVAL


def test_bf16_two_pass_entry_points_reject_invalid_arguments(lib):
    g, r = lib.eptq_f16_gemm_rows, lib.eptq_bf16_rows_to_f16
    W, x, y, rs = 1 << 20, 1 << 24, 1 << 28, 1 << 30
    assert g(W, x, None, 128, 64, 4, rs, y, _lib.EPTQ_F32, 128, None) == _lib.EPTQ_EINVAL   # y fp16 or bf16 only
    assert "y_dtype" in lib.eptq_last_error().decode()
    assert g(W, x, None, 128, 64, 4, rs + 2, y, _lib.EPTQ_BF16, 128, None) == _lib.EPTQ_EUNSUPPORTED
    assert g(W, x, None, 128, 64, 4, y + 64, y, _lib.EPTQ_BF16, 128, None) == _lib.EPTQ_EINVAL  # row_scale inside y
    assert r(x, 4096, 0, y, rs, None) == _lib.EPTQ_OK                                            # no rows: no-op
    assert r(None, 4096, 4, y, rs, None) == _lib.EPTQ_EINVAL
    assert r(x, 4096, 4, x + 16, rs, None) == _lib.EPTQ_EINVAL                                   # x16 overlaps x
    assert r(x, 4100, 4, y, rs, None) == _lib.EPTQ_EUNSUPPORTED                                  # N % 8
    assert r(x, 16392, 4, y, rs, None) == _lib.EPTQ_EUNSUPPORTED                                 # N > 16384


def test_python_wrapper_raises_on_error_codes(lib):
    with pytest.raises(_lib.EptqError, match="eptq_e8d4_forward"):
        _lib.check(lib.eptq_e8d4_forward(*_fwd_args(Q=None)), "eptq_e8d4_forward")


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.EptqError, match="not built"):
        _lib.load(tmp_path / "missing.so")


def test_multi_entry_point_validates_every_layer(lib):
    L = _lib.EptqLayer
    good = L(16, 16, 16, None, None, 16, None, None, 0, 4, 0)
    arr = (L * 2)(good, L(16, 16, 16, None, None, 16, None, None, 0, 4, 32))
    f = lib.eptq_e8d4_forward_multi
    assert f(0, arr, 16, 0, 16, 0, 64, 1, 16, 64, None, 0, None) == _lib.EPTQ_EINVAL
    assert f(2, arr, 16, 0, 16, 0, 64, 1, 16, 48, None, 0, None) == _lib.EPTQ_EINVAL   # 2nd layer past ldy
    assert "outside a y row" in lib.eptq_last_error().decode()
    bad = (L * 2)(good, L(None, 16, 16, None, None, 16, None, None, 0, 4, 32))
    assert f(2, bad, 16, 0, 16, 0, 64, 1, 16, 64, None, 0, None) == _lib.EPTQ_EINVAL
    odd = (L * 2)(good, L(16, 16, 16, None, None, 16, None, None, 0, 4, 34))
    assert f(2, odd, 16, 0, 16, 0, 64, 1, 16, 72, None, 0, None) == _lib.EPTQ_EINVAL
    assert f(2, arr, 16, 0, None, 0, 64, 0, None, 64, None, 0, None) == _lib.EPTQ_OK   # B = 0
    assert f(2, arr, 16, 0, 16, 0, 64, 1, 16, 64, 8, 1024, None) == _lib.EPTQ_EINVAL   # work misaligned
    assert lib.eptq_e8d4_work_bytes() > 0


def test_llama_ops_reject_invalid_arguments(lib):
    assert lib.eptq_llama_rmsnorm(None, None, 16, 16, 1, 64, 1e-5, None) == 1
    assert lib.eptq_llama_rmsnorm(16, None, 16, 16, 1, 60, 1e-5, None) == 1
    assert lib.eptq_llama_rope_attn(16, 16, 16, 16, 16, 16, 16, 1, 4, 3, 128, 64, None, None) == 1   # H % Hk
    assert lib.eptq_llama_rope_attn(16, 16, 16, 16, 16, 16, 16, 1, 4, 4, 64, 64, None, None) == 1    # D != 128
    assert lib.eptq_llama_rope_attn(16, 16, 16, 16, 16, 16, 16, 1, 4, 4, 128, 2048, None, None) == 1  # L
    assert lib.eptq_llama_rope_attn(16, 16, 16, 16, 16, 16, 16, 1, 4, 4, 128, 64, 24, None) == 1    # work align
    assert lib.eptq_llama_attn_work_bytes(1, 32) == 32 * (16 * 130 * 4 + 4)
    assert lib.eptq_llama_attn_work_bytes(0, 32) == 0
    assert lib.eptq_llama_silu_mul(16, 16, 1, 12, None) == 1


def test_fused_llama_linears_validate_arguments(lib):
    L = _lib.EptqLayer
    arr = (L * 1)(L(16, 16, 16, None, None, 16, None, None, 0, 4, 0))
    f = lib.eptq_llama_norm_linear
    assert f(0, arr, 16, 16, None, 16, 1e-5, None, 64, 1, 16, 32, None) == _lib.EPTQ_EINVAL
    assert f(1, arr, 16, 16, None, None, 1e-5, None, 64, 1, 16, 32, None) == _lib.EPTQ_EINVAL   # no weight
    assert "norm weight" in lib.eptq_last_error().decode()
    assert f(1, arr, 16, 16, None, 16, 1e-5, 16, 64, 1, 16, 32, None) == _lib.EPTQ_EINVAL       # out == resid
    assert "overlaps" in lib.eptq_last_error().decode()
    assert f(1, arr, 16, 16, None, 16, 1e-5, None, 64, 9, 16, 32, None) == _lib.EPTQ_EUNSUPPORTED  # B > 8
    assert f(1, arr, 16, 24, None, 16, 1e-5, None, 64, 1, 16, 32, None) == _lib.EPTQ_EUNSUPPORTED  # misaligned
    assert f(1, arr, 16, 16, None, 16, 1e-5, None, 64, 0, 16, 32, None) == _lib.EPTQ_OK             # B = 0
    assert f(1, arr, 16, 16, None, 16, 1e-5, None, 64, 1, 16, 24, None) == _lib.EPTQ_EINVAL         # 8M > ldy
    pair = (L * 2)(L(16, 16, 16, None, None, 16, None, None, 0, 4, 0), L(16, 16, 16, None, None, 16, None, None, 0, 4, 0))
    g = lib.eptq_llama_norm_swiglu
    assert g(None, 16, 16, None, 16, 1e-5, None, 64, 1, 16, None) == _lib.EPTQ_EINVAL             # no layers
    assert g(pair, 16, 16, None, None, 1e-5, None, 64, 1, 16, None) == _lib.EPTQ_EINVAL           # no weight
    assert g(pair, 16, 16, None, 16, 1e-5, None, 64, 3, 16, None) == _lib.EPTQ_EUNSUPPORTED       # B > 2
    assert g(pair, 16, 16, None, 16, 1e-5, None, 64, 0, 16, None) == _lib.EPTQ_OK                 # B = 0
    pair[1].M = 8
    assert g(pair, 16, 16, None, 16, 1e-5, None, 64, 1, 16, None) == _lib.EPTQ_EINVAL             # M differ
    assert "differ" in lib.eptq_last_error().decode()
    pair[1].M = 4
    sw = lib.eptq_llama_linear_swiglu   # gate_up, codes, x, N, B, norm_w, eps, gu, out, work, work_bytes, stream
    assert sw(None, 16, 16, 64, 1, 16, 1e-5, 4096, 8192, 16, 1 << 20, None) == _lib.EPTQ_EINVAL   # no layers
    assert sw(pair, 16, 16, 64, 1, 16, 1e-5, 4096, 8192, None, 0, None) == _lib.EPTQ_EINVAL      # no work
    assert "workspace" in lib.eptq_last_error().decode()
    assert sw(pair, 16, 16, 64, 1, 16, 1e-5, 4096, 4096, 16, 1 << 20, None) == _lib.EPTQ_EINVAL  # out == gu
    assert sw(pair, 16, 16, 64, 1, 16, 1e-5, 4096, 8194, 16, 1 << 20, None) == _lib.EPTQ_EUNSUPPORTED  # out align
    assert sw(pair, 16, 16, 64, 0, 16, 1e-5, 4096, 8192, 16, 1 << 20, None) == _lib.EPTQ_OK      # B = 0
    pair[1].M = 8
    assert sw(pair, 16, 16, 64, 1, 16, 1e-5, 4096, 8192, 16, 1 << 20, None) == _lib.EPTQ_EINVAL  # M differ
    h = lib.eptq_llama_lm_head_argmax
    assert lib.eptq_llama_lm_head_work_bytes(2) >= 24
    assert h(None, None, 16, 1e-5, 16, 100, 4096, 1, 16, 16, None, 16, None) == 1          # null x
    assert h(16, None, 16, 1e-5, 16, 100, 4096, 1, 16, 16, None, 20, None) == 1            # work misaligned
    assert h(16, None, 16, 1e-5, 16, 100, 4096, 9, 16, 16, None, 16, None) == 2            # B > 8
    assert h(16, None, 16, 1e-5, 16, 100, 1000, 1, 16, 16, None, 16, None) == 2            # hidden size


def test_noalloc_checks_like_the_workspace_form(lib):
    """The allocation-free variant runs the same argument checks as
    eptq_e8d4_forward_multi, before it looks its scratch up (no device call
    for a refused or empty call), and sets no tile limit of its own: a call
    over more 64-row tiles than the scratch counts (4 x 4097 here) passes the
    checks and, on a GPU, runs unsplit."""
    L = _lib.EptqLayer
    four = (L * 4)(*([L(16, 16, 16, None, None, 16, None, None, 0, 32769, 0)] * 4))
    fm, na = lib.eptq_e8d4_forward_multi, lib.eptq_e8d4_forward_multi_noalloc
    cases = [
        (0, four, 16, 16, 64, 1, 16, 8 * 32769, _lib.EPTQ_EINVAL),          # no layers
        (4, four, 16, 16, 64, -1, 16, 8 * 32769, _lib.EPTQ_EINVAL),         # B < 0
        (4, four, 16, 8, 64, 1, 16, 8 * 32769, _lib.EPTQ_EUNSUPPORTED),     # x misaligned
        (4, four, 16, 16, 60, 1, 16, 8 * 32769, _lib.EPTQ_EUNSUPPORTED),    # N % 8
        (4, four, 16, 16, 64, 1, 16, 8 * 32768, _lib.EPTQ_EINVAL),          # layer outside y's row
        (4, four, 16, 16, 64, 0, 16, 8 * 32769, _lib.EPTQ_OK),              # B = 0: nothing to do
    ]
    for n, ls, codes, x, N, B, y, ldy, want in cases:
        rc_w = fm(n, ls, codes, _lib.EPTQ_F16, x, _lib.EPTQ_F16, N, B, y, ldy, None, 0, None)
        msg_w = lib.eptq_last_error().decode()
        rc_n = na(n, ls, codes, _lib.EPTQ_F16, x, _lib.EPTQ_F16, N, B, y, ldy, None)
        msg_n = lib.eptq_last_error().decode()
        assert rc_w == rc_n == want, (n, N, B, ldy, rc_w, rc_n)
        if want:
            assert msg_n.replace("_noalloc", "") == msg_w, (msg_w, msg_n)
