"""The C-ABI library loads and exports every symbol include/sfl.h declares (no GPU calls)."""

import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


def declared_symbols():
    text = (ROOT / "include" / "sfl.h").read_text()
    return sorted(set(re.findall(r"\b(sfl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_entry_points():
    names = declared_symbols()
    assert "sfl_decode_attention" in names and "sfl_last_error" in names


def test_library_exports_every_declared_symbol():
    from systems_for_llms_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libsfl.so not built (run __graft_entry__.build())")
    handle = _lib.lib()
    missing = [name for name in declared_symbols() if not hasattr(handle, name)]
    assert not missing
    assert handle.sfl_version().decode().startswith("sfl")
    assert set(_lib.SIGNATURES) <= set(declared_symbols())


def test_argument_errors_are_reported_without_a_launch():
    import ctypes

    from systems_for_llms_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libsfl.so not built")
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("sfl_decode_attention", None, None, None, None, None, None, None, None,
                  1, 1, 1, 1, 64, 1, 0.125, 1, 1, 1, None)
    buf = ctypes.create_string_buffer(64)
    p = ctypes.addressof(buf)
    with pytest.raises(RuntimeError, match="divisible"):
        _lib.call("sfl_decode_attention", p, p, p, p, p, p, p, p, 1, 3, 2, 16, 64, 1, 0.125, 1, 1, 1, None)
    with pytest.raises(RuntimeError, match="head dim"):
        _lib.call("sfl_decode_attention", p, p, p, p, p, p, p, p, 1, 2, 2, 16, 48, 1, 0.125, 1, 1, 1, None)


def test_folded_norm_entry_points_reject_bad_arguments_without_a_launch():
    """Every call here fails an argument check before anything reaches HIP."""
    import ctypes

    from systems_for_llms_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libsfl.so not built")
    buf = ctypes.create_string_buffer(256)
    p = (ctypes.addressof(buf) + 15) // 16 * 16  # 16-byte aligned host address (never dereferenced)
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("sfl_gemm_residual_norm", p, p, p, 64, 128, 64, None, p, p, 1, None)
    with pytest.raises(RuntimeError, match="multiple of 4"):
        _lib.call("sfl_gemm_residual_norm", p, p, p, 64, 130, 64, p, p, p, 1, None)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.call("sfl_gemm_residual_norm", p, p, p, 64, 128, 72, p, p, p, 1, None)
    with pytest.raises(RuntimeError, match="16-byte"):
        _lib.call("sfl_gemm_residual_norm", p, p, p + 4, 64, 128, 64, p, p, p, 1, None)
    with pytest.raises(RuntimeError, match="sizes must be positive"):
        _lib.call("sfl_norm_scale", p, 0, 64, 128, p, None)
    with pytest.raises(RuntimeError, match="dtype must be BF16 or F16"):
        _lib.call("sfl_rmsnorm_rows_scaled", p, p, p, p, 4, 128, 0, None)
    with pytest.raises(RuntimeError, match="dtype must be F32, BF16 or F16"):
        _lib.call("sfl_gemm", p, p, p, 64, 128, 64, 5, 0, 0, None)
    with pytest.raises(RuntimeError, match="F32 inputs need an F32 output"):
        _lib.call("sfl_gemm", p, p, p, 64, 128, 64, 0, 1, 0, None)
    with pytest.raises(RuntimeError, match="head dim must be 16, 32, 64 or 128"):
        s3 = (ctypes.c_long * 3)(0, 0, 64)
        _lib.call("sfl_causal_attention_f32", p, p, p, p, 1, 1, 8, 48, s3, s3, s3, s3, 0.1, None)
    with pytest.raises(RuntimeError, match="output dtype must be F32 or the input dtype"):
        _lib.call("sfl_gemm", p, p, p, 64, 128, 64, 2, 1, 0, None)
    with pytest.raises(RuntimeError, match="at most 2048"):
        _lib.call("sfl_rmsnorm_rows_scaled", p, p, p, p, 4, 4096, 1, None)
    with pytest.raises(RuntimeError, match="null pointer"):
        _lib.call("sfl_gemm_qkv_rope_scaled", p, p, None, 64, 64, 128, 2, p, p, p, p, p, 64, 1, None)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.call("sfl_gemm_qkv_rope_scaled", p, p, p, 64, 64, 96, 2, p, p, p, p, p, 64, 1, None)
    with pytest.raises(RuntimeError, match="batch \\* seq"):
        _lib.call("sfl_gemm_qkv_rope_scaled", p, p, p, 65, 64, 128, 2, p, p, p, p, p, 64, 1, None)
    with pytest.raises(RuntimeError, match="multiple of 8"):
        _lib.call("sfl_gemm_swiglu_scaled", p, p, p, p, 64, 100, 128, 1, None)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        _lib.call("sfl_gemm_swiglu_scaled", p, p, p, p, 64, 128, 72, 1, None)
