"""C ABI (CPU): the library loads and exports every entry point the header declares.

No compute calls here (there is no GPU in the build container); argument
validation that fails before any HIP call is exercised, since it returns an
error status without touching a device.
"""
import ctypes
import os
import re

import pytest

from sr_dit import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "srdit_hip.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\bint\s+(srdit_\w+)\s*\(", text)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ("srdit_window_attn_fwd", "srdit_fp8_quant_rowwise", "srdit_fp8_quant_tensor",
                 "srdit_fp8_gemm", "srdit_last_error", "srdit_version", "srdit_copy_bytes"):
        assert must in names


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert set(declared_functions()) == set(_lib.SIGNATURES)


def test_version_and_error_buffer():
    lib = _lib.load()
    assert lib.srdit_version() >= 100
    buf = ctypes.create_string_buffer(8)
    n = lib.srdit_last_error(buf, 8)
    assert n >= 0 and len(buf.value) <= 7


def test_window_attn_rejects_null_and_bad_mode_without_gpu():
    lib = _lib.load()
    rc = lib.srdit_window_attn_fwd(None, None, None, None, None, None, 1, 1, 19, 0, 1, 1,
                                   1, 1, 1, 128, 1.0, 0, 0, None)
    assert rc == 1 and "null" in _lib.last_error()
    fake = ctypes.c_void_p(4096)   # aligned, never dereferenced: validation fails first
    rc = lib.srdit_window_attn_fwd(fake, fake, fake, fake, fake, fake, 1, 1, 19, 0, 1, 1,
                                   1, 1, 1, 128, 1.0, 2, 0, None)
    assert rc == 1 and "mode" in _lib.last_error()
    rc = lib.srdit_window_attn_fwd(fake, fake, fake, fake, fake, fake, 1, 1, 17, 0, 1, 1,
                                   1, 1, 1, 128, 1.0, 0, 0, None)
    assert rc == 1 and "p_stride" in _lib.last_error()
    rc = lib.srdit_window_attn_fwd(fake, fake, fake, fake, fake, fake, 1, 1, 19, 0, 1, 1,
                                   1, 1, 1, 96, 1.0, 0, 0, None)
    assert rc == 3 and "head_dim" in _lib.last_error()
    rc = lib.srdit_window_attn_fwd(ctypes.c_void_p(4098), fake, fake, fake, fake, fake, 1, 1, 19,
                                   0, 1, 1, 1, 1, 1, 128, 1.0, 0, 0, None)
    assert rc == 1 and "aligned" in _lib.last_error()


def test_copy_rejects_misaligned_size():
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    assert lib.srdit_copy_bytes(fake, fake, 15, None) == 1


def test_grouped_window_rejects_a_q_span_past_2_31_without_gpu():
    # 400,000 query tokens x 24 heads x 128 x 2 bytes > 2^31 while the K/V span
    # (1,000 tokens) passes: refused before any HIP call
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    rc = lib.srdit_window_attn_grouped_fwd(fake, fake, fake, fake, fake, fake, 1, 1, 0, 1, 1,
                                           400000, 1000, 24, 128, 0.088, 0, None)
    assert rc == 1 and "Q/O" in _lib.last_error()


def test_gemm_rejects_bad_layouts_without_gpu():
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    # ldo must be a multiple of 8 (the output leaves as 16-byte row pieces)
    rc = lib.srdit_fp8_gemm(fake, fake, fake, 1, fake, 1, None, fake, 64, 32, 256, 36, None)
    assert rc == 1 and "ldo" in _lib.last_error()
    # the bias reaches LDS by 16-byte DMAs
    rc = lib.srdit_fp8_gemm(fake, fake, fake, 1, fake, 1, ctypes.c_void_p(4104), fake, 64, 32,
                            256, 32, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    # per-tensor scales may sit anywhere; per-row ones must be 16-byte aligned
    rc = lib.srdit_fp8_gemm(fake, fake, ctypes.c_void_p(4100), 64, fake, 1, None, fake, 64, 32,
                            256, 32, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    rc = lib.srdit_fp8_gemm(fake, fake, fake, 1, fake, 1, None, fake, 64, 32, 200, 32, None)
    assert rc == 1 and "K=200" in _lib.last_error()


def test_dense_linears_reject_bad_layouts_without_gpu():
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    # bf16 linear: K a multiple of 16, rows 16-byte aligned, epilogue 0 or 1
    rc = lib.srdit_bf16_linear(fake, 40, fake, 40, None, fake, 64, 8, 64, 40, 0, None)
    assert rc == 1 and "K=40" in _lib.last_error()
    rc = lib.srdit_bf16_linear(fake, 36, fake, 32, None, fake, 64, 8, 64, 32, 0, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    rc = lib.srdit_bf16_linear(fake, 32, fake, 32, None, fake, 64, 8, 64, 32, 2, None)
    assert rc == 1 and "epilogue" in _lib.last_error()
    # the modulated fp32 linear: weights bf16 or fp32, modulation vectors 16-byte aligned
    rc = lib.srdit_linear_f32_modulated(fake, 64, fake, fake, fake, 64, None, 1, fake, 64, 8, 64,
                                        64, None)
    assert rc == 1 and "w_dtype" in _lib.last_error()
    rc = lib.srdit_linear_f32_modulated(fake, 64, ctypes.c_void_p(4100), fake, fake, 64, None, 2,
                                        fake, 64, 8, 64, 64, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    # the GEMV: K a multiple of 8, leading dimensions cover the rows
    rc = lib.srdit_gemv_f32(fake, 12, fake, 12, None, 0, fake, 4, 1, 4, 12, None)
    assert rc == 1 and "K=12" in _lib.last_error()
    rc = lib.srdit_gemv_f32(fake, 8, fake, 16, None, 0, fake, 2, 1, 4, 16, None)
    assert rc == 1 and "leading" in _lib.last_error()


def test_gemm_with_workspace_rejects_bad_arguments_without_gpu():
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    args = (fake, fake, fake, 1, fake, 1, None, fake, 1024, 3072, 3072, 3072, 0, None)
    # the workspace of the split-K tail is read by 16-byte loads
    rc = lib.srdit_fp8_gemm_ws(*args, 0, 0, ctypes.c_void_p(4104), _lib.GEMM_WS_BYTES, None)
    assert rc == 1 and "workspace" in _lib.last_error()
    rc = lib.srdit_fp8_gemm_ws(*args, -256, 0, fake, _lib.GEMM_WS_BYTES, None)
    assert rc == 1 and "split_n" in _lib.last_error()
    # the output-split rules of srdit_fp8_gemm_split hold here too
    rc = lib.srdit_fp8_gemm_ws(*args, 1000, 1024 * 3072, fake, _lib.GEMM_WS_BYTES, None)
    assert rc == 1 and "split_n" in _lib.last_error()


def test_gemm_workspace_size_matches_the_header():
    text = open(os.path.join(os.path.dirname(__file__), "..", "include", "srdit_hip.h")).read()
    m = re.search(r"#define SRDIT_GEMM_WS_BYTES \(\(int64_t\)(\d+) \+ \(int64_t\)(\d+) \* (\d+)\)",
                  text)
    assert m, "SRDIT_GEMM_WS_BYTES not found"
    assert int(m.group(1)) + int(m.group(2)) * int(m.group(3)) == _lib.GEMM_WS_BYTES


def test_dense_attention_rejects_bad_arguments_without_gpu():
    lib = _lib.load()
    fake = ctypes.c_void_p(4096)
    rc = lib.srdit_dense_attn_fwd(fake, fake, fake, ctypes.c_void_p(4100), 100, 512, 24, 128,
                                  0.088, None, 0, None)
    assert rc == 1 and "aligned" in _lib.last_error()
    rc = lib.srdit_dense_attn_fwd(fake, fake, fake, fake, 100, 0, 24, 128, 0.088, None, 0, None)
    assert rc == 1 and "kv_tokens" in _lib.last_error()
    rc = lib.srdit_dense_attn_fwd(fake, fake, fake, fake, 100, 512, 24, 96, 0.088, None, 0, None)
    assert rc == 3 and "head_dim" in _lib.last_error()
    rc = lib.srdit_dense_attn_fwd(fake, fake, fake, fake, 1 << 20, 512, 24, 128, 0.088, None, 0,
                                  None)
    assert rc == 1 and "2^31" in _lib.last_error()
