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
