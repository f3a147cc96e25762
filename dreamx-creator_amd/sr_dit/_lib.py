"""ctypes binding of ``libsrdit_hip.so`` (the C ABI in ``include/srdit_hip.h``).

The library is built in-tree next to this file by ``sr_dit.build``.  Loading
fails loudly when it is missing: there is no CPU or PyTorch fallback for any
entry point.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_NAME = "libsrdit_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

SRDIT_OK = 0
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1}

_c_int, _c_i64, _c_f, _c_p = ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_void_p

#: Every exported entry point with its (restype, argtypes).
SIGNATURES = {
    "srdit_window_attn_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                       _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                       _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_int,
                                       _c_int, _c_p]),
    "srdit_fp8_quant_rowwise": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p]),
    "srdit_fp8_quant_tensor": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_p, _c_p, _c_p]),
    "srdit_fp8_gemm": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "srdit_last_error": (_c_int, [ctypes.c_char_p, _c_int]),
    "srdit_version": (_c_int, []),
    "srdit_copy_bytes": (_c_int, [_c_p, _c_p, _c_i64, _c_p]),
}

_LIB = None


def load():
    """Load the library once; raise ``RuntimeError`` if it is not built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_NAME} is not built at {LIB_PATH}; run __graft_entry__.build() "
                "(hipcc --offload-arch=gfx950).  There is no fallback path.")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = lib
    return _LIB


def last_error() -> str:
    buf = ctypes.create_string_buffer(512)
    load().srdit_last_error(buf, 512)
    return buf.value.decode(errors="replace")


def _check(rc: int, what: str):
    if rc != SRDIT_OK:
        raise RuntimeError(f"{what} failed (status {rc}): {last_error()}")


def _ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def _stream(device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def window_attn_fwd(q, k, v, o, params, order, *, n_w, m_tiles, p_stride, hr_base,
                    H, W, n_heads, head_dim, kv_tokens, scale, mode):
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"window attention needs bf16 or fp16, got {q.dtype}")
    rc = load().srdit_window_attn_fwd(
        _ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(params), _ptr(order),
        int(n_w), int(m_tiles), int(p_stride), int(hr_base), int(H), int(W),
        int(q.shape[0]), int(kv_tokens), int(n_heads), int(head_dim), float(scale),
        int(mode), DTYPE_CODES[q.dtype], _stream(q.device))
    _check(rc, "srdit_window_attn_fwd")


def fp8_quant_rowwise(x, xq, scale):
    M, K = x.shape
    rc = load().srdit_fp8_quant_rowwise(_ptr(x), M, K, x.stride(0), _ptr(xq), _ptr(scale),
                                        _stream(x.device))
    _check(rc, "srdit_fp8_quant_rowwise")


def fp8_quant_tensor(x, xq, scale, amax_ws):
    M, K = x.shape
    rc = load().srdit_fp8_quant_tensor(_ptr(x), M, K, x.stride(0), _ptr(xq), _ptr(scale),
                                       _ptr(amax_ws), _stream(x.device))
    _check(rc, "srdit_fp8_quant_tensor")


def fp8_gemm(a, b, sa, sb, bias, out):
    M, K = a.shape
    N = b.shape[0]
    rc = load().srdit_fp8_gemm(_ptr(a), _ptr(b), _ptr(sa), int(sa.numel()), _ptr(sb),
                               int(sb.numel()), _ptr(bias), _ptr(out), M, N, K,
                               out.stride(0), _stream(a.device))
    _check(rc, "srdit_fp8_gemm")


def copy_bytes(src, dst, nbytes):
    rc = load().srdit_copy_bytes(_ptr(src), _ptr(dst), int(nbytes), _stream(src.device))
    _check(rc, "srdit_copy_bytes")
