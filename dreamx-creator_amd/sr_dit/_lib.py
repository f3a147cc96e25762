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
    "srdit_window_attn_grouped_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int, _c_int,
                                               _c_int, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                               _c_int, _c_f, _c_int, _c_p]),
    "srdit_window_attn_fwd_ex": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                          _c_int, _c_int, _c_int, _c_int, _c_int, _c_int,
                                          _c_i64, _c_i64, _c_int, _c_int, _c_f, _c_int,
                                          _c_int, _c_int, _c_p, _c_p, _c_int, _c_p]),
    "srdit_window_attn_grouped_fwd_ex": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int,
                                                  _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64,
                                                  _c_int, _c_int, _c_f, _c_int, _c_int, _c_p,
                                                  _c_p, _c_int, _c_int, _c_int, _c_p]),
    "srdit_window_attn_packed_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_int,
                                              _c_int, _c_int, _c_int, _c_int, _c_i64, _c_i64,
                                              _c_int, _c_int, _c_f, _c_int, _c_int, _c_p,
                                              _c_p, _c_int, _c_p]),
    "srdit_dense_attn_fwd": (_c_int, [_c_p, _c_p, _c_p, _c_p, _c_i64, _c_i64, _c_int, _c_int,
                                      _c_f, _c_p, _c_int, _c_p]),
    "srdit_fp8_quant_rowwise": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p]),
    "srdit_fp8_quant_tensor": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p,
                                        _c_p]),
    "srdit_fp8_gemm": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "srdit_fp8_gemm_ex": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p]),
    "srdit_fp8_gemm_split": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                      _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "srdit_fp8_gemm_ws": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p,
                                   _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_i64, _c_i64,
                                   _c_p, _c_i64, _c_p]),
    "srdit_fp8_quant_apply": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p, _c_p,
                                       _c_p]),
    "srdit_fp8_quant_tensor_gelu": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64, _c_p,
                                             _c_p, _c_p, _c_p]),
    "srdit_fp8_quant_tensor_gelu_ex": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_p, _c_i64,
                                                _c_p, _c_p, _c_p, _c_p, _c_p]),
    "srdit_ln_modulate": (_c_int, [_c_p, _c_i64, _c_int, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_f,
                                   _c_p, _c_i64, _c_p, _c_p]),
    "srdit_residual_gate": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_int, _c_i64, _c_i64, _c_p,
                                     _c_i64, _c_p]),
    "srdit_residual_ln_modulate": (_c_int, [_c_p, _c_p, _c_p, _c_i64, _c_int, _c_i64, _c_i64,
                                            _c_p, _c_i64, _c_p, _c_p, _c_p, _c_p, _c_f, _c_p,
                                            _c_i64, _c_p, _c_p]),
    "srdit_rmsnorm_rope": (_c_int, [_c_p, _c_i64, _c_int, _c_i64, _c_p, _c_f, _c_p, _c_int, _c_p,
                                    _c_p]),
    "srdit_bf16_linear": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_p, _c_i64, _c_i64,
                                   _c_i64, _c_i64, _c_int, _c_p]),
    "srdit_linear_f32_modulated": (_c_int, [_c_p, _c_i64, _c_p, _c_p, _c_p, _c_i64, _c_p, _c_int,
                                            _c_p, _c_i64, _c_i64, _c_i64, _c_i64, _c_p]),
    "srdit_gemv_f32": (_c_int, [_c_p, _c_i64, _c_p, _c_i64, _c_p, _c_int, _c_p, _c_i64, _c_i64,
                                _c_i64, _c_i64, _c_p]),
    "srdit_last_error": (_c_int, [ctypes.c_char_p, _c_int]),
    "srdit_version": (_c_int, []),
    "srdit_copy_bytes": (_c_int, [_c_p, _c_p, _c_i64, _c_p]),
    "srdit_fp8_linear_tensor_static": (_c_int, [_c_p, _c_i64, _c_i64, _c_i64, _c_int, _c_p, _c_p,
                                                _c_i64, _c_p, _c_p, _c_i64, _c_i64, _c_p]),
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


def _ex_args(ring, amax_out):
    """Trailing arguments of the _ex entry points: ``ring`` = (ring_frames,
    ring_cached, head) with ``head`` a device int32 tensor, or None;
    ``amax_out`` a device int32 [1] word, or None."""
    if ring is None:
        R, nc, head = 0, 0, None
    else:
        R, nc, head = ring
        if not (torch.is_tensor(head) and head.dtype == torch.int32 and head.is_cuda
                and head.numel() >= 1):
            raise ValueError("ring head must be a device int32 tensor")
    if amax_out is not None and not (amax_out.dtype == torch.int32 and amax_out.is_cuda):
        raise ValueError("amax_out must be a device int32 word")
    return int(R), int(nc), _ptr(head), _ptr(amax_out)


def window_attn_fwd(q, k, v, o, params, order, *, n_w, m_tiles, p_stride, hr_base,
                    H, W, n_heads, head_dim, kv_tokens, scale, mode, ring=None, amax_out=None):
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"window attention needs bf16 or fp16, got {q.dtype}")
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(params), _ptr(order),
            int(n_w), int(m_tiles), int(p_stride), int(hr_base), int(H), int(W),
            int(q.shape[0]), int(kv_tokens), int(n_heads), int(head_dim), float(scale),
            int(mode))
    tail = (DTYPE_CODES[q.dtype], _stream(q.device))
    if ring is None and amax_out is None:
        _check(load().srdit_window_attn_fwd(*args, *tail), "srdit_window_attn_fwd")
    else:
        _check(load().srdit_window_attn_fwd_ex(*args, *_ex_args(ring, amax_out), *tail),
               "srdit_window_attn_fwd_ex")


def window_attn_grouped_fwd(q, k, v, o, params, groups, *, n_w, n_groups, hr_base, H, W,
                            n_heads, head_dim, kv_tokens, scale, ring=None, amax_out=None,
                            members=2, anchor_mode=0):
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"window attention needs bf16 or fp16, got {q.dtype}")
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(params), _ptr(groups),
            int(n_w), int(n_groups), int(hr_base), int(H), int(W), int(q.shape[0]),
            int(kv_tokens), int(n_heads), int(head_dim), float(scale))
    tail = (DTYPE_CODES[q.dtype], _stream(q.device))
    if ring is None and amax_out is None and members == 2 and anchor_mode == 0:
        _check(load().srdit_window_attn_grouped_fwd(*args, *tail),
               "srdit_window_attn_grouped_fwd")
    else:
        _check(load().srdit_window_attn_grouped_fwd_ex(*args, *_ex_args(ring, amax_out),
                                                       int(members), int(anchor_mode), *tail),
               "srdit_window_attn_grouped_fwd_ex")


def window_attn_packed_fwd(q, k, v, o, params, tiles, *, n_w, hr_base, H, W, n_heads, head_dim,
                           kv_tokens, scale, ring=None, amax_out=None):
    """The one-member window kernel over packed tiles (``blockgrid_hip.build_packed``:
    int32 [T, 5], a tile holding the queries of one or two windows)."""
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"window attention needs bf16 or fp16, got {q.dtype}")
    if (tiles.dim() != 2 or tiles.shape[1] != 5 or tiles.dtype != torch.int32
            or not tiles.is_cuda or not tiles.is_contiguous()):
        raise ValueError("window_attn_packed_fwd: tiles must be a contiguous device int32 [T, 5]")
    args = (_ptr(q), _ptr(k), _ptr(v), _ptr(o), _ptr(params), _ptr(tiles),
            int(n_w), int(tiles.shape[0]), int(hr_base), int(H), int(W), int(q.shape[0]),
            int(kv_tokens), int(n_heads), int(head_dim), float(scale))
    _check(load().srdit_window_attn_packed_fwd(*args, *_ex_args(ring, amax_out),
                                               DTYPE_CODES[q.dtype], _stream(q.device)),
           "srdit_window_attn_packed_fwd")


def dense_attn_fwd(q, k, v, o, scale, amax_out=None):
    """Every query of ``q`` [Lq, H, D] attends every key of ``k``/``v`` [Lkv, H, D]
    of its head into ``o`` [Lq, H, D] (srdit_dense_attn_fwd); ``amax_out``
    (int32 [1], nullable) receives the bits of max |o|."""
    if q.dtype not in DTYPE_CODES:
        raise ValueError(f"dense attention needs bf16 or fp16, got {q.dtype}")
    for name, t in (("q", q), ("k", k), ("v", v), ("o", o)):
        if t.dim() != 3 or not t.is_contiguous() or t.dtype != q.dtype or t.device != q.device:
            raise ValueError(f"dense_attn_fwd: {name} must be a contiguous 3-D {q.dtype} tensor "
                             f"on {q.device}")
    if k.shape != v.shape or k.shape[1:] != q.shape[1:] or o.shape != q.shape:
        raise ValueError(f"dense_attn_fwd: shapes q {tuple(q.shape)}, k {tuple(k.shape)}, "
                         f"v {tuple(v.shape)}, o {tuple(o.shape)} do not match")
    _check(load().srdit_dense_attn_fwd(_ptr(q), _ptr(k), _ptr(v), _ptr(o), int(q.shape[0]),
                                       int(k.shape[0]), int(q.shape[1]), int(q.shape[2]),
                                       float(scale), _ptr(amax_out), DTYPE_CODES[q.dtype],
                                       _stream(q.device)),
           "srdit_dense_attn_fwd")


QUANT_DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}


def _quant_args(x, xq):
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError(f"fp8 quantiser needs a 2-D input with unit column stride, got "
                         f"shape {tuple(x.shape)} strides {x.stride()}")
    if x.dtype not in QUANT_DTYPE_CODES:
        raise ValueError(f"fp8 quantiser input must be bf16, fp16 or fp32, got {x.dtype}")
    if xq.dtype != torch.float8_e4m3fn or tuple(xq.shape) != tuple(x.shape) or not xq.is_contiguous():
        raise ValueError("fp8 quantiser output must be a contiguous float8_e4m3fn tensor "
                         "shaped like the input")
    M, K = x.shape
    return M, K, x.stride(0), QUANT_DTYPE_CODES[x.dtype]


def fp8_quant_rowwise(x, xq, scale):
    M, K, ldx, dt = _quant_args(x, xq)
    if scale.dtype != torch.float32 or scale.numel() != M:
        raise ValueError(f"row-wise scale must be {M} float32 values")
    rc = load().srdit_fp8_quant_rowwise(_ptr(x), M, K, ldx, dt, _ptr(xq), _ptr(scale),
                                        _stream(x.device))
    _check(rc, "srdit_fp8_quant_rowwise")


def fp8_quant_tensor(x, xq, scale, amax_ws):
    M, K, ldx, dt = _quant_args(x, xq)
    if scale.dtype != torch.float32 or scale.numel() != 1:
        raise ValueError("per-tensor scale must be one float32 value")
    if amax_ws.numel() * amax_ws.element_size() < 4:
        raise ValueError("amax workspace must hold at least 4 bytes")
    rc = load().srdit_fp8_quant_tensor(_ptr(x), M, K, ldx, dt, _ptr(xq), _ptr(scale),
                                       _ptr(amax_ws), _stream(x.device))
    _check(rc, "srdit_fp8_quant_tensor")


def fp8_gemm(a, b, sa, sb, bias, out):
    """out[M, N] (bf16, unit column stride) = a[M, K] . b[N, K]^T * sa * sb + bias."""
    for name, t in (("a", a), ("b", b)):
        if t.dtype != torch.float8_e4m3fn or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"fp8_gemm: {name} must be a contiguous 2-D float8_e4m3fn tensor")
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"fp8_gemm: inner dims differ ({K} vs {b.shape[1]})")
    for name, t in (("sa", sa), ("sb", sb)):
        if t.dtype != torch.float32 or not t.is_contiguous():
            raise ValueError(f"fp8_gemm: {name} must be contiguous float32")
    if bias is not None and (bias.dtype != torch.bfloat16 or bias.numel() != N
                             or not bias.is_contiguous()):
        raise ValueError(f"fp8_gemm: bias must be {N} contiguous bf16 values")
    if out.dtype != torch.bfloat16 or out.dim() != 2 or tuple(out.shape) != (M, N) \
            or out.stride(1) != 1:
        raise ValueError(f"fp8_gemm: out must be bf16 [{M}, {N}] with unit column stride")
    rc = load().srdit_fp8_gemm(_ptr(a), _ptr(b), _ptr(sa), int(sa.numel()), _ptr(sb),
                               int(sb.numel()), _ptr(bias), _ptr(out), M, N, K,
                               out.stride(0), _stream(a.device))
    _check(rc, "srdit_fp8_gemm")


#: epilogue flag of srdit_fp8_gemm_ex kept for old callers; it has no effect
#: (every GEMM runs on the hand-written MFMA kernel)
GEMM_MFMA = 0x100
#: epilogue flag of srdit_fp8_gemm_ex: amax_out receives the largest positive
#: output (for srdit_fp8_quant_tensor_gelu_ex) instead of max |out|
GEMM_AMAX_POS = 0x200


#: bytes of a split-K workspace of srdit_fp8_gemm_ws (SRDIT_GEMM_WS_BYTES)
GEMM_WS_BYTES = 4096 + 256 * 262144
_GEMM_WS = {}


def gemm_workspace(device, stream=None):
    """The split-K workspace of srdit_fp8_gemm_ws for ``stream`` (default: the
    current stream of ``device``): GEMM_WS_BYTES of device memory whose first
    4096 bytes (the arrival counters) are zeroed once, kept for the stream.  None
    while that stream is captured and has none yet (a graph must not own it):
    its GEMMs then run unsplit.  ``capture_stream`` gives a stream that has one."""
    device = torch.device(device)
    if device.index is None:
        device = torch.device("cuda", torch.cuda.current_device())
    s = stream if stream is not None else torch.cuda.current_stream(device)
    key = (device.index, s.cuda_stream)
    ws = _GEMM_WS.get(key)
    if ws is None:
        if torch.cuda.is_current_stream_capturing():
            return None
        with torch.cuda.stream(s):
            ws = torch.empty(GEMM_WS_BYTES, dtype=torch.uint8, device=device)
            ws[:4096].zero_()
        _GEMM_WS[key] = ws
    return ws


_CAPTURE_STREAMS = {}


def capture_stream(device):
    """A side stream of ``device`` for graph capture (torch.cuda.graph(...,
    stream=)), one per device, whose GEMM workspace exists before the capture."""
    device = torch.device(device)
    idx = device.index if device.index is not None else torch.cuda.current_device()
    s = _CAPTURE_STREAMS.get(idx)
    if s is None:
        s = _CAPTURE_STREAMS[idx] = torch.cuda.Stream(torch.device("cuda", idx))
        gemm_workspace(torch.device("cuda", idx), s)
        s.synchronize()
    return s


def _gemm_ws(a, out, M, N, K, ldo, epilogue, amax_out, split_n, split_stride, sa, sb, bias, b,
             who):
    ws = gemm_workspace(a.device)
    rc = load().srdit_fp8_gemm_ws(_ptr(a), _ptr(b), _ptr(sa), int(sa.numel()), _ptr(sb),
                                  int(sb.numel()), _ptr(bias), _ptr(out), M, N, K, ldo,
                                  int(epilogue), _ptr(amax_out), split_n, split_stride,
                                  _ptr(ws), 0 if ws is None else ws.numel(), _stream(a.device))
    _check(rc, who)


def fp8_gemm_ex(a, b, sa, sb, bias, out, *, epilogue=0, amax_out=None, split_tail=True):
    """fp8_gemm with an epilogue (0 none, 1 GELU-tanh) and an optional amax word
    (cleared by the call, then the bits of max |out|).  ``split_tail``: a last
    round of tiles less than half full runs split along K (srdit_fp8_gemm_ws,
    with this stream's workspace); the results differ from the unsplit GEMM's
    only in the fp32 summation order."""
    M, K = a.shape
    N = b.shape[0]
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"fp8_gemm_ex: out must be bf16 [{M}, {N}] with unit column stride")
    if split_tail:
        _gemm_ws(a, out, M, N, K, out.stride(0), epilogue, amax_out, 0, 0, sa, sb, bias, b,
                 "srdit_fp8_gemm_ws")
        return
    rc = load().srdit_fp8_gemm_ex(_ptr(a), _ptr(b), _ptr(sa), int(sa.numel()), _ptr(sb),
                                  int(sb.numel()), _ptr(bias), _ptr(out), M, N, K, out.stride(0),
                                  int(epilogue), _ptr(amax_out), _stream(a.device))
    _check(rc, "srdit_fp8_gemm_ex")


def fp8_gemm_split(a, b, sa, sb, bias, out, *, split_tail=True):
    """a [M, K] . b [N, K]^T * sa * sb + bias with the output split into blocks:
    ``out`` [G, M, N / G] bf16 (contiguous) receives columns [j N/G, (j+1) N/G)
    in ``out[j]``.  ``split_tail`` as fp8_gemm_ex."""
    for name, t in (("a", a), ("b", b)):
        if t.dtype != torch.float8_e4m3fn or t.dim() != 2 or not t.is_contiguous():
            raise ValueError(f"fp8_gemm_split: {name} must be a contiguous 2-D float8_e4m3fn tensor")
    M, K = a.shape
    N = b.shape[0]
    if b.shape[1] != K:
        raise ValueError(f"fp8_gemm_split: inner dims differ ({K} vs {b.shape[1]})")
    if out.dtype != torch.bfloat16 or out.dim() != 3 or not out.is_contiguous() \
            or out.shape[1] != M or out.shape[0] * out.shape[2] != N:
        raise ValueError(f"fp8_gemm_split: out must be contiguous bf16 [G, {M}, {N} / G]")
    G, _, W = out.shape
    if split_tail:
        _gemm_ws(a, out, M, N, K, W, 0, None, W, M * W, sa, sb, bias, b, "srdit_fp8_gemm_ws")
        return
    rc = load().srdit_fp8_gemm_split(_ptr(a), _ptr(b), _ptr(sa), int(sa.numel()), _ptr(sb),
                                     int(sb.numel()), _ptr(bias), _ptr(out), M, N, K, W, W,
                                     M * W, _stream(a.device))
    _check(rc, "srdit_fp8_gemm_split")


#: capacity of the static scratch of srdit_fp8_linear_tensor_static (activation codes)
LINEAR_SCRATCH_CODES = 64 << 20


def fp8_linear_tensor_static(x, w, w_scale, bias, out):
    """The per-tensor fp8 Linear with no caller workspace and no allocation:
    out [M, N] bf16 = quantise(x [M, K]) . w [N, K]^T * scales + bias, the
    activation's amax, scale and codes in the library's static per-device scratch
    (M*K <= LINEAR_SCRATCH_CODES).  Calls that overlap on one device race."""
    if x.dim() != 2 or x.stride(1) != 1 or x.dtype not in (torch.bfloat16, torch.float16,
                                                            torch.float32):
        raise ValueError("fp8_linear_tensor_static: x must be 2-D bf16/fp16/fp32 with unit "
                         "column stride")
    if w.dtype != torch.float8_e4m3fn or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("fp8_linear_tensor_static: w must be a contiguous 2-D float8_e4m3fn tensor")
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K:
        raise ValueError(f"fp8_linear_tensor_static: inner dims differ ({K} vs {w.shape[1]})")
    if w_scale.dtype != torch.float32 or not w_scale.is_contiguous():
        raise ValueError("fp8_linear_tensor_static: w_scale must be contiguous float32")
    if out.dtype != torch.bfloat16 or tuple(out.shape) != (M, N) or out.stride(1) != 1:
        raise ValueError(f"fp8_linear_tensor_static: out must be bf16 [{M}, {N}] with unit "
                         "column stride")
    dt = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}[x.dtype]
    rc = load().srdit_fp8_linear_tensor_static(_ptr(x), M, K, x.stride(0), dt, _ptr(w),
                                               _ptr(w_scale), int(w_scale.numel()), _ptr(bias),
                                               _ptr(out), N, out.stride(0), _stream(x.device))
    _check(rc, "srdit_fp8_linear_tensor_static")


def fp8_quant_tensor_gelu(x, xq, scale, amax_ws, h=None, xmax_pos=None):
    """The per-tensor e4m3 quantisation of h = bf16(gelu_tanh(x)) into xq / scale;
    h itself is also written when a buffer other than x is given.  ``xmax_pos``
    (int32 [1], nullable): the largest positive value of x as its producer wrote
    it (``GEMM_AMAX_POS``), which lets the call skip its amax pass."""
    M, K, ldx, dt = _quant_args(x, xq)
    if dt != 0:
        raise ValueError("fp8_quant_tensor_gelu: x must be bf16")
    if h is not None:
        if h.dtype != torch.bfloat16 or tuple(h.shape) != (M, K) or h.stride(1) != 1 or \
                h.data_ptr() == x.data_ptr():
            raise ValueError("fp8_quant_tensor_gelu: h must be a bf16 buffer shaped like x "
                             "(unit column stride), not x itself")
    rc = load().srdit_fp8_quant_tensor_gelu_ex(_ptr(x), M, K, ldx, _ptr(h),
                                               h.stride(0) if h is not None else 0, _ptr(xq),
                                               _ptr(scale), _ptr(amax_ws), _ptr(xmax_pos),
                                               _stream(x.device))
    _check(rc, "srdit_fp8_quant_tensor_gelu_ex")


def fp8_quant_apply(x, xq, scale, amax_ws):
    M, K, ldx, dt = _quant_args(x, xq)
    rc = load().srdit_fp8_quant_apply(_ptr(x), M, K, ldx, dt, _ptr(xq), _ptr(scale), _ptr(amax_ws),
                                      _stream(x.device))
    _check(rc, "srdit_fp8_quant_apply")


def _bf16_rows(name, t):
    if t.dtype != torch.bfloat16 or t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be a 2-D bf16 tensor with unit column stride")


def ln_modulate(x, ln_w, ln_b, scale, shift, eps, out, amax_ws=None):
    _bf16_rows("ln_modulate x", x)
    _bf16_rows("ln_modulate out", out)
    M, K = x.shape
    rc = load().srdit_ln_modulate(_ptr(x), M, K, x.stride(0), _ptr(ln_w), _ptr(ln_b), _ptr(scale),
                                  _ptr(shift), float(eps), _ptr(out), out.stride(0), _ptr(amax_ws),
                                  _stream(x.device))
    _check(rc, "srdit_ln_modulate")


def residual_gate(x, y, gate, out):
    for nm, t in (("x", x), ("y", y), ("out", out)):
        _bf16_rows(f"residual_gate {nm}", t)
    M, K = x.shape
    rc = load().srdit_residual_gate(_ptr(x), _ptr(y), _ptr(gate), M, K, x.stride(0), y.stride(0),
                                    _ptr(out), out.stride(0), _stream(x.device))
    _check(rc, "srdit_residual_gate")


def residual_ln_modulate(x, y, gate, x_out, ln_w, ln_b, scale, shift, eps, out, amax_ws=None):
    """x_out = bf16(x + y * gate), out = ln_modulate(x_out, ...): one pass, the same
    bits as residual_gate followed by ln_modulate."""
    for nm, t in (("x", x), ("y", y), ("x_out", x_out), ("out", out)):
        _bf16_rows(f"residual_ln_modulate {nm}", t)
    M, K = x.shape
    rc = load().srdit_residual_ln_modulate(
        _ptr(x), _ptr(y), _ptr(gate), M, K, x.stride(0), y.stride(0), _ptr(x_out),
        x_out.stride(0), _ptr(ln_w), _ptr(ln_b), _ptr(scale), _ptr(shift), float(eps), _ptr(out),
        out.stride(0), _ptr(amax_ws), _stream(x.device))
    _check(rc, "srdit_residual_ln_modulate")


def rmsnorm_rope(x, w, eps, rope_cs, head_dim, out):
    _bf16_rows("rmsnorm_rope x", x)
    M, K = x.shape
    rc = load().srdit_rmsnorm_rope(_ptr(x), M, K, x.stride(0), _ptr(w), float(eps), _ptr(rope_cs),
                                   int(head_dim), _ptr(out), _stream(x.device))
    _check(rc, "srdit_rmsnorm_rope")


def copy_bytes(src, dst, nbytes):
    rc = load().srdit_copy_bytes(_ptr(src), _ptr(dst), int(nbytes), _stream(src.device))
    _check(rc, "srdit_copy_bytes")


# -- dense Linears at the forward's ends (csrc/dense.hip) ----------------------
_DENSE_W_CODES = {torch.bfloat16: 0, torch.float32: 2}


def _rows2d(name, t, dtype):
    if t.dim() != 2 or t.stride(1) != 1 or t.dtype != dtype or not t.is_cuda:
        raise ValueError(f"{name} must be a 2-D {dtype} device tensor with unit column stride, "
                         f"got {t.dtype} {tuple(t.shape)} strides {t.stride()}")


def _vec(name, t, n, dtype):
    if t is not None and (t.dtype != dtype or t.numel() != n or not t.is_contiguous()):
        raise ValueError(f"{name} must be a contiguous {dtype} vector of {n} values")


def bf16_linear(a, w, bias, out, gelu=False):
    """out [M, N] = bf16(a [M, K] @ w [N, K]^T + bias) in bf16 with fp32
    accumulation; with ``gelu`` then bf16(gelu_tanh(out))."""
    _rows2d("bf16_linear a", a, torch.bfloat16)
    _rows2d("bf16_linear w", w, torch.bfloat16)
    _rows2d("bf16_linear out", out, torch.bfloat16)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or tuple(out.shape) != (M, N):
        raise ValueError(f"bf16_linear: shapes a {tuple(a.shape)} w {tuple(w.shape)} "
                         f"out {tuple(out.shape)} disagree")
    _vec("bf16_linear bias", bias, N, torch.bfloat16)
    rc = load().srdit_bf16_linear(_ptr(a), a.stride(0), _ptr(w), w.stride(0), _ptr(bias),
                                  _ptr(out), out.stride(0), M, N, K, int(bool(gelu)),
                                  _stream(a.device))
    _check(rc, "srdit_bf16_linear")


def linear_f32_modulated(a, s1, m0, w, bias, out):
    """out [M, N] fp32 = (f32(a) * s1 + m0) @ w^T + bias, a [M, K] bf16, s1/m0
    fp32 [K], w [N, K] and bias [N] both bf16 or both fp32 (bias may be None)."""
    _rows2d("linear_f32_modulated a", a, torch.bfloat16)
    if w.dtype not in _DENSE_W_CODES:
        raise ValueError(f"linear_f32_modulated: weights must be bf16 or fp32, got {w.dtype}")
    _rows2d("linear_f32_modulated w", w, w.dtype)
    _rows2d("linear_f32_modulated out", out, torch.float32)
    M, K = a.shape
    N = w.shape[0]
    if w.shape[1] != K or tuple(out.shape) != (M, N):
        raise ValueError(f"linear_f32_modulated: shapes a {tuple(a.shape)} w {tuple(w.shape)} "
                         f"out {tuple(out.shape)} disagree")
    _vec("linear_f32_modulated s1", s1, K, torch.float32)
    _vec("linear_f32_modulated m0", m0, K, torch.float32)
    _vec("linear_f32_modulated bias", bias, N, w.dtype)
    rc = load().srdit_linear_f32_modulated(_ptr(a), a.stride(0), _ptr(s1), _ptr(m0), _ptr(w),
                                           w.stride(0), _ptr(bias), _DENSE_W_CODES[w.dtype],
                                           _ptr(out), out.stride(0), M, N, K, _stream(a.device))
    _check(rc, "srdit_linear_f32_modulated")


def gemv_f32(x, w, bias, out):
    """out [M, N] fp32 = x [M, K] fp32 @ w [N, K]^T + bias, w and bias both bf16 or
    both fp32 (bias may be None); one wave per output, for a few rows."""
    _rows2d("gemv_f32 x", x, torch.float32)
    if w.dtype not in _DENSE_W_CODES:
        raise ValueError(f"gemv_f32: weights must be bf16 or fp32, got {w.dtype}")
    _rows2d("gemv_f32 w", w, w.dtype)
    _rows2d("gemv_f32 out", out, torch.float32)
    M, K = x.shape
    N = w.shape[0]
    if w.shape[1] != K or tuple(out.shape) != (M, N):
        raise ValueError(f"gemv_f32: shapes x {tuple(x.shape)} w {tuple(w.shape)} "
                         f"out {tuple(out.shape)} disagree")
    _vec("gemv_f32 bias", bias, N, w.dtype)
    rc = load().srdit_gemv_f32(_ptr(x), x.stride(0), _ptr(w), w.stride(0), _ptr(bias),
                               _DENSE_W_CODES[w.dtype], _ptr(out), out.stride(0), M, N, K,
                               _stream(x.device))
    _check(rc, "srdit_gemv_f32")
