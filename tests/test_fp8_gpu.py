"""fp8 quantisers and scaled GEMM on the GPU, through the C ABI, against the oracle.

Quantisers: bit-exact (codes and scales) against the numpy oracle and against
the reference's formula (fp8_linear.py:96-103) evaluated with torch on the GPU.
GEMM: against the float64 dequantised product, per element within the bf16
rounding of the result plus an fp32-accumulation allowance of 2^-12 times the
sum of |terms| of that element.
"""
import numpy as np
import pytest
import torch

from oracle import fp8 as of

pytestmark = pytest.mark.gpu

F8 = torch.float8_e4m3fn


def _lib():
    from sr_dit import _lib
    return _lib


def _rand(shape, dtype, seed, spread=6.0):
    g = torch.Generator("cpu").manual_seed(seed)
    rows = torch.empty(shape[0], 1).uniform_(-spread, spread, generator=g).exp()
    return (torch.randn(shape, generator=g) * rows).to(dtype)


def _torch_rowwise(x):
    """fp8_linear.py:96-103 with torch ops (on whatever device x is)."""
    amax = x.abs().amax(dim=-1, keepdim=True).float()
    scale = (amax / 448.0).clamp_min(1e-12)
    q = (x.float() / scale).clamp(-448.0, 448.0).to(F8)
    return q, scale


QUANT_CASES = [((1, 8), torch.bfloat16), ((3, 136), torch.bfloat16), ((257, 3072), torch.bfloat16),
               ((64, 14336), torch.bfloat16), ((5, 64), torch.float16), ((9, 200), torch.float32),
               ((130, 1024), torch.float32)]


@pytest.mark.parametrize("shape,dtype", QUANT_CASES, ids=lambda v: str(v))
def test_quant_rowwise_bit_exact(shape, dtype):
    print(f"quant_rowwise {shape} {dtype}", flush=True)
    x = _rand(shape, dtype, seed=shape[0] * 7 + shape[1])
    if shape[0] > 2:
        x[1] = 0
    q_ref, s_ref = of.quantize_rowwise(x.float().numpy())
    xd = x.cuda()
    q = torch.empty(shape, dtype=F8, device="cuda")
    s = torch.empty(shape[0], dtype=torch.float32, device="cuda")
    _lib().fp8_quant_rowwise(xd, q, s)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)
    qt, st = _torch_rowwise(xd)
    assert torch.equal(q.view(torch.uint8), qt.view(torch.uint8))
    assert torch.equal(s, st.reshape(-1))


def test_quant_rowwise_strided_rows():
    big = _rand((40, 512), torch.bfloat16, seed=11).cuda()
    x = big[:, 128:128 + 256]                       # ldx 512, K 256, 256-byte offset
    q = torch.empty((40, 256), dtype=F8, device="cuda")
    s = torch.empty(40, dtype=torch.float32, device="cuda")
    _lib().fp8_quant_rowwise(x, q, s)
    q_ref, s_ref = of.quantize_rowwise(x.float().cpu().numpy())
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


@pytest.mark.parametrize("shape,dtype", [((1, 8), torch.bfloat16), ((257, 3072), torch.bfloat16),
                                         ((4096, 1024), torch.bfloat16), ((9, 200), torch.float32)],
                         ids=lambda v: str(v))
def test_quant_tensor_bit_exact(shape, dtype):
    print(f"quant_tensor {shape} {dtype}", flush=True)
    x = _rand(shape, dtype, seed=shape[0] + 3)
    q_ref, s_ref = of.quantize_tensor(x.float().numpy())
    xd = x.cuda()
    q = torch.empty(shape, dtype=F8, device="cuda")
    s = torch.empty(1, dtype=torch.float32, device="cuda")
    ws = torch.full((1,), 12345, dtype=torch.int32, device="cuda")   # stale contents are cleared
    _lib().fp8_quant_tensor(xd, q, s, ws)
    torch.cuda.synchronize()
    assert np.array_equal(q.view(torch.uint8).cpu().numpy(), q_ref)
    assert np.array_equal(s.cpu().numpy(), s_ref)


def test_quant_rejects_bad_shapes():
    x = torch.zeros((4, 12), dtype=torch.bfloat16, device="cuda")     # K % 8 != 0
    q = torch.empty((4, 12), dtype=F8, device="cuda")
    s = torch.empty(4, dtype=torch.float32, device="cuda")
    with pytest.raises(RuntimeError, match="multiples of 8"):
        _lib().fp8_quant_rowwise(x, q, s)


def _quant_codes(shape, seed, spread=2.0):
    x = _rand(shape, torch.float32, seed, spread).numpy()
    return of.quantize_rowwise(x)


def _gemm_check(out, a_codes, b_codes, sa, sb, bias):
    ref = of.gemm_dequant(a_codes, b_codes, sa, sb, bias)
    t = of.e4m3_decode_table()
    sa_, sb_ = np.asarray(sa, np.float64).reshape(-1), np.asarray(sb, np.float64).reshape(-1)
    absum = np.abs(t[a_codes]) @ np.abs(t[b_codes]).T
    absum *= np.abs(sa_[:, None] if sa_.size > 1 else sa_[0])
    absum *= np.abs(sb_[None, :] if sb_.size > 1 else sb_[0])
    got = out.float().cpu().numpy().astype(np.float64)
    err = np.abs(got - ref)
    tol = 2.0 ** -8 * np.abs(ref) + 2.0 ** -12 * absum + 1e-30
    worst = np.max(err / tol)
    assert worst <= 1.0, f"worst err/tol {worst:.3f}, max err {err.max():.3e}"


GEMM_CASES = [
    # M, N, K, row-wise a scale, per-column b scale, bias
    (256, 256, 128, True, True, True),
    (300, 272, 384, True, True, True),       # ragged M and N tiles
    (64, 32, 256, False, False, False),      # per-tensor scales
    (513, 1040, 1152, True, False, True),
    (1, 16, 128, True, True, True),
    (1000, 3072, 3072, True, True, True),
]


@pytest.mark.parametrize("M,N,K,rs,cs,use_bias", GEMM_CASES, ids=lambda v: str(v))
def test_gemm_matches_dequantised_product(M, N, K, rs, cs, use_bias):
    print(f"gemm M={M} N={N} K={K} rows={rs} cols={cs} bias={use_bias}", flush=True)
    a, sa = _quant_codes((M, K), seed=M + K)
    b, sb = _quant_codes((N, K), seed=N * 3 + K)
    if not rs:
        sa = np.float32([0.75])
    if not cs:
        sb = np.float32([1.25])
    g = torch.Generator("cpu").manual_seed(5)
    bias = (torch.randn(N, generator=g) * 4).to(torch.bfloat16) if use_bias else None
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib().fp8_gemm(torch.from_numpy(a).view(F8).cuda(), torch.from_numpy(b).view(F8).cuda(),
                    torch.from_numpy(sa).cuda(), torch.from_numpy(sb).cuda(),
                    bias.cuda() if bias is not None else None, out)
    torch.cuda.synchronize()
    _gemm_check(out, a, b, sa, sb, bias.float().numpy() if bias is not None else None)


TENSOR_CASES = [
    # M, N, K, bias, ldo (None: N)
    (64, 32, 256, False, None),
    (300, 272, 384, True, None),
    (1, 16, 128, True, None),
    (96, 48, 256, True, 64),
    (1000, 3072, 3072, True, None),
    (21600, 3072, 3072, True, None),
]


@pytest.mark.parametrize("M,N,K,use_bias,ldo", TENSOR_CASES, ids=lambda v: str(v))
def test_gemm_per_tensor(M, N, K, use_bias, ldo):
    """Per-tensor scales against the dequantised product with the per-element
    bound; padding columns of a strided output stay untouched."""
    print(f"gemm per-tensor M={M} N={N} K={K} bias={use_bias} ldo={ldo}", flush=True)
    a, _ = _quant_codes((M, K), seed=M + 2 * K)
    b, _ = _quant_codes((N, K), seed=N + 5 * K)
    sa, sb = np.float32([0.75]), np.float32([1.25 / 64])
    g = torch.Generator("cpu").manual_seed(9)
    bias = (torch.randn(N, generator=g) * 4).to(torch.bfloat16) if use_bias else None
    lo = ldo or N
    buf = torch.full((M, lo), 7.0, dtype=torch.bfloat16, device="cuda")
    out = buf[:, :N]
    _lib().fp8_gemm_ex(torch.from_numpy(a).view(F8).cuda(), torch.from_numpy(b).view(F8).cuda(),
                       torch.from_numpy(sa).cuda(), torch.from_numpy(sb).cuda(),
                       bias.cuda() if bias is not None else None, out)
    torch.cuda.synchronize()
    if M * N <= 4_000_000:
        _gemm_check(out, a, b, sa, sb, bias.float().numpy() if bias is not None else None)
    else:  # production size: torch fp32 matmul of the dequantised operands
        torch.backends.cuda.matmul.allow_tf32 = False
        t = torch.from_numpy(of.e4m3_decode_table()).float().cuda()
        A, B = t[torch.from_numpy(a).cuda().long()], t[torch.from_numpy(b).cuda().long()]
        ref = (A @ B.T) * float(sa[0]) * float(sb[0]) + bias.float().cuda()
        absum = (A.abs() @ B.abs().T) * float(sa[0]) * float(sb[0])
        tol = 2.0 ** -8 * ref.abs() + 2.0 ** -12 * absum + 2.0 ** -20 * absum.max()
        worst = ((out.float() - ref).abs() / tol).max().item()
        assert worst <= 1.0, worst
    if lo > N:
        assert torch.all(buf[:, N:] == 7.0)


def test_gemm_strided_output_leaves_padding():
    M, N, K, ldo = 96, 48, 256, 64
    a, sa = _quant_codes((M, K), seed=1)
    b, sb = _quant_codes((N, K), seed=2)
    buf = torch.full((M, ldo), 7.0, dtype=torch.bfloat16, device="cuda")
    out = buf[:, :N]
    _lib().fp8_gemm(torch.from_numpy(a).view(F8).cuda(), torch.from_numpy(b).view(F8).cuda(),
                    torch.from_numpy(sa).cuda(), torch.from_numpy(sb).cuda(), None, out)
    torch.cuda.synchronize()
    _gemm_check(out, a, b, sa, sb, None)
    assert torch.all(buf[:, N:] == 7.0)


@pytest.mark.parametrize("M,N,K", [(21600, 3072, 3072), (2048, 14336, 3072), (2048, 3072, 14336)])
def test_gemm_full_size_against_fp32_matmul(M, N, K):
    """Production shapes (q/k/v/o, ffn.0, ffn.2) against torch's fp32 matmul of the
    dequantised operands, with the same per-element bound."""
    print(f"gemm full-size M={M} N={N} K={K}", flush=True)
    torch.backends.cuda.matmul.allow_tf32 = False
    x = _rand((M, K), torch.bfloat16, seed=21, spread=1.0).cuda()
    w = (_rand((N, K), torch.float32, seed=22, spread=0.5) * 0.02).to(torch.bfloat16).cuda()
    xq, xs = _torch_rowwise(x)
    wq, ws = _torch_rowwise(w)
    bias = (torch.randn(N, generator=torch.Generator("cpu").manual_seed(3)) * 0.1).to(torch.bfloat16).cuda()
    out = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    _lib().fp8_gemm(xq.contiguous(), wq.contiguous(), xs.reshape(-1).contiguous(),
                    ws.reshape(-1).contiguous(), bias, out)
    A, B = xq.float(), wq.float()
    ref = (A @ B.T) * xs * ws.reshape(1, -1) + bias.float()
    absum = (A.abs() @ B.abs().T) * xs * ws.reshape(1, -1)
    tol = 2.0 ** -8 * ref.abs() + 2.0 ** -12 * absum + 2.0 ** -20 * absum.max()
    worst = ((out.float() - ref).abs() / tol).max().item()
    assert worst <= 1.0, worst


MULTI_TILE_CASES = [
    # M, N, K, row-wise scales, ldo (None: N): more tiles than CUs, so each
    # persistent workgroup walks several tiles (one or two K stages per tile,
    # ragged last rows and columns, a strided output)
    (5000, 4096, 128, True, None),
    (3000, 6144, 256, True, None),
    (4100, 4624, 384, False, 4640),
]


def _dequant_check(out, aq, bq, sa, sb, bias, epilogue=0):
    torch.backends.cuda.matmul.allow_tf32 = False
    A, B = aq.float(), bq.float()
    sa_ = sa.reshape(-1, 1) if sa.numel() > 1 else sa.reshape(())
    sb_ = sb.reshape(1, -1) if sb.numel() > 1 else sb.reshape(())
    ref = (A @ B.T) * sa_ * sb_ + bias.float()
    absum = (A.abs() @ B.abs().T) * sa_.abs() * sb_.abs()
    tol = 2.0 ** -8 * ref.abs() + 2.0 ** -12 * absum + 2.0 ** -20 * absum.max()
    worst = ((out.float() - ref).abs() / tol).max().item()
    assert worst <= 1.0, worst


@pytest.mark.parametrize("M,N,K,rs,ldo", MULTI_TILE_CASES, ids=lambda v: str(v))
def test_gemm_persistent_multi_tile(M, N, K, rs, ldo):
    print(f"gemm multi-tile M={M} N={N} K={K} rowwise={rs} ldo={ldo}", flush=True)
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) * 0.6).to(F8).cuda()
    b = (torch.randn(N, K, generator=g) * 0.6).to(F8).cuda()
    if rs:
        sa = (torch.rand(M, generator=g) + 0.5).cuda()
        sb = (torch.rand(N, generator=g) / 64 + 1 / 128).cuda()
    else:
        sa, sb = torch.tensor([0.75]).cuda(), torch.tensor([1.25 / 64]).cuda()
    bias = (torch.randn(N, generator=g) * 2).to(torch.bfloat16).cuda()
    lo = ldo or N
    buf = torch.full((M, lo), 7.0, dtype=torch.bfloat16, device="cuda")
    out = buf[:, :N]
    _lib().fp8_gemm(a, b, sa, sb, bias, out)
    torch.cuda.synchronize()
    _dequant_check(out, a, b, sa, sb, bias)
    if lo > N:
        assert torch.all(buf[:, N:] == 7.0)
    # the GELU epilogue with the output's amax over the same tiles
    out2 = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
    amax = torch.full((1,), 12345, dtype=torch.int32, device="cuda")
    _lib().fp8_gemm_ex(a, b, sa, sb, bias, out2, epilogue=1, amax_out=amax)
    plain = out.contiguous()
    gel = torch.nn.functional.gelu(plain.float(), approximate="tanh").to(torch.bfloat16)
    torch.cuda.synchronize()
    # the epilogue rounds to bf16, then GELU, then bf16; 1 + tanh(.) cancels for
    # negative inputs, so bound by the input's magnitude
    err = (out2.float() - gel.float()).abs()
    assert (err <= 5e-3 * plain.float().abs() + 1e-30).all(), err.max().item()
    assert amax.item() == out2.float().abs().max().view(torch.int32).item()


@pytest.mark.parametrize("rs", [False, True], ids=["tensor", "rowwise"])
def test_gemm_split_output_equals_per_block_gemms(rs):
    """Stacked weights through one split-output GEMM: each output block is bit for
    bit the GEMM of its own weight block (512 context rows, 6 blocks of 3072)."""
    print(f"gemm split rowwise={rs}", flush=True)
    g = torch.Generator("cpu").manual_seed(17)
    M, K, W, G = 512, 3072, 3072, 6
    a = (torch.randn(M, K, generator=g) * 0.6).to(F8).cuda()
    b = (torch.randn(G * W, K, generator=g) * 0.6).to(F8).cuda()
    sa = (torch.rand(M, generator=g) + 0.5).cuda() if rs else torch.tensor([0.75]).cuda()
    sb_blk = [(torch.rand(W, generator=g) / 64).cuda() if rs else torch.rand(1, generator=g).cuda()
              for _ in range(G)]
    sb = torch.cat([x.expand(W) for x in sb_blk]).contiguous()
    bias = (torch.randn(G * W, generator=g)).to(torch.bfloat16).cuda()
    out = torch.full((G, M, W), float("nan"), dtype=torch.bfloat16, device="cuda")
    _lib().fp8_gemm_split(a, b, sa, sb, bias, out)
    for j in range(G):
        ref = torch.empty(M, W, dtype=torch.bfloat16, device="cuda")
        _lib().fp8_gemm(a, b[j * W:(j + 1) * W].contiguous(), sa, sb_blk[j].contiguous(),
                        bias[j * W:(j + 1) * W].contiguous(), ref)
        torch.cuda.synchronize()
        assert torch.equal(out[j], ref), j


def _tail_tiles(M, N, K):
    """Output tiles (row, column) of the GEMM's split-K tail on this device: the
    last (T mod G) tiles of the raster order (groups of 4 tile rows, column-major
    inside a group), T = 256x256 tiles, G = the CUs rounded down to 8, when that
    tail is at most G / 8 and a split along K saves a quarter of the round
    (chosen as the library's planner does; None when nothing is split)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count // 8 * 8
    tm, tn = -(-M // 256), -(-N // 256)
    T = tm * tn
    grid = min(cus, -(-T // 8) * 8)
    tail, nks = T % grid, K // 128
    if T < grid or tail == 0 or 8 * tail > grid:
        return None
    costs = [(-(-nks // S) + 5.0 + 4.0 * S, S) for S in range(2, nks + 1) if tail * S <= grid]
    if not costs or min(costs)[0] >= 0.75 * nks:
        return None
    tiles = []
    for task in range(T - tail, T):
        group, r = divmod(task, 4 * tn)
        gsize = min(tm - 4 * group, 4)
        tiles.append((4 * group + r % gsize, r // gsize))
    return tiles


TAIL_CASES = [
    # M, N, K, row-wise scales, GELU epilogue with the output amax: a streamed
    # chunk's 10,800 rows leave the last round of tiles nearly empty (516 tiles,
    # 4 in the last round); the split pays at long K
    (10800, 3072, 14336, False, False),   # FFN down: 112 K stages per tile
    (10800, 3072, 14336, True, True),     # row-wise scales, GELU + amax
    (10800, 3072, 8192, False, False),    # 64 K stages
]


@pytest.mark.parametrize("M,N,K,rs,gelu", TAIL_CASES, ids=lambda v: str(v))
def test_gemm_split_k_tail(M, N, K, rs, gelu):
    """The split-K tail (srdit_fp8_gemm_ws): within the bound of the dequantised
    product; every tile outside the tail bit for bit the unsplit GEMM's; the
    tail's tiles within one bf16 rounding of it (fp8 products sum exactly in
    fp32 for the most part, so they are mostly equal); the amax word exact; two
    calls in a row (the arrival counters left at zero) bit for bit alike; two
    launches with the split, one without."""
    print(f"[case] gemm split-K tail M={M} N={N} K={K} rowwise={rs} gelu={gelu}", flush=True)
    L = _lib()
    g = torch.Generator("cpu").manual_seed(M + N + K)
    a = (torch.randn(M, K, generator=g) * 0.6).to(F8).cuda()
    b = (torch.randn(N, K, generator=g) * 0.6).to(F8).cuda()
    if rs:
        sa = (torch.rand(M, generator=g) + 0.5).cuda()
        sb = (torch.rand(N, generator=g) / 64 + 1 / 128).cuda()
    else:
        sa, sb = torch.tensor([0.75]).cuda(), torch.tensor([1.25 / 64]).cuda()
    bias = (torch.randn(N, generator=g) * 2).to(torch.bfloat16).cuda()
    ep = 1 if gelu else 0
    outs, amaxes = [], []
    for split in (True, True, False):
        out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device="cuda")
        amax = torch.full((1,), 12345, dtype=torch.int32, device="cuda") if gelu else None
        L.fp8_gemm_ex(a, b, sa, sb, bias, out, epilogue=ep, amax_out=amax, split_tail=split)
        outs.append(out)
        amaxes.append(amax)
    torch.cuda.synchronize()
    split1, split2, plain = outs
    assert torch.equal(split1, split2)
    if not gelu:
        _dequant_check(split1, a, b, sa, sb, bias)
    else:
        assert amaxes[0].item() == split1.float().abs().max().view(torch.int32).item()
        assert amaxes[2].item() == plain.float().abs().max().view(torch.int32).item()
    tiles = _tail_tiles(M, N, K)
    assert tiles, "this shape has a split tail on a 256-CU MI355X"
    mask = torch.zeros(M, N, dtype=torch.bool, device="cuda")
    for tr, tc in tiles:
        mask[tr * 256:(tr + 1) * 256, tc * 256:(tc + 1) * 256] = True
    assert torch.equal(split1[~mask], plain[~mask])
    d = (split1[mask].float() - plain[mask].float()).abs()
    assert (d <= 2.0 ** -7 * plain[mask].float().abs() + 1e-30).all(), d.max().item()
    # the split ran: a second launch, the split instantiation of the kernel
    from torch.profiler import ProfilerActivity, profile
    for split, launches in ((True, 2), (False, 1)):
        with profile(activities=[ProfilerActivity.CUDA]) as prof:
            L.fp8_gemm_ex(a, b, sa, sb, bias, plain, epilogue=ep, amax_out=amaxes[2],
                          split_tail=split)
            torch.cuda.synchronize()
        names = [ev.name for ev in prof.events()
                 if ev.device_type == torch.autograd.DeviceType.CUDA and "fp8_gemm_kernel" in ev.name]
        assert len(names) == launches, names


def test_gemm_split_k_tail_split_output_and_graph():
    """Three column blocks of one split-output GEMM with a split-K tail (1548
    tiles, 12 in the last round, K = 8192), captured on the library's capture stream
    and replayed on changing inputs with eager work between replays: every
    replay bit for bit the eager call, each block within the bound of the
    dequantised product."""
    print("[case] gemm split-K tail, split output, graph", flush=True)
    L = _lib()
    M, K, W, G = 10800, 8192, 3072, 3
    g = torch.Generator("cpu").manual_seed(23)
    a = (torch.randn(M, K, generator=g) * 0.6).to(F8).cuda()
    b = (torch.randn(G * W, K, generator=g) * 0.6).to(F8).cuda()
    sa = torch.tensor([0.75]).cuda()
    sb = torch.cat([torch.rand(1, generator=g).expand(W) for _ in range(G)]).contiguous().cuda()
    bias = torch.randn(G * W, generator=g).to(torch.bfloat16).cuda()
    assert _tail_tiles(M, G * W, K)
    out = torch.empty((G, M, W), dtype=torch.bfloat16, device="cuda")
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=L.capture_stream("cuda")):
        L.fp8_gemm_split(a, b, sa, sb, bias, out)
    for it in range(3):
        a.copy_((torch.randn(M, K, generator=g) * (0.3 + 0.3 * it)).to(F8).cuda())
        graph.replay()
        want = torch.empty_like(out)
        L.fp8_gemm_split(a, b, sa, sb, bias, want)
        torch.cuda.synchronize()
        assert torch.equal(out, want), it
    for j in range(G):
        _dequant_check(out[j], a, b[j * W:(j + 1) * W], sa, sb[j * W:(j + 1) * W],
                       bias[j * W:(j + 1) * W])


def test_fp8_linear_rowwise_and_tensor():
    from sr_dit.fp8_linear import Fp8Linear
    torch.manual_seed(0)
    lin = torch.nn.Linear(384, 272).to(torch.bfloat16).cuda()
    x = torch.randn(2, 150, 384, dtype=torch.bfloat16, device="cuda")
    for scaling in ("rowwise", "tensor"):
        m = Fp8Linear.from_linear(lin, scaling=scaling)
        y = m(x)
        assert y.shape == (2, 150, 272) and y.dtype == torch.bfloat16
        # reference semantics with torch ops: quantise, dequantised fp32 product, bias
        x2 = x.reshape(-1, 384)
        if scaling == "rowwise":
            xq, xs = _torch_rowwise(x2)
            wq, ws = _torch_rowwise(lin.weight.detach())
            ws = ws.reshape(1, -1)
        else:
            def tq(t):
                s = (t.abs().amax().float() / 448.0).clamp_min(1e-12)
                return (t.float() / s).clamp(-448, 448).to(F8), s
            xq, xs = tq(x2)
            wq, ws = tq(lin.weight.detach())
        assert torch.equal(m.weight_fp8.view(torch.uint8), wq.view(torch.uint8))
        ref = (xq.float() @ wq.float().T) * xs * ws + lin.bias.float()
        err = (y.reshape(-1, 272).float() - ref).abs()
        assert err.max().item() <= 2.0 ** -7 * ref.abs().max().item(), scaling
        # .to(bf16) keeps the fp8 buffers' dtypes (fp8_linear.py:260-280)
        m2 = m.to(torch.bfloat16)
        assert m2.weight_fp8.dtype == F8 and m2.weight_scale.dtype == torch.float32
        assert m2.weight.numel() == 0 and m2.weight.dtype == torch.bfloat16


def test_convert_linears_to_fp8_swaps_blocks_in_range():
    from sr_dit.fp8_linear import Fp8Linear, TARGETS_ALL, convert_linears_to_fp8

    class Attn(torch.nn.Module):
        def __init__(self):
            super().__init__()
            for n in ("q", "k", "v", "o"):
                setattr(self, n, torch.nn.Linear(128, 128))

    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn, self.cross_attn = Attn(), Attn()
            self.ffn = torch.nn.Sequential(torch.nn.Linear(128, 256), torch.nn.GELU(),
                                           torch.nn.Linear(256, 128))

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([Block() for _ in range(4)])
            self.head = torch.nn.Linear(128, 16)

    model = Model().to(torch.bfloat16).cuda()
    names = convert_linears_to_fp8(model, skip_first=1, skip_last=1)
    assert names == [f"blocks.{i}.{s}" for i in (1, 2) for s in TARGETS_ALL]
    assert isinstance(model.blocks[1].ffn[2], Fp8Linear)
    assert isinstance(model.blocks[0].ffn[0], torch.nn.Linear)
    assert isinstance(model.head, torch.nn.Linear)
    assert convert_linears_to_fp8(model, skip_first=1, skip_last=1) == []     # idempotent


def test_quantise_and_gemm_replay_in_a_graph():
    """Per-tensor quantiser (kernel-cleared workspace) + GEMM captured once and
    replayed on changing inputs, eager work between replays, every replay checked."""
    from sr_dit import fp8_linear as fl
    torch.manual_seed(1)
    lin = torch.nn.Linear(256, 512, bias=True).to(torch.bfloat16).cuda()
    m = fl.Fp8Linear.from_linear(lin, scaling="tensor")
    x = torch.randn(640, 256, dtype=torch.bfloat16, device="cuda")
    m(x)                                      # allocate the workspace outside the capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = m(x)
    for it in range(4):
        x.copy_(torch.randn(640, 256, dtype=torch.bfloat16, device="cuda") * (1 + 3 * it))
        g.replay()
        torch.cuda.synchronize()
        want = m(x)
        torch.cuda.synchronize()
        assert torch.equal(y, want), it


def _finite_bf16_values():
    """Every finite bf16 value (both zeros included), as float32."""
    bits = np.arange(1 << 16, dtype=np.uint32)
    finite = ((bits >> 7) & 0xFF) != 0xFF
    return (bits[finite] << 16).view(np.float32)


def _to_bf16_gpu(vals, cols=64):
    """float32 values that are bf16-exact -> bf16 [rows, cols] on the GPU (zero padded)."""
    n = len(vals)
    rows = -(-n // cols)
    buf = np.zeros(rows * cols, dtype=np.float32)
    buf[:n] = vals
    u16 = (buf.view(np.uint32) >> 16).astype(np.uint16)
    return torch.from_numpy(u16.view(np.int16)).view(torch.bfloat16).reshape(rows, cols).cuda(), buf


def test_quant_apply_every_bf16_value_many_scales():
    """The quantise pass divides by the shared scale through its reciprocal and one
    FMA correction; over every finite bf16 value |x| <= amax, for amax across the
    whole float range and at the 1e-12 scale floor, the codes and the scale equal
    the oracle's (numpy's IEEE x / s, clamp, round-to-nearest-even e4m3)."""
    vals = _finite_bf16_values()
    rng = np.random.default_rng(11)
    amaxes = [448.0, 1.0, 3.0, 0.1, 4.48e-10, 4.4e-10, 1e-30, 1e-40, 3.3895314e38, 2.0 ** -126]
    amaxes += list((rng.uniform(1.0, 2.0, 48) * 2.0 ** rng.integers(-133, 127, 48)).astype(np.float32))
    L = _lib()
    for amax in amaxes:
        amax32 = np.float32(amax)
        if not (np.isfinite(amax32) and amax32 > 0):
            continue
        x = vals[np.abs(vals) <= amax32]
        xt, buf = _to_bf16_gpu(x)
        scale = np.float32(max(np.float32(amax32 * of.INV_FP8_MAX), of.SCALE_FLOOR))
        want = of.e4m3_encode(np.clip(buf / scale, -of.FP8_MAX, of.FP8_MAX).astype(np.float32))
        word = torch.from_numpy(np.array([amax32], dtype=np.float32).view(np.int32)).cuda()
        tq = torch.empty(xt.shape, dtype=F8, device="cuda")
        ts = torch.empty(1, dtype=torch.float32, device="cuda")
        L.fp8_quant_apply(xt, tq, ts, word)
        torch.cuda.synchronize()
        got = tq.view(torch.uint8).cpu().numpy().reshape(-1)
        bad = np.nonzero(got != want)[0]
        assert len(bad) == 0, (f"amax {amax32!r}: {len(bad)} codes differ, first x={buf[bad[0]]!r} "
                               f"got {got[bad[0]]:#x} want {want[bad[0]]:#x}")
        assert ts.item() == scale


def test_quant_rowwise_every_bf16_value():
    """All finite bf16 values, sorted by magnitude and cut into rows of 64 (so the row
    scales span the float range, floor included): codes and scales equal the oracle's."""
    vals = _finite_bf16_values()
    vals = vals[np.argsort(np.abs(vals), kind="stable")]
    xt, buf = _to_bf16_gpu(vals)
    want_q, want_s = of.quantize_rowwise(buf.reshape(xt.shape))
    tq = torch.empty(xt.shape, dtype=F8, device="cuda")
    ts = torch.empty(xt.shape[0], dtype=torch.float32, device="cuda")
    _lib().fp8_quant_rowwise(xt, tq, ts)
    torch.cuda.synchronize()
    assert np.array_equal(ts.cpu().numpy(), want_s)
    assert np.array_equal(tq.view(torch.uint8).cpu().numpy(), want_q)
