"""SR-DiT 5B refiner block stack on the gfx950 kernels: inference forward.

Restates the pieces of video_refiner/wan/modules/sr_dit/models.py that one
refiner step runs:

* ``WanRMSNorm`` (models.py:424-440) and ``WanLayerNorm`` (:443-503), fp32;
* 3-D RoPE: ``rope_params`` (:80-88), ``_rope_axis_dims`` (:91-97) and
  ``rope_apply`` (:173-214);
* ``WanSelfAttention.forward``'s window path (:583-676): q/k/v projections,
  RMSNorm on q and k, RoPE, block-grid window attention, output projection;
* ``WanT2VCrossAttention.forward`` (:1042-1062): dense attention of every video
  token over the text context;
* ``WanAttentionBlock.forward``'s non-teacher-forcing path (:1304-1351) with
  ``cross_attn_ffn`` (:1256-1262): adaLN modulation, residuals, GELU(tanh) FFN;
* ``Head`` (:1357-1384), ``sinusoidal_embedding_1d`` (:67-77), the time and
  text embeddings of ``_prepare_embeddings`` (:1827-1875) and ``unpatchify``
  (:2234-2257).

Every Linear inside a block is an ``Fp8Linear`` (HIP fp8 GEMM); self-attention
is the HIP block-grid window kernel; cross-attention runs on the same kernel
with a plan of 64-token query windows that all see the whole text context.
Weights are random-initialised (no checkpoint); the module is inference-only.

RoPE is evaluated in fp32 where the reference uses complex128; the rotated
values are rounded to bf16 either way, and the fp32 rotation differs from the
fp64 one by ~1e-7 relative before that rounding.
"""
from __future__ import annotations

import math
from dataclasses import dataclass

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from . import attention as att
from . import blockgrid_hip as bgh
from .fp8_linear import FP8_DTYPE, Fp8Linear, quantize_rowwise, quantize_tensor


@dataclass(frozen=True)
class SRDiTConfig:
    """Architecture of the 5B refiner (video_refiner/configs/sr_dit_5b.yaml:29-55)."""
    dim: int = 3072
    ffn_dim: int = 14336
    num_heads: int = 24
    num_layers: int = 30
    in_dim: int = 48
    out_dim: int = 48
    patch_size: tuple = (1, 2, 2)
    freq_dim: int = 256
    text_dim: int = 4096
    text_len: int = 512
    eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_max_seq_len: int = 1024
    # window geometry of the benchmark: 8x8 blocks, 3x3 neighbourhood, +-1 frame
    block_hw: tuple = (8, 8)
    block_radius_hw: tuple = (1, 1)
    sym_radius_t: int = 1

    @property
    def head_dim(self) -> int:
        return self.dim // self.num_heads


class RMSNorm(nn.Module):
    """models.py:424-440: x * rsqrt(mean(x^2) + eps) in fp32, back to x's dtype, * weight."""

    def __init__(self, dim, eps=1e-5):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x):
        xf = x.float()
        return (xf * torch.rsqrt(xf.pow(2).mean(dim=-1, keepdim=True) + self.eps)).type_as(x) * self.weight


class LayerNormF32(nn.LayerNorm):
    """models.py:443-503 (non-DTensor path): layer_norm in fp32, back to x's dtype."""

    def __init__(self, dim, eps=1e-6, elementwise_affine=False):
        super().__init__(dim, elementwise_affine=elementwise_affine, eps=eps)

    def forward(self, x):
        w = self.weight.float() if self.weight is not None else None
        b = self.bias.float() if self.bias is not None else None
        return F.layer_norm(x.float(), self.normalized_shape, w, b, self.eps).type_as(x)


def rope_axis_dims(head_dim: int) -> tuple:
    """Real RoPE dims along T/H/W (models.py:91-97): 128 -> (44, 42, 42)."""
    return (head_dim - 4 * (head_dim // 6), 2 * (head_dim // 6), 2 * (head_dim // 6))


def rope_params(max_seq_len, dim, theta=10000.0):
    """models.py:80-88: complex128 [max_seq_len, dim/2] unit phasors pos * theta^(-2i/dim)."""
    pos = torch.arange(max_seq_len, dtype=torch.float64)
    inv = 1.0 / torch.pow(theta, torch.arange(0, dim, 2, dtype=torch.float64).div(dim))
    ang = torch.outer(pos, inv)
    return torch.polar(torch.ones_like(ang), ang)


def rope_positions(cfg: SRDiTConfig, f, h, w, t_offset=0, hw_stride=(1, 1)) -> int:
    """Positions the per-axis tables of a (f, h, w) grid need: they reach
    t_offset + f - 1 and (h - 1) * s_h, (w - 1) * s_w, and grow in whole
    multiples of rope_max_seq_len, as _ensure_rope_freqs (models.py:1789-1809)
    extends the reference's cache."""
    s_h, s_w = (int(hw_stride[0]), int(hw_stride[1]))
    need = max(int(t_offset) + f, s_h * h, s_w * w, 1)
    base = int(cfg.rope_max_seq_len)
    return base * -(-need // base)


def rope_axis_tables(cfg: SRDiTConfig, n_pos, device="cpu"):
    """The (t, h, w) frequency tables of rope_apply (models.py:176-178), each
    complex64 [n_pos, pairs]: c = head_dim/2 complex pairs split
    [c - 2(c//3), c//3, c//3], computed in float64 and rounded once."""
    dt, dh, dw = rope_axis_dims(cfg.head_dim)
    return tuple(rope_params(n_pos, dx, cfg.rope_theta).to(torch.complex64).to(device)
                 for dx in (dt, dh, dw))


def rope_table_from_axes(axes, f, h, w, t_offset=0, hw_stride=(1, 1)):
    """Per-token rotation [f*h*w, 1, head_dim/2] gathered from per-axis tables
    (rope_axis_tables) on their device: frame t_offset + i, row i*s_h, column
    j*s_w.  Only copies, so the result is the same on any device."""
    ft, fh, fw = axes
    s_h, s_w = (int(hw_stride[0]), int(hw_stride[1]))
    c = ft.shape[1] + fh.shape[1] + fw.shape[1]
    if t_offset + f > ft.shape[0] or s_h * (h - 1) >= fh.shape[0] or s_w * (w - 1) >= fw.shape[0]:
        raise ValueError("rope_table_from_axes: the axis tables are too short for this grid")
    return torch.cat([
        ft[t_offset:t_offset + f].view(f, 1, 1, -1).expand(f, h, w, -1),
        fh[0:s_h * h:s_h].view(1, h, 1, -1).expand(f, h, w, -1),
        fw[0:s_w * w:s_w].view(1, 1, w, -1).expand(f, h, w, -1)], dim=-1).reshape(f * h * w, 1, c)


def rope_table(cfg: SRDiTConfig, f, h, w, t_offset=0, device="cuda", hw_stride=(1, 1)):
    """Per-token complex64 rotation [f*h*w, 1, head_dim/2] for a (f, h, w) grid.

    The frequency split follows rope_apply (models.py:176-178): c = head_dim/2
    complex pairs split [c - 2(c//3), c//3, c//3] over (t, h, w).  ``hw_stride``
    (s_h, s_w) puts grid row i at position i*s_h and column j at j*s_w, as the
    native LQ-anchor harvest does (models.py:1761-1785).
    """
    s_h, s_w = (int(hw_stride[0]), int(hw_stride[1]))
    if s_h < 1 or s_w < 1:
        raise ValueError(f"rope_table: hw_stride must be >= 1, got {hw_stride!r}")
    axes = rope_axis_tables(cfg, rope_positions(cfg, f, h, w, t_offset, hw_stride))
    return rope_table_from_axes(axes, f, h, w, t_offset, hw_stride).to(device)


def rope_apply(x, table):
    """x [s, n, d] (bf16) rotated pairwise by table [s, 1, d/2]; result in x's dtype."""
    s, n, d = x.shape
    xc = torch.view_as_complex(x.float().reshape(s, n, d // 2, 2))
    return torch.view_as_real(xc * table).reshape(s, n, d).to(x.dtype)


def sinusoidal_embedding_1d(dim, position):
    """Timestep embedding of models.py:67-77: positions [n] -> [n, dim] float64,
    cos(p w_j) for j < dim/2 then sin(p w_j), with w_j = 10000^(-j / (dim/2)).
    Everything is made on the positions' device, so the call captures in a graph."""
    half = dim // 2
    j = torch.arange(half, dtype=torch.float64, device=position.device)
    ang = position.to(torch.float64)[:, None] * (10000.0 ** (-j / half))[None, :]
    return torch.cat([ang.cos(), ang.sin()], dim=1)


#: Cross-attention on the persistent dense kernel (srdit_dense_attn_fwd);
#: False runs it on the window kernel as a 1 x Lq grid of 64-query windows.
DENSE_CROSS = True


class CrossAttentionPlan:
    """Dense attention of Lq video tokens over Lc context tokens on the window kernel.

    The query tokens are laid out as one frame of a 1 x Lq grid; window i holds
    queries [64i, 64i + 64) and its KV cuboid is columns [0, Lc) of that grid,
    i.e. context tokens 0 .. Lc-1.  Rows use the plain 19-field layout with no
    anchor.
    """

    def __init__(self, lq: int, lc: int):
        rows = []
        for q0 in range(0, lq, 64):
            ql = min(64, lq - q0)
            rows.append([0, 1, 0, q0, 1, ql, 0, 1, 0, 1, 0, lc, 0, 0, 1, 0, lc, 1, lq])
        self.lq, self.lc = lq, lc
        self.plan = {"params": torch.tensor(rows, dtype=torch.int32), "n_w": len(rows),
                     "block_m": 64, "m_tiles": 1, "block_n": 64, "hr_base": 0,
                     "p_stride": bgh.P_PLAIN}

    def run(self, q, k, v, out, amax_out=None):
        """out = softmax(q k^T d^-1/2) v per head.  On the dense kernel
        (srdit_dense_attn_fwd) when ``DENSE_CROSS`` is set and the shapes fit it,
        else on the window kernel with this plan."""
        d = q.shape[2]
        if DENSE_CROSS and d in (64, 128) and q.dtype in (torch.bfloat16, torch.float16) \
                and all(t.is_contiguous() for t in (q, k, v, out)) and k.shape[0] == self.lc:
            _lib.dense_attn_fwd(q, k, v, out, d ** -0.5, amax_out)
            return out
        bgh.run_blockgrid_hip(q, k, v, out, plan=self.plan, f_cur=1, h=1, w=self.lq,
                              n=q.shape[1], d=d, amax_out=amax_out)
        return out


class SelfAttention(nn.Module):
    """WanSelfAttention, window path (models.py:583-676), one sample."""

    def __init__(self, cfg: SRDiTConfig):
        super().__init__()
        self.cfg = cfg
        dim = cfg.dim
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.norm_q = RMSNorm(dim, eps=cfg.eps)
        self.norm_k = RMSNorm(dim, eps=cfg.eps)

    def forward(self, x, geom):
        """x [s, dim] -> [s, dim]; geom: the step's geometry (SRDiT.geometry)."""
        n, d = self.cfg.num_heads, self.cfg.head_dim
        s = x.shape[0]
        q = self.norm_q(self.q(x)).view(s, n, d)
        k = self.norm_k(self.k(x)).view(s, n, d)
        v = self.v(x).view(s, n, d)
        q = rope_apply(q, geom["rope"]).contiguous()
        k = rope_apply(k, geom["rope"]).contiguous()
        out = torch.empty_like(q)
        f, h, w = geom["grid"]
        bgh.run_blockgrid_hip(q, k, v.contiguous(), out, plan=geom["plan"], f_cur=f, h=h, w=w,
                              n=n, d=d)
        return self.o(out.view(s, n * d))


class CrossAttention(nn.Module):
    """WanT2VCrossAttention (models.py:1042-1062), one sample, no context lengths."""

    def __init__(self, cfg: SRDiTConfig):
        super().__init__()
        self.cfg = cfg
        dim = cfg.dim
        self.q = nn.Linear(dim, dim)
        self.k = nn.Linear(dim, dim)
        self.v = nn.Linear(dim, dim)
        self.o = nn.Linear(dim, dim)
        self.norm_q = RMSNorm(dim, eps=cfg.eps)
        self.norm_k = RMSNorm(dim, eps=cfg.eps)

    def forward(self, x, context, geom):
        n, d = self.cfg.num_heads, self.cfg.head_dim
        s, lc = x.shape[0], context.shape[0]
        q = self.norm_q(self.q(x)).view(s, n, d).contiguous()
        k = self.norm_k(self.k(context)).view(lc, n, d).contiguous()
        v = self.v(context).view(lc, n, d).contiguous()
        out = torch.empty_like(q)
        geom["cross"].run(q, k, v, out)
        return self.o(out.view(s, n * d))


def _fp8_pack(owner, attr, lins):
    """Fp8Linear ``lins`` of one input stacked along their outputs, for one GEMM
    whose output column blocks land in separate tensors (srdit_fp8_gemm_split):
    (weights [sum N, K] e4m3, per-output-channel scales, bf16 biases (zeros
    where a Linear has none), row-wise?).  Cached in ``owner.__dict__[attr]``
    and rebuilt when a weight, scale or bias changes.  None unless every Linear
    is an Fp8Linear of one scaling and shape, or while a stream is captured and
    nothing is cached (building allocates)."""
    if not lins or not all(isinstance(m, Fp8Linear) for m in lins) \
            or len({(m.scaling, m.in_features, m.out_features) for m in lins}) != 1:
        return None
    key = tuple((m.weight_fp8.data_ptr(), m.weight_fp8._version, m.weight_scale.data_ptr(),
                 m.weight_scale._version, None if m.bias is None else
                 (m.bias.data_ptr(), m.bias._version)) for m in lins)
    cached = owner.__dict__.get(attr)
    if cached is not None and cached[0] == key:
        return cached[1]
    if torch.cuda.is_current_stream_capturing():
        return None
    n = lins[0].out_features
    w = torch.cat([m.weight_fp8 for m in lins]).contiguous()
    sb = torch.cat([m.weight_scale.reshape(-1).float().expand(n) for m in lins]).contiguous()
    bias = torch.cat([m.bias.to(torch.bfloat16) if m.bias is not None else
                      torch.zeros(n, dtype=torch.bfloat16, device=w.device)
                      for m in lins]).contiguous()
    pack = (w, sb, bias, lins[0].scaling == "rowwise")
    owner.__dict__[attr] = (key, pack)
    return pack


#: Self-attention q, k and v of a fused block as one split-output GEMM over the
#: block's quantised input (V then copied where it goes: a ring or a caller's
#: buffer); False runs three GEMMs.  Bit-identical either way.
QKV_PACK = True


class Block(nn.Module):
    """WanAttentionBlock, non-teacher-forcing forward (models.py:1304-1351, :1256-1262)."""

    def __init__(self, cfg: SRDiTConfig):
        super().__init__()
        dim = cfg.dim
        self.norm1 = LayerNormF32(dim, cfg.eps)
        self.self_attn = SelfAttention(cfg)
        self.norm3 = LayerNormF32(dim, cfg.eps, elementwise_affine=True)
        self.cross_attn = CrossAttention(cfg)
        self.norm2 = LayerNormF32(dim, cfg.eps)
        self.ffn = nn.Sequential(nn.Linear(dim, cfg.ffn_dim), nn.GELU(approximate="tanh"),
                                 nn.Linear(cfg.ffn_dim, dim))
        self.modulation = nn.Parameter(torch.randn(1, 6, dim) / dim ** 0.5)

    def _linears(self):
        return (self.self_attn.q, self.self_attn.k, self.self_attn.v, self.self_attn.o,
                self.cross_attn.q, self.cross_attn.k, self.cross_attn.v, self.cross_attn.o,
                self.ffn[0], self.ffn[2])

    def fusable(self) -> bool:
        """All Linears are Fp8Linear with one scaling mode (per-tensor or row-wise):
        the fused forward applies."""
        lins = self._linears()
        return (all(isinstance(m, Fp8Linear) for m in lins)
                and len({m.scaling for m in lins}) == 1)

    def forward(self, x, e, context, geom, ring=None, cross_kv=None, kv_out=None):
        """x [s, dim] (bf16), e [1, 6, dim] (fp32), context [lc, dim] -> [s, dim].

        ``ring``: this layer's streaming KV cache (``KVRing``, fused path only);
        ``cross_kv``: this layer's text K/V, computed once per video
        (``SRDiT.cross_cache``) as WanT2VCrossAttention.init_cache
        (models.py:1035-1040) keeps them.
        """
        if FUSED and x.dtype == torch.bfloat16 and self.fusable():
            return self.forward_fused(x, e, context, geom, ring=ring, cross_kv=cross_kv,
                                      kv_out=kv_out)
        if ring is not None or cross_kv is not None or kv_out is not None:
            raise ValueError("Block: the streaming cache and the cached text K/V need the fused "
                             "forward (bf16 activations, per-tensor Fp8Linear).")
        dt = x.dtype
        ep = (self.modulation.float() + e).chunk(6, dim=1)
        ep = [t.reshape(1, -1) for t in ep]
        attn_in = self.norm1(x).float() * (1 + ep[1]) + ep[0]
        y = self.self_attn(attn_in.to(dt), geom)
        x = (x.float() + y.float() * ep[2]).to(dt)
        x = x + self.cross_attn(self.norm3(x), context, geom)
        ffn_in = self.norm2(x).float() * (1 + ep[4]) + ep[3]
        y = self.ffn(ffn_in.to(dt))
        return (x.float() + y.float() * ep[5]).to(dt)


    def _qkv_pack(self):
        """This block's self-attention q, k, v as one stacked fp8 Linear
        (``_fp8_pack``), or None."""
        sa = self.self_attn
        return _fp8_pack(self, "_qkv_pack_cache", [sa.q, sa.k, sa.v])

    def forward_fused(self, x, e, context, geom, ring=None, cross_kv=None, kv_out=None,
                      pending=None, defer=False, kv_only=False, mod=None):
        """The same block with the elementwise chains fused into single-pass kernels.

        LayerNorm + modulation (+ the amax of its output), RMSNorm + RoPE and
        the gated residuals are one kernel each, and each gated residual runs in
        the same pass as the LayerNorm that reads its result
        (``residual_ln_modulate``, bit for bit the two kernels).  ``pending =
        (y, gate)``: the previous block's last residual, not yet applied to
        ``x``, joins this block's first LayerNorm the same way; ``defer``
        returns ``(x, (y, gate))`` with this block's last residual left to the
        caller.  ``kv_only``: only this layer's K and V are computed (into the
        ring or ``kv_out``) and nothing is returned: the forwards whose output is
        discarded need nothing else from their last layer.  The per-tensor fp8
        quantiser of a Linear's input reuses the
        amax its producer wrote, and one quantised input feeds q, k and v
        (likewise the text context for the cross-attention k and v).  The FFN's
        first GEMM writes its bf16 output; one call then looks the GELU up in a
        table, reduces the amax and writes the e4m3 codes the second GEMM
        reads.  The arithmetic at each point is the reference's
        (models.py:1256-1262, :1304-1351); only reduction orders differ.

        With a ``ring`` the RMSNorm + RoPE kernel writes K, and the V GEMM
        writes V, straight into the ring's current-chunk region, and the window
        kernel reads the cached frames in place (no concatenation); with an
        anchored geometry (``geom["anchor"]``) it also reads the LQ anchor from
        the ring's prefix.  ``kv_out = (k, v)`` ([s, dim] views, no ring):
        where the K and V of this layer go instead of scratch tensors -- the
        LQ-anchor harvest writes them into the rings' anchor prefixes.
        The window and cross attention write the amax of their outputs, so the
        output projections' quantisers need only their quantise pass.

        Row-wise Linears (the reference's default scaling, fp8_linear.py:93-103)
        take the same order of operations: every quantiser is the row-wise one
        (one pass per row, no amax words), the GEMMs read per-row activation and
        per-channel weight scales, and the FFN's first GEMM applies the GELU in
        its epilogue before the row-wise quantiser of h.
        """
        sa, ca = self.self_attn, self.cross_attn
        cfg = sa.cfg
        s, dim = x.shape
        n, d = cfg.num_heads, cfg.head_dim
        dev, bf = x.device, torch.bfloat16
        f, h, w = geom["grid"]
        rowwise = sa.q.scaling == "rowwise"
        amax = geom["amax"]
        a0, a1, a2 = (None, None, None) if rowwise else (amax[0:1], amax[1:2], amax[2:3])
        # bf16 modulation + fp32 e in fp32, as .float() + e does (``mod``: the
        # caller computed it with every block's at once)
        if mod is None:
            mod = (self.modulation.float() + e).reshape(6, dim).contiguous()

        def quant_from(t, word):
            """e4m3 codes and scale of t: per row, or per tensor from the amax its
            producer wrote into word."""
            tq = torch.empty(t.shape, dtype=FP8_DTYPE, device=dev)
            if rowwise:
                ts = torch.empty(t.shape[0], dtype=torch.float32, device=dev)
                _lib.fp8_quant_rowwise(t, tq, ts)
            else:
                ts = torch.empty(1, dtype=torch.float32, device=dev)
                _lib.fp8_quant_apply(t, tq, ts, word)
            return tq, ts

        # self-attention
        attn_in = torch.empty(s, dim, dtype=bf, device=dev)
        if pending is None:
            _lib.ln_modulate(x, None, None, mod[1], mod[0], self.norm1.eps, attn_in, a0)
        else:
            xr = torch.empty_like(x)
            _lib.residual_ln_modulate(x, pending[0], pending[1], xr, None, None, mod[1], mod[0],
                                      self.norm1.eps, attn_in, a0)
            x = xr
        xq, xs = quant_from(attn_in, a0)
        pack = self._qkv_pack() if (QKV_PACK and not kv_only and dim % 256 == 0) else None
        if pack is not None:
            # q, k and v from one GEMM over xq; V is then copied to its ring region
            # or the caller's buffer (a 16-byte copy costs less than the GEMM round
            # a separate V GEMM adds at 10,800 rows)
            pw, psb, pbias, _ = pack
            qkv = torch.empty(3, s, dim, dtype=bf, device=dev)
            _lib.fp8_gemm_split(xq, pw, xs.reshape(-1), psb, pbias, qkv)
            q_lin, k_lin, v = qkv[0], qkv[1], qkv[2]
            if ring is None and kv_out is None:
                k = torch.empty(s, dim, dtype=bf, device=dev)
            else:
                vdst = kv_out[1] if ring is None else ring.current_v(0, f).view(s, dim)
                k = kv_out[0] if ring is None else ring.current_k(0, f).view(s, dim)
                _lib.copy_bytes(v, vdst, v.numel() * v.element_size())
                v = vdst
        else:
            q_lin = None if kv_only else sa.q.gemm(xq, xs)
            k_lin = sa.k.gemm(xq, xs)
            if ring is None and kv_out is not None:
                v = sa.v.gemm(xq, xs, out=kv_out[1])
                k = kv_out[0]
            elif ring is None:
                v = sa.v.gemm(xq, xs)
                k = torch.empty(s, dim, dtype=bf, device=dev)
            else:
                v = sa.v.gemm(xq, xs, out=ring.current_v(0, f).view(s, dim))
                k = ring.current_k(0, f).view(s, dim)
        _lib.rmsnorm_rope(k_lin, sa.norm_k.weight, sa.norm_k.eps, geom["rope_cs"], d, k)
        if kv_only:
            return None
        q = torch.empty(s, dim, dtype=bf, device=dev)
        _lib.rmsnorm_rope(q_lin, sa.norm_q.weight, sa.norm_q.eps, geom["rope_cs"], d, q)
        att_out = torch.empty(s, n, d, dtype=bf, device=dev)
        if ring is None:
            bgh.run_blockgrid_hip(q.view(s, n, d), k.view(s, n, d), v.view(s, n, d), att_out,
                                  plan=geom["plan"], f_cur=f, h=h, w=w, n=n, d=d, amax_out=a2)
        elif geom.get("ring_cat"):
            # the reference's concatenation of anchor, cache and chunk (tests only)
            lk, lv = ring.logical(0)
            anc = geom.get("anchor")
            pk = [ring.anchor_k(0)] if anc else []
            pv = [ring.anchor_v(0)] if anc else []
            bgh.run_blockgrid_hip(q.view(s, n, d), torch.cat(pk + [lk, k.view(s, n, d)]),
                                  torch.cat(pv + [lv, v.view(s, n, d)]), att_out,
                                  plan=geom["plan"], f_cur=f, h=h, w=w, n=n, d=d,
                                  anchor_mode=anc, amax_out=a2)
        else:
            bgh.run_blockgrid_hip(q.view(s, n, d), ring.k[0], ring.v[0], att_out,
                                  plan=geom["plan"], f_cur=f, h=h, w=w, n=n, d=d,
                                  anchor_mode=geom.get("anchor"), ring=ring.kernel_ring(),
                                  hr_base=ring.A, amax_out=a2)
        # the output projection's quantiser reuses the amax the attention wrote
        y = sa.o.gemm(*quant_from(att_out.view(s, dim), a2))

        # gated residual and norm3, then the cross-attention
        x1, xn = torch.empty_like(x), torch.empty_like(x)
        _lib.residual_ln_modulate(x, y, mod[2], x1, self.norm3.weight, self.norm3.bias, None, None,
                                  self.norm3.eps, xn, a0)
        xq, xs = quant_from(xn, a0)
        cq = torch.empty(s, dim, dtype=bf, device=dev)
        _lib.rmsnorm_rope(ca.q.gemm(xq, xs), ca.norm_q.weight, ca.norm_q.eps, None, d, cq)
        lc = context.shape[0]
        ck, cv = self.cross_kv(context, geom) if cross_kv is None else cross_kv
        c_out = torch.empty(s, n, d, dtype=bf, device=dev)
        geom["cross"].run(cq.view(s, n, d), ck.view(lc, n, d), cv.view(lc, n, d), c_out,
                          amax_out=a2)
        co = ca.o.gemm(*quant_from(c_out.view(s, dim), a2))

        # residual, norm2 and modulation, then the FFN
        x2, ffn_in = torch.empty_like(x), torch.empty_like(x)
        _lib.residual_ln_modulate(x1, co, geom["ones"], x2, None, None, mod[4], mod[3],
                                  self.norm2.eps, ffn_in, a0)
        xq, xs = quant_from(ffn_in, a0)
        if rowwise:
            hq, hs = quant_from(self.ffn[0].gemm(xq, xs, epilogue=1), None)  # GELU in the epilogue
        elif FFN_GELU_IN_GEMM:
            # GELU and the amax of h in the GEMM's epilogue, then the quantise pass
            hq, hs = quant_from(self.ffn[0].gemm(xq, xs, epilogue=1, amax_out=a1), a1)
        else:
            # the GEMM reduces its largest positive output, which fixes the amax
            # of GELU(x) whenever it is at least 0.375; the table call then skips
            # its amax pass (and runs it otherwise)
            xpos = amax[3:4]
            hlin = self.ffn[0].gemm(xq, xs, epilogue=_lib.GEMM_AMAX_POS, amax_out=xpos)
            hq = torch.empty(hlin.shape, dtype=FP8_DTYPE, device=dev)
            hs = torch.empty(1, dtype=torch.float32, device=dev)
            _lib.fp8_quant_tensor_gelu(hlin, hq, hs, a1, xmax_pos=xpos)  # GELU by table, amax, codes
        y2 = self.ffn[2].gemm(hq, hs)
        if defer:
            return x2, (y2, mod[5])
        return apply_residual(x2, (y2, mod[5]))

    def cross_kv(self, context, geom, context_q=None):
        """The cross-attention's text K (RMSNorm'd) and V, [lc, dim] bf16 each.
        ``context_q``: the context's fp8 codes and scale(s) in this block's scaling
        mode (``quantize_context``), when the caller quantised it once for every
        block."""
        ca = self.cross_attn
        lc, dim = context.shape
        if context_q is None:
            context_q = quantize_context(context, geom, ca.k.scaling == "rowwise")
        cxq, cxs = context_q
        ck = torch.empty(lc, dim, dtype=torch.bfloat16, device=context.device)
        _lib.rmsnorm_rope(ca.k.gemm(cxq, cxs), ca.norm_k.weight, ca.norm_k.eps, None,
                          ca.cfg.head_dim, ck)
        return ck, ca.v.gemm(cxq, cxs)


#: Use the fused block forward when a block's Linears are all per-tensor Fp8Linear.
FUSED = True
#: Per-tensor FFN: True has the first GEMM apply the GELU and reduce the amax of
#: h in its epilogue (the same gelu_tanh and bf16 rounding as the table path, so
#: the same codes), leaving only the quantise pass; False (the default) looks the
#: GELU up in a table over the GEMM's bf16 output (srdit_fp8_quant_tensor_gelu).
#: The c5 forward took 127.3-127.9 ms with True against 123.0-123.8 ms with
#: False (interleaved in one process): tanhf in the epilogue runs while no MFMA
#: does, the table pass runs at memory speed.
FFN_GELU_IN_GEMM = False


def quantize_context(context, geom, rowwise):
    """fp8 codes and scale(s) of the text context for the cross-attention's K and V
    Linears: per row, or per tensor (amax word ``geom["amax_ctx"]``)."""
    return quantize_rowwise(context) if rowwise else quantize_tensor(context, geom["amax_ctx"])


def apply_residual(x, res):
    """bf16(x + y * gate) for res = (y, gate) (models.py:1351)."""
    out = torch.empty_like(x)
    _lib.residual_gate(x, res[0], res[1], out)
    return out


class Head(nn.Module):
    """models.py:1357-1384: modulated LayerNorm and the output Linear, in fp32."""

    def __init__(self, cfg: SRDiTConfig):
        super().__init__()
        self.cfg = cfg
        out = math.prod(cfg.patch_size) * cfg.out_dim
        self.norm = LayerNormF32(cfg.dim, cfg.eps)
        self.head = nn.Linear(cfg.dim, out)
        self.modulation = nn.Parameter(torch.randn(1, 2, cfg.dim) / cfg.dim ** 0.5)

    def forward(self, x, e):
        if x.is_cuda and x.dtype == torch.bfloat16:
            return self.forward_hip(x, e)
        m = (self.modulation.float() + e.float().unsqueeze(1)).chunk(2, dim=1)
        xin = self.norm(x).float() * (1 + m[1].reshape(1, -1)) + m[0].reshape(1, -1)
        return F.linear(xin, self.head.weight.float(), self.head.bias.float())

    def forward_hip(self, x, e):
        """The same arithmetic in two kernels: the LayerNorm's bf16 output
        (srdit_ln_modulate without modulation), then the fp32 Linear that
        applies f32(ln) * (1 + scale) + shift to its input as it reads it
        (srdit_linear_f32_modulated); the weights stay in their dtype (bf16 or
        fp32), as .float() of them is exact."""
        m = self.modulation.float() + e.float().unsqueeze(1)          # [1, 2, dim]
        s1 = (1 + m[0, 1]).contiguous()
        m0 = m[0, 0].contiguous()
        xb = x.contiguous()
        ln = torch.empty_like(xb)
        nw, nb = self.norm.weight, self.norm.bias
        if nw is not None:
            nw, nb = nw.to(torch.bfloat16).contiguous(), nb.to(torch.bfloat16).contiguous()
        _lib.ln_modulate(xb, nw, nb, None, None, self.norm.eps, ln)
        w = self.head.weight
        w = w if w.dtype in (torch.bfloat16, torch.float32) else w.float()
        b = None if self.head.bias is None else self.head.bias.to(w.dtype).contiguous()
        out = torch.empty(x.shape[0], w.shape[0], dtype=torch.float32, device=x.device)
        _lib.linear_f32_modulated(ln, s1, m0, w.contiguous(), b, out)
        return out


class SRDiT(nn.Module):
    """The refiner DiT for one sample: embeddings, blocks, head, unpatchify."""

    def __init__(self, cfg: SRDiTConfig):
        super().__init__()
        self.cfg = cfg
        dim = cfg.dim
        self.patch_embedding = nn.Conv3d(cfg.in_dim, dim, kernel_size=cfg.patch_size,
                                         stride=cfg.patch_size)
        self.text_embedding = nn.Sequential(nn.Linear(cfg.text_dim, dim), nn.GELU(approximate="tanh"),
                                            nn.Linear(dim, dim))
        self.time_embedding = nn.Sequential(nn.Linear(cfg.freq_dim, dim), nn.SiLU(),
                                            nn.Linear(dim, dim))
        self.time_projection = nn.Sequential(nn.SiLU(), nn.Linear(dim, dim * 6))
        self.blocks = nn.ModuleList([Block(cfg) for _ in range(cfg.num_layers)])
        self.head = Head(cfg)

    # -- geometry ---------------------------------------------------------
    def geometry(self, f, h, w, lc, device, t_offset=0):
        """Plans and tables for a (f, h, w) token grid and lc context tokens.

        Built once per grid and reused by every block and every step: the
        window plan (block_hw, radius, +-sym_radius_t frames), the
        cross-attention plan and the RoPE table.
        """
        cfg = self.cfg
        spec = att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=1,
                                  bh=cfg.block_hw[0], bw=cfg.block_hw[1],
                                  rh=cfg.block_radius_hw[0], rw=cfg.block_radius_hw[1],
                                  sym_rt=cfg.sym_radius_t)
        return self._geometry(spec, lc, device, t_offset)

    def stream_geometry(self, f, h, w, lc, device, *, cached, chunk=3, t_offset=0,
                        block_hw=(4, 4), block_radius_hw=(3, 3), anchor=None, anchor_hw=None):
        """Geometry of one streaming chunk: ``f`` query frames against ``cached``
        cached frames plus themselves, under the reference's streaming rule with
        ``block_t = chunk`` and ``rt = f_kv // chunk - 1`` (attention.py:1575-1604
        as models.py:651-676 calls it; the shipped window is 4x4 blocks, radius 3,
        sr_dit_5b.yaml:45-55).  ``anchor`` = "frame" / "chunk": the denoising
        steps' plan with the LQ anchor on the token grid (query frame i sees
        anchor frame i, or every query frame the whole anchor chunk;
        attention.py:1520-1565, blockgrid_triton.py:117-133).  ``anchor_hw``:
        the anchor's own coarser token grid (the native LQ anchor,
        causal_inference.py:725-752), None for the HR grid."""
        if anchor not in (None, "frame", "chunk"):
            raise ValueError(f"stream_geometry: anchor must be None, 'frame' or 'chunk', got {anchor!r}.")
        f_kv = int(cached) + f
        a_hw = None
        if anchor is not None and anchor_hw is not None and tuple(anchor_hw) != (h, w):
            a_hw = (int(anchor_hw[0]), int(anchor_hw[1]))
        spec = att._BlockGridSpec(f_cur=f, f_kv=f_kv, h=h, w=w, block_t=chunk,
                                  bh=block_hw[0], bw=block_hw[1],
                                  rh=block_radius_hw[0], rw=block_radius_hw[1],
                                  rt=max(f_kv // chunk - 1, 0), streaming=True, anchor_hw=a_hw)
        return self._geometry(spec, lc, device, t_offset, anchor=anchor)

    def harvest_geometry(self, f, h, w, lc, device, *, per_frame=True, chunk=3, t_offset=0,
                         block_hw=(4, 4), block_radius_hw=(3, 3), hw_stride=(1, 1)):
        """Geometry of the LQ-anchor harvest forward over ``f`` LQ frames, with no cache
        (causal_inference.py:426-508).  ``per_frame``: the reference runs each frame
        as its own one-frame sample at temporal offset ``t_offset + i``; every op but
        the self-attention is per token, and a one-frame sample's windows see only
        that frame (rt clamps to 0, attention.py:1598-1603), so this is one forward
        over the chunk at ``t_offset`` whose windows each see their own frame
        (``sym_rt = 0``).  Otherwise the whole chunk is one sample without a cache:
        the non-streaming rule with ``block_t = chunk``.  ``hw_stride``: the
        native LQ anchor's harvest runs on the LQ token grid (h, w) with RoPE at
        HR positions (i * s_h, j * s_w)."""
        if per_frame:
            spec = att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=chunk,
                                      bh=block_hw[0], bw=block_hw[1],
                                      rh=block_radius_hw[0], rw=block_radius_hw[1],
                                      rt=0, streaming=False, sym_rt=0)
        else:
            spec = att._BlockGridSpec(f_cur=f, f_kv=f, h=h, w=w, block_t=chunk,
                                      bh=block_hw[0], bw=block_hw[1],
                                      rh=block_radius_hw[0], rw=block_radius_hw[1],
                                      rt=max(f // chunk - 1, 0), streaming=False)
        return self._geometry(spec, lc, device, t_offset, hw_stride=hw_stride)

    def _geometry(self, spec, lc, device, t_offset, anchor=None, hw_stride=(1, 1)):
        cfg = self.cfg
        f, h, w = spec.f_cur, spec.h, spec.w
        rope = rope_table(cfg, f, h, w, t_offset, device, hw_stride=hw_stride)
        return {"grid": (f, h, w), "plan": bgh.cached_plan(spec, anchor_mode=anchor),
                "anchor": anchor, "hw_stride": tuple(hw_stride),
                "cross": CrossAttentionPlan(f * h * w, lc),
                "rope": rope,
                # (cos, sin) pairs [s, head_dim/2] for the fused RMSNorm + RoPE kernel
                "rope_cs": torch.view_as_real(rope).reshape(f * h * w, -1).contiguous(),
                # amax words of the per-tensor quantisers, reused in stream order
                "amax": torch.zeros(4, dtype=torch.int32, device=device),
                "amax_ctx": torch.zeros(1, dtype=torch.int32, device=device),
                "ones": torch.ones(cfg.dim, dtype=torch.float32, device=device)}

    # -- forward pieces -----------------------------------------------------
    def time_embed(self, t):
        """t [1] -> (e [1, dim], e0 [1, 6, dim]), fp32 whatever the weights' dtype, as
        the reference's fp32 autocast region computes them (models.py:1845-1849)."""
        def lin(m, x):
            if not x.is_cuda:
                return F.linear(x, m.weight.float(), None if m.bias is None else m.bias.float())
            # one row: srdit_gemv_f32 reads the weights in their dtype (bf16 or fp32)
            w = m.weight if m.weight.dtype in (torch.bfloat16, torch.float32) else m.weight.float()
            b = None if m.bias is None else m.bias.to(w.dtype).contiguous()
            out = torch.empty(x.shape[0], w.shape[0], dtype=torch.float32, device=x.device)
            _lib.gemv_f32(x.float().contiguous(), w.contiguous(), b, out)
            return out

        te, tp = self.time_embedding, self.time_projection
        e = lin(te[2], F.silu(lin(te[0], sinusoidal_embedding_1d(self.cfg.freq_dim, t).float())))
        e0 = lin(tp[1], F.silu(e)).unflatten(1, (6, self.cfg.dim))
        return e, e0

    def blocks_forward(self, x, e0, context, geom, rings=None, cross=None, kv_outs=None,
                       kv_only=False):
        """The 30-block stack: x [s, dim] bf16 -> [s, dim].  ``rings``/``cross``:
        per-layer streaming KV caches and cached text K/V (or None); ``kv_outs``:
        per-layer (k, v) destinations of the self-attention K/V (or None).
        ``kv_only`` (fused blocks): the stack is run for its layers' K/V alone, the
        last layer stops once its K/V are written, and None is returned."""
        fused = FUSED and x.dtype == torch.bfloat16 and all(b.fusable() for b in self.blocks)
        if kv_only and not fused:
            raise ValueError("SRDiT.blocks_forward: kv_only needs the fused blocks (bf16 "
                             "activations, fp8 Linears).")
        if not fused:
            for i, blk in enumerate(self.blocks):
                x = blk(x, e0, context, geom, ring=None if rings is None else rings[i],
                        cross_kv=None if cross is None else cross[i],
                        kv_out=None if kv_outs is None else kv_outs[i])
            return x
        # fused blocks: each layer's text K/V first (the context quantised once),
        # then the stack, with each block's last residual run in the next block's
        # first LayerNorm pass and the last one applied here
        if cross is None:
            cross = self.cross_cache(context, geom)
        pending = None
        last = len(self.blocks) - 1
        mods = self.block_mods(e0)
        for i, blk in enumerate(self.blocks):
            res = blk.forward_fused(x, e0, context, geom,
                                    ring=None if rings is None else rings[i],
                                    cross_kv=None if cross is None else cross[i],
                                    kv_out=None if kv_outs is None else kv_outs[i],
                                    pending=pending, defer=True, kv_only=kv_only and i == last,
                                    mod=None if mods is None else mods[i])
            if res is None:
                return None
            x, pending = res
        return x if pending is None else apply_residual(x, pending)

    def block_mods(self, e0):
        """Every block's modulation + e0 in fp32 ([layers, 6, dim]), one add over the
        blocks' stacked modulations (kept in fp32, which holds bf16 exactly, and
        rebuilt when one changes), as each block's .float() + e computes it; None
        while a stream is captured with nothing stacked yet."""
        if not self.blocks:
            return None
        key = tuple((b.modulation.data_ptr(), b.modulation._version) for b in self.blocks)
        cached = self.__dict__.get("_mod_stack")
        if cached is None or cached[0] != key:
            if torch.cuda.is_current_stream_capturing():
                return None
            stack = torch.cat([b.modulation.float() for b in self.blocks]).contiguous()
            self.__dict__["_mod_stack"] = cached = (key, stack)
        dim = self.cfg.dim
        return (cached[1] + e0.float().reshape(1, 6, dim)).reshape(len(self.blocks), 6, dim)

    def embed_patches(self, latent):
        """The patch-embedding Conv3d (models.py:1551-1552; kernel = stride = patch)
        as the GEMM it is: latent [C, F, ph*h, pw*w] -> tokens [F*h*w, dim] in
        (frame, row, column) order, and the token grid.  On the GPU the GEMM is
        srdit_bf16_linear (bf16 products, fp32 accumulation, the bias added
        before the one rounding), which also captures in a HIP graph."""
        pt, ph, pw = self.cfg.patch_size
        wgt = self.patch_embedding.weight
        c, fr, hh, ww = latent.shape
        f, h, w = fr // pt, hh // ph, ww // pw
        patches = (latent.to(wgt.dtype).view(c, f, pt, h, ph, w, pw)
                   .permute(1, 3, 5, 0, 2, 4, 6).reshape(f * h * w, c * pt * ph * pw))
        w2 = wgt.reshape(wgt.shape[0], -1)
        if latent.is_cuda and wgt.dtype == torch.bfloat16:
            x = torch.empty(f * h * w, wgt.shape[0], dtype=torch.bfloat16, device=latent.device)
            bias = self.patch_embedding.bias
            _lib.bf16_linear(patches.contiguous(), w2.contiguous(),
                             None if bias is None else bias.contiguous(), x)
            return x, (f, h, w)
        x = F.linear(patches, w2, self.patch_embedding.bias)
        return x.contiguous(), (f, h, w)

    def embed_text(self, context_raw):
        """Text embedding of the padded context (models.py:1860-1866): [lc, dim]."""
        cfg = self.cfg
        dt = self.patch_embedding.weight.dtype
        ctx = context_raw
        if ctx.shape[0] < cfg.text_len:
            ctx = torch.cat([ctx, ctx.new_zeros(cfg.text_len - ctx.shape[0], ctx.shape[1])])
        l0, l2 = self.text_embedding[0], self.text_embedding[2]
        if ctx.is_cuda and dt == torch.bfloat16 and l0.weight.dtype == l2.weight.dtype == dt:
            # the two Linears, the first with the tanh GELU on its rounded output
            # in its epilogue (srdit_bf16_linear)
            x = ctx.to(dt).contiguous()
            hid = torch.empty(x.shape[0], l0.weight.shape[0], dtype=dt, device=x.device)
            _lib.bf16_linear(x, l0.weight, l0.bias, hid, gelu=True)
            out = torch.empty(x.shape[0], l2.weight.shape[0], dtype=dt, device=x.device)
            _lib.bf16_linear(hid, l2.weight, l2.bias, out)
            return out
        return self.text_embedding(ctx.to(dt))

    def _text_kv_pack(self):
        """Every layer's cross-attention k and v weights stacked in one fp8 matrix
        (layer by layer, k then v), their scales as one per-output-channel vector
        and their biases as one vector, for a single split-output GEMM over the
        context; None unless all of them are Fp8Linear of one scaling."""
        return _fp8_pack(self, "_kv_pack",
                         [m for blk in self.blocks for m in (blk.cross_attn.k, blk.cross_attn.v)])

    def cross_cache(self, ctx, geom):
        """Every layer's cross-attention K/V of the embedded context, computed once
        and reused by every step (WanT2VCrossAttention.init_cache, models.py:1035-1040).
        The context is quantised once per scaling mode, not once per layer, and
        when every layer's k and v are fp8 Linears of one scaling they run as one
        GEMM (srdit_fp8_gemm_split): 60 projections of 512 rows each would leave
        most CUs idle one at a time."""
        pack = self._text_kv_pack()
        if pack is not None:
            w, sb, bias, rw = pack
            cxq, cxs = quantize_context(ctx, geom, rw)
            lc, dim = ctx.shape
            kv = torch.empty(2 * len(self.blocks), lc, w.shape[0] // (2 * len(self.blocks)),
                             dtype=torch.bfloat16, device=ctx.device)
            _lib.fp8_gemm_split(cxq, w, cxs.reshape(-1), sb, bias, kv)
            out = []
            for i, blk in enumerate(self.blocks):
                ca = blk.cross_attn
                ck = torch.empty(lc, dim, dtype=torch.bfloat16, device=ctx.device)
                _lib.rmsnorm_rope(kv[2 * i], ca.norm_k.weight, ca.norm_k.eps, None,
                                  ca.cfg.head_dim, ck)
                out.append((ck, kv[2 * i + 1]))
            return out
        quantised, out = {}, []
        for blk in self.blocks:
            rw = blk.cross_attn.k.scaling == "rowwise"
            if rw not in quantised:
                quantised[rw] = quantize_context(ctx, geom, rw)
            out.append(blk.cross_kv(ctx, geom, quantised[rw]))
        return out

    def forward_embedded(self, latent, e, e0, ctx, geom, rings=None, cross=None, kv_outs=None,
                         kv_only=False):
        """Patch embedding, blocks and head for an embedded context and timestep:
        latent [in_dim, f, 2h, 2w] -> [out_dim, f, 2h, 2w] fp32.  ``kv_only``: the
        forward is run for the layers' K/V (into ``rings`` or ``kv_outs``) alone;
        the last layer stops after its K/V, the head is skipped and None is
        returned."""
        cfg = self.cfg
        x, (f, h, w) = self.embed_patches(latent)
        x = self.blocks_forward(x, e0, ctx, geom, rings=rings, cross=cross, kv_outs=kv_outs,
                                kv_only=kv_only)
        if kv_only:
            return None
        return unpatchify(self.head(x, e), (f, h, w), cfg.patch_size, cfg.out_dim)

    def forward(self, latent, t, context_raw, geom):
        """latent [in_dim, f, 2h, 2w] -> [out_dim, f, 2h, 2w] (one sample)."""
        e, e0 = self.time_embed(t)
        return self.forward_embedded(latent, e, e0, self.embed_text(context_raw), geom)


def unpatchify(x, grid, patch_size, c):
    """models.py:2234-2257: [L, c*prod(patch)] -> [c, f*pt, h*ph, w*pw]."""
    f, h, w = grid
    pt, ph, pw = patch_size
    u = x[: f * h * w].view(f, h, w, pt, ph, pw, c)
    u = u.permute(6, 0, 3, 1, 4, 2, 5)
    return u.reshape(c, f * pt, h * ph, w * pw)


def init_weights(model: SRDiT, std=0.02, seed=0):
    """Random N(0, std) Linear/Conv weights, zero biases, N(0,1)/sqrt(dim)
    modulations (the benchmark's synthetic weights; no checkpoint)."""
    g = torch.Generator(device=next(model.parameters()).device).manual_seed(seed)
    with torch.no_grad():
        for m in model.modules():
            if isinstance(m, (nn.Linear, nn.Conv3d)):
                m.weight.copy_(torch.randn(m.weight.shape, generator=g, device=m.weight.device) * std)
                if m.bias is not None:
                    m.bias.zero_()
        for blk in model.blocks:
            blk.modulation.copy_(torch.randn(blk.modulation.shape, generator=g,
                                             device=blk.modulation.device) / model.cfg.dim ** 0.5)
        model.head.modulation.copy_(torch.randn(model.head.modulation.shape, generator=g,
                                                device=model.head.modulation.device)
                                    / model.cfg.dim ** 0.5)
    return model


def build_refiner(cfg: SRDiTConfig, device="cuda", dtype=torch.bfloat16, fp8=True,
                  scaling="tensor", seed=0, num_layers=None):
    """Random-initialised refiner on ``device``; with ``fp8`` every block Linear is an
    Fp8Linear with ``scaling`` ("tensor" or "rowwise").  Blocks are built and
    converted one at a time, so only one block's bf16 weights are ever resident."""
    if num_layers is not None:
        cfg = SRDiTConfig(**{**cfg.__dict__, "num_layers": int(num_layers)})
    proto = SRDiTConfig(**{**cfg.__dict__, "num_layers": 0})
    model = SRDiT(proto).to(device=device, dtype=dtype)
    init_weights(model, seed=seed)
    model.cfg = cfg
    blocks = []
    for i in range(cfg.num_layers):
        blk = Block(cfg).to(device=device, dtype=dtype)
        g = torch.Generator(device=device).manual_seed(seed * 1000 + i + 1)
        with torch.no_grad():
            for m in blk.modules():
                if isinstance(m, nn.Linear):
                    m.weight.copy_(torch.randn(m.weight.shape, generator=g, device=device) * 0.02)
                    m.bias.zero_()
            blk.modulation.copy_(torch.randn(blk.modulation.shape, generator=g, device=device)
                                 / cfg.dim ** 0.5)
        if fp8:
            for parent, names in ((blk.self_attn, ("q", "k", "v", "o")),
                                  (blk.cross_attn, ("q", "k", "v", "o"))):
                for nm in names:
                    setattr(parent, nm, Fp8Linear.from_linear(getattr(parent, nm), scaling=scaling))
            blk.ffn[0] = Fp8Linear.from_linear(blk.ffn[0], scaling=scaling)
            blk.ffn[2] = Fp8Linear.from_linear(blk.ffn[2], scaling=scaling)
        blocks.append(blk)
    model.blocks = nn.ModuleList(blocks)
    return model.eval()
