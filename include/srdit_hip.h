/*
 * srdit_hip.h -- C ABI of libsrdit_hip.so, the MI355X (gfx950) kernels behind
 * the SR-DiT refiner's block-grid window attention and fp8 linears.
 *
 * Plain pointers, sizes and a hipStream_t passed as void*; no framework types.
 * Every entry point returns 0 on success and a nonzero status on failure;
 * srdit_last_error() returns the message of the last failure on the calling
 * thread.  Launches are asynchronous on `stream`; nothing allocates device
 * memory unless its comment says so.  Device pointers must be 16-byte aligned.
 */
#ifndef SRDIT_HIP_H
#define SRDIT_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes */
#define SRDIT_OK 0
#define SRDIT_EINVAL 1       /* bad argument (shape, alignment, mode, null pointer) */
#define SRDIT_EHIP 2         /* a HIP runtime call failed */
#define SRDIT_EUNSUPPORTED 3 /* valid but not implemented (dtype, head dim) */

/* element type codes */
#define SRDIT_DTYPE_BF16 0
#define SRDIT_DTYPE_FP16 1
#define SRDIT_DTYPE_FP32 2  /* fp8 quantiser input; fp32 dense weights */

/*
 * Block-grid window attention, forward.
 *
 * Replaces the launch of the fused window kernels in
 * video_refiner/wan/modules/sr_dit/blockgrid_triton.py:392-422
 * (run_blockgrid_triton -> _blockgrid_fused_kernel :184-278 for mode 0,
 *  _blockgrid_fused_frame_kernel :281-389 for mode 1).
 *
 * q, o        [q_tokens, n_heads, head_dim]  (token stride n_heads*head_dim)
 * k, v        [kv_tokens, n_heads, head_dim] (anchor prefix of hr_base tokens,
 *                                             then the HR KV)
 * params      int32 [n_w, p_stride] device table, the planner's rows
 *             (p_stride 19 for mode 0, 17 for mode 1)
 * order       int32 [n_w] device permutation of window indices: launch order
 * m_tiles     64-row query tiles per window (ceil(max Lq / 64))
 * H, W        token grid of the queries / HR KV
 * scale       softmax scale applied to q.k (head_dim^-1/2 in the reference)
 * mode        0 plain (no anchor or a whole-chunk anchor), 1 per-frame anchor
 * dtype       SRDIT_DTYPE_BF16 or SRDIT_DTYPE_FP16
 * Token indices computed from the table are clamped into the tensors, so a
 * malformed table gives wrong numbers, never an out-of-bounds access.
 */
int srdit_window_attn_fwd(const void* q, const void* k, const void* v, void* o,
                          const int32_t* params, const int32_t* order,
                          int n_w, int m_tiles, int p_stride, int hr_base,
                          int H, int W, int64_t q_tokens, int64_t kv_tokens,
                          int n_heads, int head_dim, float scale, int mode,
                          int dtype, void* stream);

/*
 * Block-grid window attention, forward, plain windows without an anchor prefix,
 * two 64-query members per workgroup sharing their K/V fetches.
 *
 * Replaces the same launch as srdit_window_attn_fwd mode 0
 * (run_blockgrid_triton -> _blockgrid_fused_kernel, blockgrid_triton.py:392-422,
 * :184-278) for tables whose rows all have a_frames == 0.
 *
 * params      int32 [n_w, 19] device table (the planner's plain rows)
 * groups      int32 [n_groups, 4] device table: row0, m_tile0, row1, m_tile1;
 *             row1 = -1 for a single member.  Paired rows must have the same
 *             spatial KV extent (kh0, khL, kw0, kwL); m-tiles are 64 query rows.
 * Other arguments as srdit_window_attn_fwd.
 */
int srdit_window_attn_grouped_fwd(const void* q, const void* k, const void* v, void* o,
                                  const int32_t* params, const int32_t* groups,
                                  int n_w, int n_groups, int hr_base, int H, int W,
                                  int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                  int head_dim, float scale, int dtype, void* stream);

/*
 * The two launches above with two additions, ring addressing and the output's
 * amax; with ring_frames == 0 and amax_out == NULL they are the launches above.
 *
 * Ring: replaces the per-call concatenation of the cached K/V with the chunk's
 * K/V and the tail slice kept as the next cache
 * (video_refiner/wan/modules/sr_dit/attention.py:1506-1510, :964-974), ahead
 * of the launch that srdit_window_attn_fwd / _grouped_fwd replace.
 * k, v         [kv_tokens, n_heads, head_dim] = hr_base anchor tokens, then
 *              ring_frames ring slots of H*W tokens, then the current chunk's
 *              frames.  Logical KV frame f (the frame index of the params
 *              table) lives in slot (ring_head[0] + f) mod ring_frames for
 *              f < ring_cached, and in frame ring_frames + (f - ring_cached)
 *              otherwise.
 * ring_frames  slots of the ring (0: the plain layout; ring_head may then be NULL)
 * ring_cached  cached frames, 0 <= ring_cached <= ring_frames
 * ring_head    device int32, the slot of the oldest cached frame, read by the
 *              kernels at launch (a launch captured in a graph follows the ring
 *              as it advances); a value outside [0, ring_frames) reads as 0.
 * Amax: amax_out (nullable) is cleared, then receives the fp32 bits of
 * max |o| over the written outputs (NaN above infinity): the first pass of
 * the output projection's per-tensor quantiser (fp8_linear.py:80-130), which
 * srdit_fp8_quant_apply then completes.
 * members (grouped only): 2 runs the grouped launch above (two 64-query
 * members per workgroup of four wavefronts); 1 runs one member per workgroup
 * of two wavefronts (row1 of the groups table is ignored), for tables whose
 * members do not pair.
 * anchor_mode (grouped only, needs members == 1): 0 plain rows without an
 * anchor prefix; 2 plain rows with a whole-chunk anchor prefix (a_frames > 0,
 * the launch srdit_window_attn_fwd mode 0 also runs); 1 per-frame anchor rows
 * (p_stride 17, as srdit_window_attn_fwd mode 1).  The anchor keys are walked
 * after the HR keys.
 * Other arguments as srdit_window_attn_fwd / srdit_window_attn_grouped_fwd.
 */
int srdit_window_attn_fwd_ex(const void* q, const void* k, const void* v, void* o,
                             const int32_t* params, const int32_t* order,
                             int n_w, int m_tiles, int p_stride, int hr_base,
                             int H, int W, int64_t q_tokens, int64_t kv_tokens,
                             int n_heads, int head_dim, float scale, int mode,
                             int ring_frames, int ring_cached, const int32_t* ring_head,
                             uint32_t* amax_out, int dtype, void* stream);

int srdit_window_attn_grouped_fwd_ex(const void* q, const void* k, const void* v, void* o,
                                     const int32_t* params, const int32_t* groups,
                                     int n_w, int n_groups, int hr_base, int H, int W,
                                     int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                     int head_dim, float scale, int ring_frames,
                                     int ring_cached, const int32_t* ring_head,
                                     uint32_t* amax_out, int members, int anchor_mode, int dtype,
                                     void* stream);

/*
 * Block-grid window attention, forward, plain windows without an anchor prefix,
 * one workgroup per 64-row tile, where a tile may hold the queries of two
 * windows (the end of one, the start of the next).
 *
 * Replaces the same launch as srdit_window_attn_fwd mode 0
 * (run_blockgrid_triton -> _blockgrid_fused_kernel, blockgrid_triton.py:392-422,
 * :184-278) for tables whose rows all have a_frames == 0 and at most 16 KV
 * frames.  Windows of fewer than 64 queries (48 for 4x4-token blocks over three
 * frames) otherwise pad their tile; two of them share one here.
 *
 * tiles       int32 [n_tiles, 5] device table: row A, A's first query, A's rows
 *             in the tile (1..64), row B or -1, B's first query.  Tile row r is
 *             query (first + r) of A for r below A's rows, else query
 *             (B's first + r - A's rows) of B; rows past a window's queries are
 *             not written.  A and B must have the same query frames and the
 *             same KV frames and token rows, and their KV column ranges must
 *             span exactly 32 columns together: the tile walks that union and
 *             each query drops the columns outside its own window.
 * Other arguments as srdit_window_attn_grouped_fwd_ex (members 1, anchor_mode 0).
 */
int srdit_window_attn_packed_fwd(const void* q, const void* k, const void* v, void* o,
                                 const int32_t* params, const int32_t* tiles,
                                 int n_w, int n_tiles, int hr_base, int H, int W,
                                 int64_t q_tokens, int64_t kv_tokens, int n_heads,
                                 int head_dim, float scale, int ring_frames, int ring_cached,
                                 const int32_t* ring_head, uint32_t* amax_out, int dtype,
                                 void* stream);

/*
 * Dense attention: o[i, h] = softmax(q[i, h] . k[:, h]^T * scale) v[:, h] for
 * every query token i and head h, over all kv_tokens keys.  q and o are
 * [q_tokens, n_heads, head_dim], k and v [kv_tokens, n_heads, head_dim], all
 * contiguous.  Replaces the attention of WanT2VCrossAttention.forward
 * (models.py:1042-1062): the video tokens' queries over the text context's
 * keys and values.  Persistent workgroups that prefetch the next 128 queries
 * while the current ones run; the numerics of the window kernels (q scaled by
 * scale*log2(e) and rounded once, base-2 softmax, P rounded to the input type,
 * fp32 accumulation).  amax_out (nullable): cleared, then max |o| (fp32 bits).
 * head_dim 64 or 128, bf16 or fp16, token strides below 16384 bytes, Q/O and
 * K/V below 2^31 bytes each.
 */
int srdit_dense_attn_fwd(const void* q, const void* k, const void* v, void* o,
                         int64_t q_tokens, int64_t kv_tokens, int n_heads, int head_dim,
                         float scale, uint32_t* amax_out, int dtype, void* stream);

/*
 * Row-wise fp8 e4m3 quantiser: for each row of x [M, K] (row stride ldx),
 *   scale[m] = max(amax(|x[m,:]|) * fl32(1/448), 1e-12)   (fp32; what torch computes
 *              for amax / 448.0 on a GPU tensor)
 *   xq[m,k]  = e4m3(clamp(x[m,k] / scale[m], -448, 448))   (round to nearest even)
 * Replaces _quantize_rowwise_impl (video_refiner/wan/modules/sr_dit/fp8_linear.py:93-103),
 * used for the activation on every Fp8Linear call and for the weight once.
 * x is bf16, fp16 or fp32 (dtype); xq [M, K] contiguous OCP e4m3fn bytes;
 * scale [M] float.  K % 8 == 0, ldx % 8 == 0.
 */
int srdit_fp8_quant_rowwise(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                            void* xq, float* scale, void* stream);

/*
 * Per-tensor fp8 e4m3 quantiser, three launches on `stream`: clear amax_ws (a
 * fill kernel, so the sequence can be captured in a graph), amax of |x| over
 * all of x [M, K] into amax_ws (one uint32 holding the float's bits, device),
 * then scale[0] = max(amax * fl32(1/448), 1e-12) and xq = e4m3(clamp(x / scale, +-448)).
 * The per-tensor mode of the fp8 Linear: the reference quantises row-wise
 * (fp8_linear.py:93-103) and names per-tensor scaling as its faster
 * alternative (fp8_linear.py:22, :31-38).  Same dtype and layout rules as the
 * row-wise quantiser.
 */
int srdit_fp8_quant_tensor(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                           void* xq, float* scale, uint32_t* amax_ws, void* stream);

/*
 * Scaled fp8 GEMM:  out[m, n] = bf16( sum_k a[m,k] b[n,k] * sa[m or 0] * sb[n or 0]
 *                                     + bias[n] )
 * a [M, K] e4m3 row-major, b [N, K] e4m3 row-major (the nn.Linear weight
 * layout), fp32 accumulate, bias bf16 [N] or NULL, out bf16 [M, N] with row
 * stride ldo.  sa_rows is 1 (per-tensor) or M (row-wise); sb_cols is 1 or N.
 * Replaces torch._scaled_mm(xq, w_fp8.t(), scale_a, scale_b, bias,
 * out_dtype=bf16) in Fp8Linear.forward (fp8_linear.py:282-297); the bias is
 * applied to the fp32 value before the single bf16 rounding, as the reference's
 * epilogue does (fp8_linear.py:238-241).
 * Runs on one hand-written MFMA kernel for every shape and scale mode (one
 * persistent workgroup per CU).  Requires K % 128 == 0, N % 16 == 0,
 * ldo % 8 == 0 with (255 * ldo + N) * 2 + 16 below 2^31, M*K and N*K below
 * 2^31; a, b, out and bias
 * 16-byte aligned, and sa / sb too when they hold one scale per row / column.
 */
int srdit_fp8_gemm(const void* a, const void* b, const float* sa, int64_t sa_rows,
                   const float* sb, int64_t sb_cols, const void* bias, void* out,
                   int64_t M, int64_t N, int64_t K, int64_t ldo, void* stream);

/*
 * The scaled fp8 GEMM with an epilogue: epilogue 0 stores bf16(v) as
 * srdit_fp8_gemm does; epilogue 1 stores bf16(gelu_tanh(bf16(v))), the
 * Linear's bf16 output fed to nn.GELU(approximate='tanh') as the FFN does
 * (models.py:1200-1202).  amax_out (nullable, one uint32, device): cleared by
 * the call, then set to the bits of max |out| for a per-tensor quantiser of
 * the output (srdit_fp8_quant_apply).  Same layout rules as srdit_fp8_gemm.
 */
/*
 * The scaled fp8 GEMM with its output split into column blocks: columns
 * [j split_n, (j + 1) split_n) of out = a . b^T * sa * sb + bias go to
 * out + j * split_stride (elements) as an [M, split_n] block with row stride
 * ldo.  For several Linears that read one input: their weights stacked into b
 * (and their scales into sb, their biases into bias) make one GEMM whose
 * blocks are the separate outputs.  The refiner uses it for the text K and V
 * of every layer, WanT2VCrossAttention.init_cache's k and v Linears over the
 * one context (models.py:1035-1040, :1042-1062) run as per-layer
 * Fp8Linear.forward calls in the reference (fp8_linear.py:282-297).
 * Requires split_n % 256 == 0, N % split_n == 0, split_stride >= M * ldo and a
 * multiple of 8; other rules as srdit_fp8_gemm.
 */
int srdit_fp8_gemm_split(const void* a, const void* b, const float* sa, int64_t sa_rows,
                         const float* sb, int64_t sb_cols, const void* bias, void* out,
                         int64_t M, int64_t N, int64_t K, int64_t ldo, int64_t split_n,
                         int64_t split_stride, void* stream);

/*
 * The FFN's hidden activation and its per-tensor e4m3 quantiser: quantises
 * h = bf16(gelu_tanh(x)) for x [M, K] bf16 (row stride ldx) as
 * srdit_fp8_quant_tensor does (same outputs, same workspace rule).  h is looked
 * up in a table of all 65,536 bf16 inputs, rebuilt by every call in a static
 * 128 KB device array (no allocation); x is read twice (amax, then codes) and
 * not modified.  h (nullable; row stride ldh, not x): also stores h there.  The
 * GELU of models.py:1200-1202 on the first Linear's bf16 output, then the
 * second Linear's per-tensor quantiser (fp8_linear.py:80-130 with one scale).
 * bf16 only.
 */
int srdit_fp8_quant_tensor_gelu(const void* x, int64_t M, int64_t K, int64_t ldx, void* h,
                                int64_t ldh, void* xq, float* scale, uint32_t* amax_ws,
                                void* stream);

/*
 * srdit_fp8_quant_tensor_gelu with the largest positive value of x, as the
 * producing GEMM wrote it (srdit_fp8_gemm_ex with SRDIT_GEMM_AMAX_POS), in
 * xmax_pos (device uint32, nullable).  When it is at least 0.375 the amax of
 * h is the table's value there (h is non-decreasing over x >= 0 and |h| <=
 * 0.17 below 0), so the amax pass over x is skipped; otherwise, or with h
 * non-null, the call is srdit_fp8_quant_tensor_gelu.  Same codes and scale
 * either way.  Replaces the same reference steps (models.py:1200-1202,
 * fp8_linear.py:80-130).
 */
int srdit_fp8_quant_tensor_gelu_ex(const void* x, int64_t M, int64_t K, int64_t ldx, void* h,
                                   int64_t ldh, void* xq, float* scale, uint32_t* amax_ws,
                                   const uint32_t* xmax_pos, void* stream);

/* Flag for the epilogue argument of srdit_fp8_gemm_ex, kept for callers that
 * still pass it: it once selected the hand-written kernel over a library path.
 * Every GEMM runs on that kernel now; the flag is accepted and has no effect. */
#define SRDIT_GEMM_MFMA 0x100

/* Flag for the epilogue argument of srdit_fp8_gemm_ex (epilogue 0 only):
 * amax_out receives the largest positive output instead of max |out| (the
 * float bits of a non-negative value, 0 when every output is negative, the
 * bits of a NaN when an output is NaN).  No counterpart in the reference: it
 * lets srdit_fp8_quant_tensor_gelu_ex skip its amax pass. */
#define SRDIT_GEMM_AMAX_POS 0x200

int srdit_fp8_gemm_ex(const void* a, const void* b, const float* sa, int64_t sa_rows,
                      const float* sb, int64_t sb_cols, const void* bias, void* out,
                      int64_t M, int64_t N, int64_t K, int64_t ldo, int epilogue,
                      uint32_t* amax_out, void* stream);

/* Bytes of workspace with which srdit_fp8_gemm_ws may split any GEMM's last
 * round of tiles (256 workgroups of fp32 partials and the counters). */
#define SRDIT_GEMM_WS_BYTES ((int64_t)4096 + (int64_t)256 * 262144)

/*
 * srdit_fp8_gemm_ex with the output split of srdit_fp8_gemm_split (split_n 0:
 * none) and a workspace (nullable) for a split-K tail: when the tiles of the
 * output leave the last round of the persistent launch nearly empty and K is
 * long (10800 x 3072 x 14336: 516 tiles, two rounds of 256 CUs and 4 tiles of
 * 112 K stages), those tiles run in a second launch, each split along K over
 * a few workgroups whose fp32 partials are summed in K order by the last of
 * them to finish.  The results
 * differ from the unsplit GEMM's only by the fp32 summation order.  The
 * workspace (16-byte aligned, device) must hold zeros in its first 4096 bytes
 * when first used (every call leaves them zero); up to workspace_bytes of it
 * are used, SRDIT_GEMM_WS_BYTES allows every split.  Calls that share a
 * workspace must be ordered (one stream).  Replaces what srdit_fp8_gemm_ex
 * and srdit_fp8_gemm_split do (fp8_linear.py:282-297; models.py:1035-1062).
 */
int srdit_fp8_gemm_ws(const void* a, const void* b, const float* sa, int64_t sa_rows,
                      const float* sb, int64_t sb_cols, const void* bias, void* out,
                      int64_t M, int64_t N, int64_t K, int64_t ldo, int epilogue,
                      uint32_t* amax_out, int64_t split_n, int64_t split_stride,
                      void* workspace, int64_t workspace_bytes, void* stream);

/*
 * The quantise pass of srdit_fp8_quant_tensor alone: amax_ws already holds the
 * bits of max |x| (written by a producer: srdit_ln_modulate or
 * srdit_fp8_gemm_ex), scale[0] = max(amax * fl32(1/448), 1e-12) and
 * xq = e4m3(clamp(x / scale, +-448)).
 */
int srdit_fp8_quant_apply(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                          void* xq, float* scale, const uint32_t* amax_ws, void* stream);

/*
 * Fused LayerNorm + adaLN modulation, one pass per row of x [M, K] (bf16):
 *   y = bf16(LayerNorm(x; eps) [* ln_w + ln_b])      (ln_w, ln_b bf16 [K] or both NULL)
 *   out = bf16(f32(y) * (1 + scale) + shift)          (scale, shift fp32 [K] or both NULL)
 * WanLayerNorm (video_refiner/wan/modules/sr_dit/models.py:443-503) followed by
 * the block's modulation (models.py:1308, :1258).  amax_ws (nullable): cleared,
 * then max |out| bits, for srdit_fp8_quant_apply.  K % 8 == 0, 16-byte rows.
 */
int srdit_ln_modulate(const void* x, int64_t M, int K, int64_t ldx, const void* ln_w,
                      const void* ln_b, const float* scale, const float* shift, float eps,
                      void* out, int64_t ldo, uint32_t* amax_ws, void* stream);

/*
 * Gated residual: out = bf16(f32(x) + f32(y) * gate[k]) over [M, K] bf16,
 * gate fp32 [K]; out may alias x.  The block's residual updates
 * (models.py:1344, :1260).
 */
int srdit_residual_gate(const void* x, const void* y, const float* gate, int64_t M, int K,
                        int64_t ldx, int64_t ldy, void* out, int64_t ldo, void* stream);

/*
 * The gated residual and the LayerNorm that reads its result, in one pass:
 *   x_out = bf16(f32(x) + f32(y) * gate[k])                 (srdit_residual_gate)
 *   out   = srdit_ln_modulate(x_out, ln_w, ln_b, scale, shift, eps, amax_ws)
 * with the same arithmetic as the two calls (bit for bit).  A residual update
 * of the block followed by the norm that reads the new residual stream
 * (models.py:1344-1345 then norm3 at :1257; :1257 then norm2 at :1258).
 * gate fp32 [K] 16-byte aligned; x_out and out are buffers of their own
 * (neither aliases x, y or the other).  K > 4096 runs the two kernels.
 */
int srdit_residual_ln_modulate(const void* x, const void* y, const float* gate, int64_t M, int K,
                               int64_t ldx, int64_t ldy, void* x_out, int64_t ldxo,
                               const void* ln_w, const void* ln_b, const float* scale,
                               const float* shift, float eps, void* out, int64_t ldo,
                               uint32_t* amax_ws, void* stream);

/*
 * RMSNorm over each row of x [M, K] (bf16, K = heads * head_dim) with weight w
 * (bf16 [K]), then RoPE per head: pair j of a head rotated by
 * (cos, sin) = rope_cs[row][j] (fp32 pairs, [M, head_dim/2]); rope_cs NULL skips
 * the rotation (RMSNorm alone).  out [M, K] contiguous.  WanRMSNorm
 * (models.py:424-440) then rope_apply (models.py:173-214).
 */
int srdit_rmsnorm_rope(const void* x, int64_t M, int K, int64_t ldx, const void* w, float eps,
                       const float* rope_cs, int head_dim, void* out, void* stream);

/*
 * Dense Linears at the two ends of the forward (csrc/dense.hip).  Products
 * exact, fp32 accumulators, the bias added to the accumulator before the one
 * rounding to the output type; only the summation order differs from torch's
 * GEMMs on the same dtypes.  Row strides in elements; A and W rows 16-byte
 * aligned.
 *
 * srdit_bf16_linear: out [M, N] = bf16(a [M, K] @ w [N, K]^T + bias [N]), all
 * bf16 (bias may be NULL), K % 16 == 0; epilogue 1 then stores
 * bf16(gelu_tanh(out)) of the rounded value.  Replaces the patch embedding's
 * Conv3d with kernel = stride = patch (video_refiner/wan/modules/sr_dit/
 * models.py:1551-1552, called at :1837) as a GEMM over the patches, and
 * the text embedding's Linear - GELU(tanh) - Linear (models.py:1553-1556,
 * called at :1860-1866).
 */
int srdit_bf16_linear(const void* a, int64_t lda, const void* w, int64_t ldw, const void* bias,
                      void* out, int64_t ldo, int64_t M, int64_t N, int64_t K, int epilogue,
                      void* stream);

/*
 * out [M, N] fp32 = xin @ w^T + bias with xin = (f32(a) * s1) + m0 rounded
 * after the product and after the sum: a [M, K] bf16, s1 and m0 fp32 [K]
 * (16-byte aligned), w [N, K] and bias [N] both bf16 (w_dtype
 * SRDIT_DTYPE_BF16) or both fp32 (SRDIT_DTYPE_FP32), bias may be NULL;
 * K % 16 == 0.  Replaces Head.forward's modulation and fp32 Linear
 * (models.py:1372-1384) after its LayerNorm (srdit_ln_modulate with no
 * modulation gives that LayerNorm's bf16 output).
 */
int srdit_linear_f32_modulated(const void* a, int64_t lda, const float* s1, const float* m0,
                               const void* w, int64_t ldw, const void* bias, int w_dtype,
                               float* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                               void* stream);

/*
 * out [M, N] fp32 = x [M, K] fp32 @ w [N, K]^T + bias, w and bias both bf16 or
 * both fp32 (w_dtype), bias may be NULL; K % 8 == 0, M < 65536.  One wave per
 * output: for the time embedding's and time projection's Linears on the
 * one-row sinusoid (models.py:1845-1849, the fp32 region of the timestep MLP).
 */
int srdit_gemv_f32(const float* x, int64_t ldx, const void* w, int64_t ldw, const void* bias,
                   int w_dtype, float* out, int64_t ldo, int64_t M, int64_t N, int64_t K,
                   void* stream);

/* Message of the last failed call on this thread (NUL-terminated, truncated to
 * len).  Returns the message length. */
int srdit_last_error(char* buf, int len);

/* Library version, packed as major*10000 + minor*100 + patch. */
int srdit_version(void);

/*
 * Measurement helper with no counterpart in the reference: copies `bytes`
 * (a multiple of 16) from src to dst with 16-byte vector loads and stores.
 * Used to calibrate hardware byte counters against a kernel of known traffic.
 */
int srdit_copy_bytes(const void* src, void* dst, int64_t bytes, void* stream);

/* Capacity of the static scratch of srdit_fp8_linear_tensor_static, in e4m3
 * codes of the activation: M*K may not exceed it (64 MiB). */
#define SRDIT_LINEAR_SCRATCH_CODES ((int64_t)64 << 20)

/*
 * No counterpart in the reference: for callers that cannot allocate (code
 * under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The per-tensor fp8 Linear in one call that allocates nothing:
 *   out = srdit_fp8_gemm_ex(e4m3(x / s_x), w, s_x, w_scale, bias) with
 *   s_x = max(amax(|x|) * fl32(1/448), 1e-12),
 * the same kernels and results as srdit_fp8_quant_tensor followed by
 * srdit_fp8_gemm_ex(..., SRDIT_GEMM_MFMA, NULL), with the amax word, the
 * scale and the activation codes in a static per-device scratch array
 * instead of caller buffers.  Rejects M*K > SRDIT_LINEAR_SCRATCH_CODES
 * (SRDIT_EINVAL).  x [M, K] bf16/fp16/fp32 (dtype, row stride ldx); w [N, K]
 * e4m3; w_scale [1] or [N] (w_scale_cols 1 or N); bias bf16 [N] or NULL;
 * out bf16 [M, N] (row stride ldo).  Calls that overlap on one device race
 * on the shared scratch; each device holds its array until the process ends.
 */
int srdit_fp8_linear_tensor_static(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype,
                                   const void* w, const float* w_scale, int64_t w_scale_cols,
                                   const void* bias, void* out, int64_t N, int64_t ldo,
                                   void* stream);

#ifdef __cplusplus
}
#endif

#endif /* SRDIT_HIP_H */
