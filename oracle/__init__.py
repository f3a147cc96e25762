"""Oracle: CPU restatement of the reference algorithms for the window-attention and
fp8-linear path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the reference that outputs are
compared against (or the timed CPU baseline) -- never as the thing measured or
shipped.  The product path in
``dreamx-creator_amd/sr_dit`` must not import it and has no CPU fallback.

Modules
  blockgrid   planner restatement (windows, temporal rules, params rows), the
              per-token closed-form visibility rule, float64 numpy attention
  gather_torch  torch restatement of the reference gather backend
              (index_select + SDPA + index_copy_), the CPU baseline
  fp8         closed-form row-wise / per-tensor e4m3 quantiser and the
              dequantised GEMM

Pinning (what checks each function, beyond retyping):
  * params rows / temporal runs: golden fixtures written by the reference's own
    build_plan and _BlockGridSpec (tests/golden/make_golden.py), plus the
    per-token block-distance rule (a different formulation) on tiny grids;
  * window attention: dense masked softmax attention in float64 with the
    per-token mask (brute force), and the one-window case == plain attention;
  * fp8 quantiser: torch's float8_e4m3fn cast (RNE) as the library oracle and
    hand-computed e4m3 encodings;
  * fp8 GEMM: float64 dequantised matmul.
"""
