"""MI355X-native SR-DiT refiner hot path: block-grid window attention and fp8 linears.

Host side in Python on PyTorch-ROCm; compute in hand-written gfx950 HIP kernels
reached through the C ABI of ``libsrdit_hip.so`` (``include/srdit_hip.h``).

Modules mirror video_refiner/wan/modules/sr_dit/ of the reference:
``attention`` (window attention op), ``blockgrid_hip`` (planner + launcher),
``fp8_linear`` (fp8 e4m3 Linear), ``models`` (the one-step refiner forward).
"""
