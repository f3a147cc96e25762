"""Benchmark: block-grid window attention at 2K (6x45x80 = 21,600 tokens, 24x128, bf16).

One step = one window-attention layer forward over the full 2K latent (the
fused HIP kernel, one launch), inputs resident in HBM.  Reports useful TFLOP/s
(sum over windows and heads of 4*Lq*Lkv*d) and the fraction of MI355X dense
bf16 MFMA peak, plus the reference's gather path restated in torch, timed on
the host CPU over a bounded sample, as a baseline only.

    python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--config c3]
"""
from __future__ import annotations

import argparse
import hashlib
import json
import os
import platform
import re
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "dreamx-creator_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0      # MI355X dense bf16 MFMA, spec sheet
PEAK_HBM_GBS = 8000.0          # MI355X HBM3E, spec sheet
CONFIG_DESC = {
    "c2": "window attention 1080p latent 6x34x60 (12,240 tok), 24 heads x 128, 8x8 blocks, 3x3 nbhd, +-1 frame",
    "c3": "window attention 2K latent 6x45x80 (21,600 tok), 24 heads x 128, 8x8 blocks, 3x3 nbhd, +-1 frame",
    "c4": "AR window attention: 2x45x80 query frames vs 4 cached + 2 current frames, 24 heads x 128, 8x8 blocks, 3x3 nbhd",
}


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c3", choices=sorted(CONFIG_DESC))
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-step", action="store_true",
                    help="skip the SR-DiT refiner step (30 blocks, hipGraph) measurement")
    ap.add_argument("--no-prod", action="store_true",
                    help="skip the shipped-geometry (4x4 blocks, radius 3) window timings")
    ap.add_argument("--no-stream", action="store_true",
                    help="skip the streaming SR loop (chunks over the ring KV cache) measurement")
    ap.add_argument("--step-iters", type=int, default=50,
                    help="timed graph replays of the refiner forward (median reported)")
    ap.add_argument("--no-rowwise", action="store_true",
                    help="skip the refiner forward with row-wise fp8 scales")
    ap.add_argument("--cpu-seconds", type=float, default=20.0,
                    help="rough budget for the CPU baseline sample")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="only run the library's 16-byte copy kernel over BYTES (counter calibration)")
    ap.add_argument("--settle-ms", type=float, default=100.0,
                    help="untimed launches of the c3 step for this long before the warm-up "
                         "(0: none), so the timed steps see the sustained-load clock")
    ap.add_argument("--no-comparator", action="store_true",
                    help="skip the torch gather + SDPA comparator on the GPU")
    ap.add_argument("--no-gemm", action="store_true",
                    help="skip the fp8 GEMM timings at the refiner's projection shapes")
    ap.add_argument("--source-hash", action="store_true",
                    help="only print the hash of the sources that decide the window kernel's traffic")
    return ap.parse_args()


def copy_calibration(nbytes, reps=5):
    """Launch the plain copy kernel `reps` times over `nbytes`: a kernel of known traffic
    (nbytes read + nbytes written per launch) to scale hardware byte counters against."""
    import torch
    from sr_dit import _lib
    src = torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(1)
    dst = torch.empty_like(src)
    for _ in range(reps):
        _lib.copy_bytes(src, dst, nbytes)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes": nbytes, "launches": reps}), flush=True)


# The files that decide the window kernel's memory traffic on a workload: its
# source, the launcher's tables and launch order, the workload shapes and the
# compiler flags.
TRAFFIC_SOURCES = ("dreamx-creator_amd/csrc/window_group.hip",
                   "dreamx-creator_amd/csrc/window_common.h",
                   "dreamx-creator_amd/csrc/common.h",
                   "dreamx-creator_amd/sr_dit/blockgrid_hip.py",
                   "dreamx-creator_amd/sr_dit/workloads.py",
                   "dreamx-creator_amd/sr_dit/build.py")


def traffic_source_hash():
    """sha256 (16 hex digits) over the traffic-deciding sources, names included."""
    h = hashlib.sha256()
    for rel in TRAFFIC_SOURCES:
        h.update(rel.encode())
        with open(os.path.join(ROOT, rel), "rb") as f:
            h.update(f.read())
    return h.hexdigest()[:16]


def profile_traffic(config):
    """(HBM bytes per launch, where from) out of the committed rocprofv3 PMC summary.

    The summary records the source hash of the build it measured; a summary of
    other sources is stale and gives no figure (None), so a kernel change never
    reports the old kernel's traffic."""
    rel = f"profiles/window_attn_{config}_pmc.md"
    path = os.path.join(ROOT, rel)
    if not os.path.exists(path):
        return None, f"no PMC summary {rel}"
    text = open(path).read()
    m = re.search(r"traffic_bytes_per_launch:\s*([0-9.eE+]+)", text)
    hm = re.search(r"source_hash:\s*([0-9a-f]+)", text)
    cur = traffic_source_hash()
    if not m:
        return None, f"{rel} holds no traffic figure"
    if not hm or hm.group(1) != cur:
        return None, (f"stale: {rel} measured sources {hm.group(1) if hm else '(unstamped)'}, "
                      f"the current sources are {cur}")
    return float(m.group(1)), f"{rel} (FETCH_SIZE + WRITE_SIZE, sources {cur})"


def cpu_baseline(config, budget_s):
    """The oracle's torch gather path (fp32) on the host cores, bounded sample.

    Sample: the windows of one interior query frame (frame 2: 60 windows of the
    6x45x80 grid), all 24 heads, fp32, same seeded inputs.  3 warm-up runs, then
    the median of up to 10 timed runs within the budget.
    """
    import torch
    from oracle import blockgrid as obg
    from oracle import gather_torch as ogt
    from sr_dit import workloads as wl

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)
    c = wl.WINDOW_CONFIGS[config]
    q, k, v, kc, vc = wl.make_window_inputs(config, torch.float32, "cpu", seed=0)
    q, k, v = q[0], k[0], v[0]
    if kc is not None:
        k, v = torch.cat([kc[0], k]), torch.cat([vc[0], v])
    spec = wl.window_spec(config)
    g = obg.Geometry(**{f: getattr(spec, f) for f in obg.Geometry.__dataclass_fields__})
    wins = obg.windows(g)
    L = c["h"] * c["w"]
    frame = min(2, c["f_cur"] - 1)
    sample = [w for w in wins if w[0][0] // L == frame] if c["rule"] == "sym1" else wins[:12]
    flops = sum(4 * len(a) * len(b) * wl.HEAD_DIM for a, b in sample) * wl.N_HEADS
    plan = ogt.GatherPlan(g)
    # restrict the plan to the sample windows
    keep = {int(a[0]) for a, _ in sample}
    groups = []
    for grp in plan.groups:
        qs = grp["q"].view(grp["Nw"], grp["Lq"])
        kvs = grp["kv"].view(grp["Nw"], grp["Lkv"])
        sel = [i for i in range(grp["Nw"]) if int(qs[i, 0]) in keep]
        if sel:
            groups.append({"q": qs[sel].reshape(-1), "kv": kvs[sel].reshape(-1), "Nw": len(sel),
                           "Lq": grp["Lq"], "Lkv": grp["Lkv"]})
    plan.groups = groups
    times = []
    t_start = time.perf_counter()
    for i in range(13):
        t0 = time.perf_counter()
        ogt.gather_attend(plan, q, k, v)
        dt = time.perf_counter() - t0
        if i >= 3:
            times.append(dt)
        if time.perf_counter() - t_start > budget_s and len(times) >= 3:
            break
    med = statistics.median(times)
    cpu_model = ""
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                cpu_model = line.split(":", 1)[1].strip()
                break
    except OSError:
        cpu_model = platform.processor()
    # The CPU configuration itself (c1: 3x16x16, 768 tokens), every window, timed
    # whole: the reference's CPU-runnable case.
    q1, k1, v1, _, _ = wl.make_window_inputs("c1", torch.float32, "cpu", seed=0)
    q1, k1, v1 = q1[0], k1[0], v1[0]
    spec1 = wl.window_spec("c1")
    g1 = obg.Geometry(**{f: getattr(spec1, f) for f in obg.Geometry.__dataclass_fields__})
    plan1 = ogt.GatherPlan(g1)
    flops1 = sum(4 * len(a) * len(b) * wl.HEAD_DIM for a, b in obg.windows(g1)) * wl.N_HEADS
    t1 = []
    for i in range(23):
        t0 = time.perf_counter()
        ogt.gather_attend(plan1, q1, k1, v1)
        if i >= 3:
            t1.append(time.perf_counter() - t0)
    med1 = statistics.median(t1)
    c1_full = {"ms": round(med1 * 1e3, 3), "tflops": round(flops1 / med1 / 1e12, 4),
               "useful_gflop": round(flops1 / 1e9, 3), "windows": len(obg.windows(g1)),
               "runs": len(t1), "workload": "c1 3x16x16 (768 tokens), 24 heads x 128, fp32, all windows"}
    return {"value": flops / med / 1e12, "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "c1_full": c1_full,
            "sample": (f"{config} query frame {frame}: {len(sample)} windows x 24 heads, fp32, "
                       f"{flops / 1e9:.2f} GFLOP useful, median of {len(times)} runs "
                       f"{med * 1e3:.1f} ms; os.cpu_count()={os.cpu_count()}; {cpu_model}")}


def build_model(layers=30, scaling="tensor"):
    """The 5B refiner (random weights, fp8 Linears with ``scaling`` scales) and its build time."""
    import torch
    from sr_dit import model as mdl

    t0 = time.perf_counter()
    model = mdl.build_refiner(mdl.SRDiTConfig(num_layers=layers), device=torch.device("cuda:0"),
                              scaling=scaling, seed=0)
    return model, time.perf_counter() - t0


def refiner_step(model, build_s, replays, warmup):
    """One SR-DiT 5B refiner forward at 2K, whole: time and text embeddings, patch
    embedding of the 48x6x90x160 latent, 30 blocks (fp8 linears, window
    self-attention as in c3, cross-attention to 512 text tokens), head and
    unpatchify (models.py:1827-1875, :2234-2257), captured once in a HIP graph.
    Each replay is timed on its own with HIP events on the replay stream; the
    median and mean over ``replays`` replays are reported."""
    import torch
    from sr_dit import workloads as wl
    from sr_dit.fp8_linear import Fp8Linear

    dev = torch.device("cuda:0")
    cfg = model.cfg
    layers = cfg.num_layers
    f, h, w = 6, 45, 80
    s_tok = f * h * w
    geom = model.geometry(f, h, w, cfg.text_len, dev)
    g = torch.Generator("cpu").manual_seed(0)
    latent = torch.randn(cfg.in_dim, f, 2 * h, 2 * w, generator=g).to(dev)
    ctx_raw = torch.randn(cfg.text_len, cfg.text_dim, generator=g).to(torch.bfloat16).to(dev)
    t = torch.tensor([625.0], device=dev)

    def fwd():
        return model.forward(latent, t, ctx_raw, geom)

    # useful work: every fp8 GEMM (2*M*N*K), window attention and cross-attention
    gemm = 0
    for blk in model.blocks:
        for m in blk.modules():
            if isinstance(m, Fp8Linear):
                rows = cfg.text_len if m in (blk.cross_attn.k, blk.cross_attn.v) else s_tok
                gemm += 2 * rows * m.in_features * m.out_features
    win = wl.plan_useful_flops(geom["plan"]) * layers
    cross = 4 * s_tok * cfg.text_len * cfg.head_dim * cfg.num_heads * layers
    ends = 2 * s_tok * cfg.dim * (cfg.in_dim * 4 + cfg.out_dim * 4)  # patch embedding + head
    total = gemm + win + cross + ends
    stream = torch.cuda.current_stream(dev)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(replays)]
    with torch.no_grad():
        for _ in range(max(1, warmup)):
            want = fwd()
        torch.cuda.synchronize()
        ev[0][0].record(stream)
        fwd()
        ev[0][1].record(stream)
        torch.cuda.synchronize()
        eager_ms = ev[0][0].elapsed_time(ev[0][1])
        from sr_dit import _lib
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=_lib.capture_stream(dev)):
            y = fwd()
        graph.replay()
        torch.cuda.synchronize()
        same = bool(torch.equal(y, want))
        for a, b in ev:
            a.record(stream)
            graph.replay()
            b.record(stream)
        torch.cuda.synchronize()
        times = [a.elapsed_time(b) for a, b in ev]
        same_last = bool(torch.equal(y, want))  # the output of the last timed replay
    ms = statistics.median(times)
    return {"ms_per_step": round(ms, 3), "mean_ms": round(statistics.fmean(times), 3),
            "min_ms": round(min(times), 3), "max_ms": round(max(times), 3), "replays": replays,
            "eager_ms": round(eager_ms, 3), "graph_equals_eager": same and same_last,
            "graph_first_replay_equals_eager": same, "graph_last_replay_equals_eager": same_last,
            "hip_graph": True, "layers": layers, "tokens": s_tok, "context_tokens": cfg.text_len,
            "scope": "time + text embeddings, patch embedding, 30 blocks, head, unpatchify",
            "linears": "fp8 e4m3, " + ("per-tensor" if scaling_of(model) == "tensor"
                                       else "row-wise (per-token activation, per-channel weight)")
                       + " scales",
            "useful_tflop": round(total / 1e12, 2), "gemm_tflop": round(gemm / 1e12, 2),
            "tflops": round(total / (ms * 1e-3) / 1e12, 1), "build_s": round(build_s, 1),
            "data": "synthetic: N(0,0.02) weights, N(0,1) latent and text context"}


def scaling_of(model):
    from sr_dit.fp8_linear import Fp8Linear
    for m in model.modules():
        if isinstance(m, Fp8Linear):
            return m.scaling
    return "none"


def stream_chunks(model, chunks=8, timed=4, anchor=None, sigma_start=0.6251):
    """The streaming SR loop: 45x80-token frames (90x160 latent), 3-frame chunks, a
    9-frame KV cache per layer kept in place (ring), 4x4-block radius-3 windows,
    every forward a HIP graph replay.  ``sigma_start`` 0.6251 is the shipped
    schedule (sr_dit_5b.yaml:65): of the warped list 1000/937.5/833.3/625 only
    t=625 remains, so a chunk is one denoising forward plus the refresh pass;
    1.0 keeps all four steps.  ``anchor`` "frame": the LQ anchor
    (run_inference.sh:59-65), harvested per chunk by one more forward over the LQ
    frames.  The first chunks fill the cache (one graph per cache length); the
    last ``timed`` chunks run at the full 12-frame KV and are timed, and their
    median is reported (one slow chunk on a box does not move it)."""
    import torch
    from sr_dit.stream import StreamingRefiner

    dev = torch.device("cuda:0")
    cfg = model.cfg
    h, w, chunk = 45, 80, 3
    g = torch.Generator("cpu").manual_seed(0)
    noise = torch.randn(cfg.in_dim, chunk * chunks, 2 * h, 2 * w, generator=g).to(dev)
    ctx = torch.randn(cfg.text_len, cfg.text_dim, generator=g).to(torch.bfloat16).to(dev)
    lq = torch.randn(cfg.in_dim, chunk * chunks, 2 * h, 2 * w, generator=g).to(dev)
    t0 = time.perf_counter()
    r = StreamingRefiner(model, h, w, ctx, chunk=chunk, kv_len=9, device=dev, anchor=anchor,
                         sigma_start=sigma_start)
    per_chunk = []
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    for c in range(chunks):
        sl = slice(c * chunk, (c + 1) * chunk)
        e0.record(stream)
        r.refine_chunk(noise[:, sl], c * chunk, lq[:, sl] if anchor else None)
        e1.record(stream)
        torch.cuda.synchronize()
        per_chunk.append(e0.elapsed_time(e1))
    wall = time.perf_counter() - t0
    steady = sorted(per_chunk[-timed:])
    ms = (steady[(len(steady) - 1) // 2] + steady[len(steady) // 2]) / 2
    # one eager forward at the full cache for comparison
    r.use_graph = False
    e0.record(stream)
    r.forward(noise[:, :chunk], r.steps[0], chunks * chunk, anchored=anchor is not None)
    e1.record(stream)
    torch.cuda.synchronize()
    eager_fwd = e0.elapsed_time(e1)
    n_fwd = len(r.steps) + 1 + (1 if anchor else 0)
    sched = ("shipped one-step schedule (sigma_start 0.6251: t=625)" if len(r.steps) == 1
             else f"{len(r.steps)}-step schedule (sigma_start {sigma_start})")
    return {"workload": "streaming SR loop, 5B refiner (30 layers), 3 x 45x80-token chunk vs "
                        "9 cached frames (ring), 4x4 blocks radius 3, " + sched
                        + " + KV refresh per chunk, 512 context tokens"
                        + (f", LQ anchor ({anchor}-aligned, harvested per chunk)" if anchor
                           else ", no LQ anchor"),
            "ms_per_chunk": round(ms, 2), "ms_per_forward": round(ms / n_fwd, 2),
            "eager_ms_per_forward": round(eager_fwd, 2), "forwards_per_chunk": n_fwd,
            "sigma_start": sigma_start, "steps": [round(t, 2) for t in r.steps],
            "kv_frames": 9 + chunk,
            "chunk_ms_all": [round(x, 1) for x in per_chunk], "hip_graphs": len(r._graphs),
            "wall_s": round(wall, 1),
            "data": "synthetic: N(0,0.02) weights, N(0,1) noise latents and context"}


def production_window(steps, warmup=3):
    """The refiner's shipped window geometry: 4x4-token blocks, radius 3, one 3-frame
    query chunk of 45x80 against 12 KV frames (streaming rule), without an anchor and
    with the LQ anchor in its "frame" and "chunk" alignments (one 45x80 anchor frame per
    query frame).  Useful TFLOP/s per kernel launch.  Without an anchor the launcher
    packs two 48-query windows into one 64-row tile where neighbours allow; the
    anchored forms run one window per workgroup (48-query windows give the grouped
    kernel nothing to pair)."""
    import torch
    from sr_dit import attention as att
    from sr_dit import blockgrid_hip as bgh
    from sr_dit import workloads as wl

    dev = torch.device("cuda:0")
    f_cur, f_kv, h, w = 3, 12, 45, 80
    spec = att._BlockGridSpec(f_cur=f_cur, f_kv=f_kv, h=h, w=w, block_t=3, bh=4, bw=4, rh=3,
                              rw=3, rt=3, streaming=True)
    n, d = wl.N_HEADS, wl.HEAD_DIM
    L = h * w
    g = torch.Generator("cpu").manual_seed(0)
    sc = d ** -0.5
    # KV tensor = f_cur anchor frames, then the 12 HR frames (the kernel reads the
    # anchor prefix only in the anchor modes)
    q = (torch.randn(f_cur * L, n, d, generator=g) * sc).to(torch.bfloat16).to(dev)
    k = (torch.randn((f_cur + f_kv) * L, n, d, generator=g) * sc).to(torch.bfloat16).to(dev)
    v = (torch.randn((f_cur + f_kv) * L, n, d, generator=g) * sc).to(torch.bfloat16).to(dev)
    out = torch.empty_like(q)
    res = {"workload": "window attention 3x45x80 query chunk vs 12 KV frames, 24 heads x 128, "
                       "4x4 blocks, radius 3 (7x7 blocks), streaming rule; anchor: one 45x80 LQ "
                       "frame per query frame",
           "steps": steps}
    stream = torch.cuda.current_stream(dev)
    for mode in (None, "frame", "chunk"):
        plan = bgh.build_plan(spec, anchor_mode=mode)

        def run():
            bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=f_cur, h=h, w=w, n=n, d=d,
                                  anchor_mode=mode)

        for _ in range(warmup):
            run()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            run()
        e1.record(stream)
        torch.cuda.synchronize()
        ms = e0.elapsed_time(e1) / steps
        flops = wl.plan_useful_flops(plan)
        res[mode or "no_anchor"] = {"us": round(ms * 1e3, 1), "useful_gflop": round(flops / 1e9, 1),
                                    "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
    return res


def gemm_shapes(reps=20, settle_ms=60.0):
    """The fp8 e4m3 GEMM of the refiner's projections in isolation, per-tensor scales
    and a bf16 bias, bf16 output (srdit_fp8_gemm, the persistent MFMA kernel): the
    21,600-token q/k/v/o and cross-attention projections (N = K = 3072) and the two
    FFN Linears (3072 -> 14336 -> 3072).  Each shape runs untimed for settle_ms
    first, as the window step does, then reps timed launches."""
    import torch
    from sr_dit import _lib

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    f8 = torch.float8_e4m3fn
    g = torch.Generator(device=dev).manual_seed(0)
    res = {"kernel": "fp8_gemm_kernel (persistent 256x256 tiles, LDS DMA ring)",
           "scales": "per-tensor", "reps": reps, "peak_fp8_tflops": 5000.0}
    for name, (M, N, K) in (("qkvo_21600x3072x3072", (21600, 3072, 3072)),
                            ("ffn_up_21600x14336x3072", (21600, 14336, 3072)),
                            ("ffn_down_21600x3072x14336", (21600, 3072, 14336))):
        a = (torch.randn(M, K, generator=g, device=dev) * 2).to(f8)
        b = (torch.randn(N, K, generator=g, device=dev) * 2).to(f8)
        sa = torch.full((1,), 0.01, device=dev)
        sb = torch.full((1,), 0.02, device=dev)
        bias = torch.randn(N, generator=g, device=dev).to(torch.bfloat16)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < settle_ms:
            for _ in range(4):
                _lib.fp8_gemm(a, b, sa, sb, bias, out)
            torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(reps):
            _lib.fp8_gemm(a, b, sa, sb, bias, out)
        e1.record(stream)
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) / reps * 1e3
        pf = 2.0 * M * N * K / (us * 1e-6) / 1e15
        res[name] = {"us": round(us, 1), "pflops": round(pf, 3),
                     "frac_fp8_peak": round(pf * 1e3 / 5000.0, 4)}
        del a, b, out
    torch.cuda.empty_cache()
    return res


def gather_buckets(plan, H, W):
    """Token indices of every window of a plain plan without an anchor prefix,
    bucketed by shape: a list of ([Nw, Lq], [Nw, Lkv]) int64 CPU tensors.  Query
    tokens are the row's query cuboid (fields 0-5), keys its KV cuboid (fields
    6-11), t-major then row then column on an H x W grid."""
    import torch
    L = H * W

    def cuboid(t0, tl, h0, hl, w0, wl_):
        t = torch.arange(t0, t0 + tl).view(-1, 1, 1) * L
        r = torch.arange(h0, h0 + hl).view(1, -1, 1) * W
        cc = torch.arange(w0, w0 + wl_).view(1, 1, -1)
        return (t + r + cc).reshape(-1)

    buckets = {}
    for row in plan["params"].tolist():
        qi = cuboid(row[0], row[1], row[2], row[4], row[3], row[5])
        ki = cuboid(row[6], row[7], row[8], row[9], row[10], row[11])
        if qi.numel() == 0 or ki.numel() == 0:
            continue
        b = buckets.setdefault((qi.numel(), ki.numel()), ([], []))
        b[0].append(qi)
        b[1].append(ki)
    return [(torch.stack(a), torch.stack(b)) for a, b in buckets.values()]


def gpu_gather_comparator(config, steps, warmup=2):
    """The reference's gather path (attention.py:650-687: per-window token gather,
    then dense attention per window) restated in torch on the GPU, in bf16, as the
    on-box comparator for the fused kernel.  Windows are bucketed by (Lq, Lkv) and
    their token indices built once outside the timed region; each step gathers Q,
    K and V per bucket, runs torch's fused SDPA on it and scatters the outputs.
    Only the flash or memory-efficient SDPA backends are used (never the math
    path in bf16); with neither available the leg reports that instead of a time."""
    import torch
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    from sr_dit import blockgrid_hip as bgh
    from sr_dit import workloads as wl

    dev = torch.device("cuda:0")
    c = wl.WINDOW_CONFIGS[config]
    spec = wl.window_spec(config)
    plan = bgh.build_plan(spec)
    if plan["p_stride"] != bgh.P_PLAIN or plan.get("hr_base", 0):
        return {"skipped": "plain plans without an anchor only"}
    H, W = c["h"], c["w"]
    L = H * W
    q, k, v, kc, vc = wl.make_window_inputs(config, torch.bfloat16, dev, seed=0)
    q, k, v = q[0].contiguous(), k[0], v[0]
    if kc is not None:
        k, v = torch.cat([kc[0], k]), torch.cat([vc[0], v])
    k, v = k.contiguous(), v.contiguous()

    groups = [(a.to(dev), b.to(dev)) for a, b in gather_buckets(plan, H, W)]
    out = torch.empty_like(q)
    n, d = q.shape[1], q.shape[2]

    def step():
        for qi, ki in groups:
            nw, lq = qi.shape
            lkv = ki.shape[1]
            qg = q.index_select(0, qi.reshape(-1)).view(nw, lq, n, d).transpose(1, 2)
            kg = k.index_select(0, ki.reshape(-1)).view(nw, lkv, n, d).transpose(1, 2)
            vg = v.index_select(0, ki.reshape(-1)).view(nw, lkv, n, d).transpose(1, 2)
            og = F.scaled_dot_product_attention(qg.contiguous(), kg.contiguous(), vg.contiguous())
            out.index_copy_(0, qi.reshape(-1), og.transpose(1, 2).reshape(nw * lq, n, d))

    backend = None
    for name, bk in (("flash", SDPBackend.FLASH_ATTENTION),
                     ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([bk]):
                step()
            torch.cuda.synchronize()
            backend = (name, bk)
            break
        except RuntimeError:
            continue
    if backend is None:
        return {"skipped": "neither the flash nor the memory-efficient SDPA backend runs here"}
    stream = torch.cuda.current_stream(dev)
    with sdpa_kernel([backend[1]]):
        for _ in range(warmup):
            step()
        torch.cuda.synchronize()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
        torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    flops = wl.plan_useful_flops(plan)
    return {"workload": config, "sdpa_backend": backend[0], "buckets": len(groups),
            "ms_per_step": round(ms, 3), "tflops": round(flops / (ms * 1e-3) / 1e12, 1),
            "note": "torch gather + SDPA restatement of the reference's gather path, bf16, "
                    "index tables built outside the timed region"}


def leg(name, fn, *a, **kw):
    """Run one measurement leg inside a named range (a roctx range under rocprofv3
    --marker-trace), so kernel traces can be split by leg."""
    import torch
    torch.cuda.nvtx.range_push(name)
    try:
        return fn(*a, **kw)
    finally:
        torch.cuda.synchronize()
        torch.cuda.nvtx.range_pop()


def main():
    args = parse()
    if args.source_hash:
        print(traffic_source_hash(), flush=True)
        return
    if args.copy_calibration:
        copy_calibration(args.copy_calibration)
        return
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (got --gpus {args.gpus}); the window attention "
              "and fp8 paths have no multi-GPU implementation here.", file=sys.stderr)
        sys.exit(2)
    import torch
    from sr_dit import blockgrid_hip as bgh
    from sr_dit import workloads as wl

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    dev = torch.device("cuda:0")
    cfg = args.config
    spec = wl.window_spec(cfg)
    plan = bgh.build_plan(spec)
    q, k, v, kc, vc = wl.make_window_inputs(cfg, torch.bfloat16, dev, seed=0)
    q, k, v = q[0].contiguous(), k[0], v[0]
    if kc is not None:
        k, v = torch.cat([kc[0], k]), torch.cat([vc[0], v])
    k, v = k.contiguous(), v.contiguous()
    out = torch.empty_like(q)
    n, d = wl.N_HEADS, wl.HEAD_DIM

    def step():
        bgh.run_blockgrid_hip(q, k, v, out, plan=plan, f_cur=spec.f_cur, h=spec.h, w=spec.w,
                              n=n, d=d)

    torch.cuda.nvtx.range_push("window_" + cfg)
    # Settle: untimed launches of the same step for --settle-ms of wall time before
    # the warm-up.  The GPU raises its clock over the first few tens of
    # milliseconds of sustained load (c3 with 5 warm-up launches: 477 us per
    # timed launch; with 50: 400 us), so without it the timed steps would see a
    # clock the GPU does not hold under load.  Reported in the JSON line.
    step()
    torch.cuda.synchronize()  # first launch: module load and table uploads
    settle_n, t_settle = 1, time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < args.settle_ms and settle_n < 4096:
        for _ in range(16):
            step()
        settle_n += 16
        torch.cuda.synchronize()
    settle_s = time.perf_counter() - t_settle
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    torch.cuda.nvtx.range_pop()
    ms = e0.elapsed_time(e1) / args.steps

    flops = wl.plan_useful_flops(plan)
    tflops = flops / (ms * 1e-3) / 1e12
    s_q = q.shape[0]
    s_kv = k.shape[0]
    alg_bytes = (2 * s_q + 2 * s_kv) * n * d * 2      # Q + O + K + V once, bf16
    traffic, traffic_src = profile_traffic(cfg)
    result = {
        "metric": "window-attn TFLOP/s & % MFMA peak @2K (21.6k tok); ms per SR-DiT 5B step",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1)/sqrt(128) Q/K/V, generated on the CPU)",
        "config": {"workload": CONFIG_DESC[cfg], "tokens": s_q, "kv_tokens": s_kv,
                   "heads": n, "head_dim": d, "windows": plan["n_w"],
                   "useful_gflop": round(flops / 1e9, 2), "parallelism": "single GPU"},
        "pct_bf16_peak": round(100 * tflops / PEAK_BF16_TFLOPS, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic,
                     "traffic_source": traffic_src,
                     "algorithmic_bytes": alg_bytes,
                     "algorithmic_hbm_gbs": round(alg_bytes / (ms * 1e-3) / 1e9, 1)},
        "wall_s_timed_region": round(wall, 4),
        "settle": {"launches": settle_n, "wall_ms": round(settle_s * 1e3, 1),
                   "note": "untimed launches of the same step before the warm-up steps, so the "
                           "timed steps run at the clock the GPU holds under sustained load"},
    }
    if not args.no_comparator:
        try:  # a comparator that cannot run here must not cost the bench line
            result["gpu_comparator"] = leg("gpu_comparator", gpu_gather_comparator, cfg, 5)
        except Exception as e:  # noqa: BLE001
            torch.cuda.synchronize()
            result["gpu_comparator"] = {"skipped": f"{type(e).__name__}: {e}"[:300]}
        if result["gpu_comparator"].get("ms_per_step"):
            result["gpu_comparator"]["speedup_of_kernel"] = round(
                result["gpu_comparator"]["ms_per_step"] / ms, 2)
    if not args.no_prod:
        result["production_window"] = leg("production_window", production_window, 20)
    if not args.no_gemm:
        result["fp8_gemm"] = leg("fp8_gemm", gemm_shapes)
    if not (args.no_step and args.no_stream):
        model, build_s = build_model()
        if not args.no_step:
            result["refiner_step"] = leg("refiner_step", refiner_step, model, build_s,
                                        args.step_iters, 1)
        if not args.no_stream:
            result["stream"] = leg("stream", stream_chunks, model)
            result["stream_lq_anchor"] = leg("stream_lq_anchor", stream_chunks, model,
                                             anchor="frame")
            result["stream_4step"] = leg("stream_4step", stream_chunks, model, sigma_start=1.0)
        del model
        torch.cuda.empty_cache()
        if not (args.no_step or args.no_rowwise):
            model, build_s = build_model(scaling="rowwise")
            result["refiner_step_rowwise"] = leg("refiner_step_rowwise", refiner_step, model,
                                                 build_s, max(10, args.step_iters // 5), 1)
            del model
            torch.cuda.empty_cache()
    if not args.no_cpu_baseline:
        result["cpu_baseline"] = cpu_baseline(cfg, args.cpu_seconds)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
