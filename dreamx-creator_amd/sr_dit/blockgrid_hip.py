"""Block-grid window attention: params-row planner and the HIP launcher.

The planner turns one window geometry (a ``_BlockGridSpec``) into ONE int32
params table, one row per query window, plus the launch tiling. The table
layout, the row order and the ``block_m``/``m_tiles``/``hr_base``/``p_stride``
values are the reference's launch contract
(video_refiner/wan/modules/sr_dit/blockgrid_triton.py:68-150), kept bit-exact so
a plan built here and a plan built by the reference are interchangeable.

The launcher (:func:`run_blockgrid_hip`, the counterpart of
``run_blockgrid_triton``, blockgrid_triton.py:392-422) hands the table to the
HIP kernel through the C ABI in ``libsrdit_hip.so``.  There is no CPU path and
no fallback: a missing library raises.
"""
from __future__ import annotations

import torch

from . import _lib

# Params row layouts (int32, one row per window); the kernel reads them with
# raw pointer arithmetic.  All lengths are lengths, not end indices.
#   plain (19): q_t0 q_tL q_h0 q_w0 qhL qwL kv_t0 kv_tL kh0 khL kw0 kwL a_frames
#               kh0_a khL_a kw0_a kwL_a H_a W_a
#   frame (17): q_h0 q_w0 qhL qwL kv_t0 kv_tL kh0 khL kw0 kwL f_cur
#               kh0_a khL_a kw0_a kwL_a H_a W_a
# (field order: blockgrid_triton.py:77-80, rows: :127-141)
P_PLAIN = 19
P_FRAME = 17

#: Query rows per HIP workgroup: two wavefronts, one 32-row MFMA tile each.
HIP_BLOCK_M = 64


def _next_pow2(x: int) -> int:
    p = 1
    while p < x:
        p <<= 1
    return p


def build_plan(spec, *, anchor_mode=None, block_n=64):
    """One launch spec covering every window of ``spec``.

    Returns ``{"params": int32 [Nw, P] (CPU), "n_w", "block_m", "m_tiles",
    "block_n", "hr_base", "p_stride"}`` exactly as blockgrid_triton.py:83-150
    does.  ``spec`` is read only through ``temporal_runs()``, ``h_blocks()``,
    ``w_blocks()``, the optional ``anchor_h_blocks()``/``anchor_w_blocks()``/
    ``anchor_grid`` and ``f_cur``/``h``/``w``.

    ``anchor_mode``: ``"frame"`` (per-frame anchor, 17-field rows, the query
    time axis must be the single run ``[0, f_cur)``), ``"chunk"`` (whole anchor
    chunk visible, ``a_frames = f_cur``) or ``None`` (no anchor).
    """
    hb, wb = spec.h_blocks(), spec.w_blocks()
    hb_a = spec.anchor_h_blocks() if hasattr(spec, "anchor_h_blocks") else hb
    wb_a = spec.anchor_w_blocks() if hasattr(spec, "anchor_w_blocks") else wb
    a_h, a_w = getattr(spec, "anchor_grid", (int(spec.h), int(spec.w)))
    runs = spec.temporal_runs()
    f_cur = int(spec.f_cur)

    rows: list[list[int]] = []
    lqs: list[int] = []
    if anchor_mode == "frame":
        if len(runs) != 1 or runs[0][0] != 0 or runs[0][1] != f_cur:
            raise ValueError(
                f'anchor_mode="frame" needs the query time axis to be the single '
                f"run [0, {f_cur}); got {runs}.  Frame rows carry no q_t0, so a "
                f"partitioned query axis needs anchor_mode=None or 'chunk'.")
        kv0, kv1 = runs[0][2], runs[0][3]
        for (qh0, qhL, kh0, khL), (_, _, kh0a, khLa) in zip(hb, hb_a):
            for (qw0, qwL, kw0, kwL), (_, _, kw0a, kwLa) in zip(wb, wb_a):
                rows.append([qh0, qw0, qhL, qwL, kv0, kv1 - kv0,
                             kh0, khL, kw0, kwL, f_cur,
                             kh0a, khLa, kw0a, kwLa, a_h, a_w])
                lqs.append(f_cur * qhL * qwL)
    else:
        a_frames = f_cur if anchor_mode == "chunk" else 0
        for (q0, q1, kv0, kv1) in runs:
            for (qh0, qhL, kh0, khL), (_, _, kh0a, khLa) in zip(hb, hb_a):
                for (qw0, qwL, kw0, kwL), (_, _, kw0a, kwLa) in zip(wb, wb_a):
                    rows.append([q0, q1 - q0, qh0, qw0, qhL, qwL,
                                 kv0, kv1 - kv0, kh0, khL, kw0, kwL, a_frames,
                                 kh0a, khLa, kw0a, kwLa, a_h, a_w])
                    lqs.append((q1 - q0) * qhL * qwL)

    # Shared tile height: the largest window, at least 16 and at most 64 rows.
    block_m = max(16, min(_next_pow2(max(lqs)), 64))
    m_tiles = max(-(-x // block_m) for x in lqs)
    return {"params": torch.tensor(rows, dtype=torch.int32).contiguous(),
            "n_w": len(rows), "block_m": block_m, "m_tiles": m_tiles,
            "block_n": block_n,
            "hr_base": (f_cur * a_h * a_w) if anchor_mode is not None else 0,
            "p_stride": P_FRAME if anchor_mode == "frame" else P_PLAIN}


#: Plans memoised on the geometry (``tuple(spec)``), the anchor mode and
#: ``block_n``.  Keyed on the geometry, not on the temporal rule it implies: a
#: caller that swaps ``temporal_runs`` must clear it.
HIP_PLAN_CACHE: dict = {}


def cached_plan(spec, *, anchor_mode=None, block_n=64):
    """:func:`build_plan`, memoised (blockgrid_triton.py:158-167)."""
    key = (tuple(spec), anchor_mode, block_n)
    plan = HIP_PLAN_CACHE.get(key)
    if plan is None:
        plan = HIP_PLAN_CACHE[key] = build_plan(
            spec, anchor_mode=anchor_mode, block_n=block_n)
    return plan


def clear_plan_cache():
    HIP_PLAN_CACHE.clear()


def hip_kernel_keys(plan, *, anchor_mode=None, d=None):
    """The kernel variants a plan launches: one, by construction.

    The HIP kernels are compiled ahead of time, so this is the set of
    (mode, query tile, head dim) instantiations the launch selects
    (the counterpart of ``triton_compile_keys``, blockgrid_triton.py:170-181).
    """
    return {("frame" if anchor_mode == "frame" else "plain", HIP_BLOCK_M, d)}


def kernel_m_tiles(plan) -> int:
    """Query tiles of :data:`HIP_BLOCK_M` rows needed by the largest window.

    Every window has at most ``block_m * m_tiles`` query rows, so this many
    64-row tiles cover it.
    """
    return max(1, -(-(plan["block_m"] * plan["m_tiles"]) // HIP_BLOCK_M))


def _window_cost(plan) -> torch.Tensor:
    """Useful MACs per window (Lq * Lkv), the launch-order key."""
    p = plan["params"].to(torch.int64)
    if plan["p_stride"] == P_FRAME:
        qsp = p[:, 2] * p[:, 3]
        lq = p[:, 10] * qsp
        lkv = p[:, 5] * p[:, 7] * p[:, 9] + p[:, 12] * p[:, 14]
    else:
        qsp = p[:, 4] * p[:, 5]
        lq = p[:, 1] * qsp
        lkv = p[:, 7] * p[:, 9] * p[:, 11] + p[:, 12] * p[:, 14] * p[:, 16]
    return lq * lkv


def mean_kv_tokens(plan) -> float:
    """Mean KV tokens per window (HR cuboid plus anchor prefix)."""
    p = plan["params"].to(torch.int64)
    if p.shape[0] == 0:
        return 0.0
    if plan["p_stride"] == P_FRAME:
        lkv = p[:, 5] * p[:, 7] * p[:, 9] + p[:, 12] * p[:, 14]
    else:
        lkv = p[:, 7] * p[:, 9] * p[:, 11] + p[:, 12] * p[:, 14] * p[:, 16]
    return float(lkv.double().mean())


#: Smallest mean KV length per window for which ``auto`` pairs members.  Since
#: the plain kernel stages Q and O through LDS, pairs of identical-KV members
#: win at every length measured: dense attention of 21,600 queries over 64 to
#: 1024 context tokens, 78 vs 82 us up to 280 vs 315 us (one process, identical
#: outputs), so no minimum applies.
GROUPED_MIN_KV = 0


def launch_order(plan) -> torch.Tensor:
    """Window launch order: the planner's own row order (run -> h-block -> w-block).

    The kernel hands each XCD a contiguous range of tasks, head-major, so in
    row order the workgroups sharing an L2 work on neighbouring windows of one
    head, whose KV cuboids overlap.  Measured on the 2K and 1080p grids this
    beats a longest-first order, whose locality loss outweighs its shorter tail.
    """
    return torch.arange(plan["n_w"], dtype=torch.int32)


def longest_first_order(plan) -> torch.Tensor:
    """Most expensive window first (longest-processing-time order), ties in row order."""
    cost = _window_cost(plan)
    order = sorted(range(cost.numel()), key=lambda i: (-int(cost[i]), i))
    return torch.tensor(order, dtype=torch.int32)


def groups_supported(plan) -> bool:
    """True when the grouped kernel can run the plan: plain rows, no anchor
    prefix, at most 16 KV frames per window (a pair walks at most 32 frame
    slots)."""
    if plan["p_stride"] != P_PLAIN:
        return False
    params = plan["params"]
    return bool((params[:, 12] == 0).all()) and bool((params[:, 7] <= 16).all())


def build_groups(plan) -> torch.Tensor:
    """Pair the plan's 64-query members for the grouped kernel; int32 [G, 4].

    A member is (row, m-tile) for every 64-row tile of a window's queries.  The
    m-tiles of one window pair with each other (identical KV).  Remaining
    members pair with the next member, in frame order, whose window has the
    same spatial KV extent (kh0, khL, kw0, kwL) and an overlapping frame range
    (the neighbouring query frames of the +-1-frame and streaming rules); those
    pairs share the K/V fetches of their common frames.  Unpaired members run
    alone (row1 = -1).  Groups are ordered by the query run of their first
    member, then heaviest first (both members' Lq * Lkv; stable, so equal
    groups keep the planner's raster order), as ``build_singles`` orders its
    members: c4's m-tile pairs 280.5 -> 272.7 us.
    """
    p = plan["params"].tolist()
    singles = []
    groups = []
    for r, row in enumerate(p):
        lq = row[1] * row[4] * row[5]
        tiles = list(range(-(-lq // HIP_BLOCK_M))) if lq > 0 else []
        while len(tiles) >= 2:
            groups.append((r, tiles[0], r, tiles[1]))
            tiles = tiles[2:]
        if tiles:
            singles.append((r, tiles[0]))
    buckets: dict = {}
    for r, mt in singles:
        row = p[r]
        buckets.setdefault((row[8], row[9], row[10], row[11]), []).append((row[6], r, mt))
    for lst in buckets.values():
        lst.sort()
        i = 0
        while i < len(lst):
            a0, r0, m0 = lst[i]
            if i + 1 < len(lst):
                a1, r1, m1 = lst[i + 1]
                if min(a0 + p[r0][7], a1 + p[r1][7]) > max(a0, a1):
                    groups.append((r0, m0, r1, m1))
                    i += 2
                    continue
            groups.append((r0, m0, -1, 0))
            i += 1
    groups.sort(key=lambda g: (g[0], g[1]))
    cost = _window_cost(plan).tolist()
    weight = [cost[g[0]] + (cost[g[2]] if g[2] >= 0 else 0) for g in groups]
    order = sorted(range(len(groups)), key=lambda i: (p[groups[i][0]][0], -weight[i]))
    return torch.tensor([groups[i] for i in order], dtype=torch.int32).reshape(-1, 4).contiguous()


def _row_lq(plan, row) -> int:
    """Queries of a params row (plain: q_tl * qh_l * qw_l at fields 1, 4, 5; per-frame
    anchor rows: fields 10, 2, 3)."""
    if plan["p_stride"] == P_FRAME:
        return row[10] * row[2] * row[3]
    return row[1] * row[4] * row[5]


def solo_supported(plan) -> bool:
    """True when the one-member form of the grouped kernel can run the plan: at
    most 16 HR KV frames per window and at most 32 frame slots (HR frames plus
    the anchor frames a 64-query tile walks)."""
    p = plan["params"]
    if plan["p_stride"] == P_FRAME:
        hr = p[:, 5]
        q_sp = (p[:, 2] * p[:, 3]).clamp(min=1)
        anc = torch.minimum(p[:, 10], 64 // q_sp + 2)
    else:
        hr = p[:, 7]
        anc = p[:, 12]
    return bool((hr <= 16).all()) and bool((hr + anc <= 32).all())


def plan_anchor_mode(plan) -> int:
    """Anchor mode code of the grouped kernel: 0 none, 1 per frame, 2 whole chunk."""
    if plan["p_stride"] == P_FRAME:
        return 1
    return 2 if bool((plan["params"][:, 12] > 0).any()) else 0


def build_singles(plan) -> torch.Tensor:
    """Every 64-query member alone: int32 [G, 4] rows (row, m-tile, -1, 0) for the
    one-member-per-workgroup form of the grouped kernel.

    Launch order: query run by query run (the plan's row order, so workgroups
    running together on an XCD share KV through its L2), the heaviest windows
    of a run first (stable, so equal windows keep raster order): the light
    edge windows then fill the last, partial round of workgroups.  Measured on
    the shipped 4x4/r3 geometry (one run of 240 windows): 1409 -> 1324 us,
    with the per-frame anchor 1830 -> 1646 us; c2 228 -> 224 us; c3 unchanged.
    Ordering across runs instead (heaviest first overall) costs c3 3%."""
    p = plan["params"].tolist()
    rows, keys = [], []
    cost = _window_cost(plan).tolist()
    for r, row in enumerate(p):
        lq = _row_lq(plan, row)
        run = row[0] if plan["p_stride"] == P_PLAIN else 0  # q_t0; frame rows hold one run
        for mt in range(-(-lq // HIP_BLOCK_M) if lq > 0 else 0):
            rows.append((r, mt, -1, 0))
            keys.append((run, -cost[r]))
    order = sorted(range(len(rows)), key=lambda i: keys[i])  # stable
    return torch.tensor([rows[i] for i in order], dtype=torch.int32).reshape(-1, 4).contiguous()


#: Width in tokens of the KV column union a two-window packed tile walks: one
#: 32-key step is then one token row of the union, so a key's column is its
#: index in the step and each lane's window mask is the same every step.
PACK_WIDTH = 32


def _packs(a, b) -> bool:
    """Plain rows ``a`` then ``b`` (b to the right of a) can share packed tiles:
    the same query frames and KV frames and rows, at most one 64-row tile of
    queries each, and KV columns whose union is exactly PACK_WIDTH wide."""
    if a[0:2] != b[0:2] or a[6:10] != b[6:10] or a[12] or b[12]:
        return False
    if not (0 < a[1] * a[4] * a[5] <= HIP_BLOCK_M and 0 < b[1] * b[4] * b[5] <= HIP_BLOCK_M):
        return False
    lo, hi = min(a[10], b[10]), max(a[10] + a[11], b[10] + b[11])
    overlap = min(a[10] + a[11], b[10] + b[11]) - max(a[10], b[10])
    return hi - lo == PACK_WIDTH and overlap >= 0 and b[10] > a[10]


def build_packed(plan):
    """Packed one-member tiles for a plain plan without an anchor prefix, or
    None when no tile would hold two windows.

    Windows whose KV cuboids differ only in their columns and whose column
    union is PACK_WIDTH wide (horizontal neighbours of the shipped 4x4/r3
    geometry: 28-column windows four columns apart) form runs.  A run's
    queries, window after window, are cut into tiles of at most 64 rows, so a
    48-query window no longer pads a tile by 16 rows: a tile holds the end of
    one window and the start of the next and walks the union of their columns,
    each lane masking the columns outside its own window.  The cut is greedy
    and never puts a third window in a tile (40-query windows: three windows in
    two tiles).  Other windows get one tile per 64 queries, as in
    ``build_singles``.

    Returns int32 [T, 5]: (row A, first query of A, A's rows in the tile,
    row B or -1, first query of B).  Launch order: query run by query run,
    the heaviest tiles first within one (cost = tile rows' KV cuboid)."""
    if not groups_supported(plan):
        return None
    p = plan["params"].tolist()
    by_cuboid: dict = {}
    for r, row in enumerate(p):
        by_cuboid.setdefault((row[0], row[1], row[6], row[7], row[8], row[9]), []).append(r)
    tiles, keys = [], []
    packed_any = False

    def add(tile, run_key, cost):
        tiles.append(tile)
        keys.append((run_key, -cost))

    def singles(r):
        row = p[r]
        lq = _row_lq(plan, row)
        cost = row[7] * row[9] * row[11]
        for mt in range(-(-lq // HIP_BLOCK_M) if lq > 0 else 0):
            add([r, HIP_BLOCK_M * mt, min(HIP_BLOCK_M, lq - HIP_BLOCK_M * mt), -1, 0], row[0], cost)

    for rows in by_cuboid.values():
        rows.sort(key=lambda r: (p[r][10], p[r][3]))
        i = 0
        while i < len(rows):
            j = i
            while j + 1 < len(rows) and _packs(p[rows[j]], p[rows[j + 1]]):
                j += 1
            run = rows[i:j + 1]
            i = j + 1
            if len(run) < 2:
                singles(run[0])
                continue
            # Greedy cut: a tile takes what is left of window A and, when that is
            # under 64 rows, the head of the next window B; never a third one.
            lqs = [_row_lq(plan, p[r]) for r in run]
            wi, pos = 0, 0
            while wi < len(run):
                ra = run[wi]
                row = p[ra]
                na = min(HIP_BLOCK_M, lqs[wi] - pos)
                if na == HIP_BLOCK_M or wi + 1 == len(run):
                    add([ra, pos, na, -1, 0], row[0], row[7] * row[9] * row[11])
                    pos += na
                    if pos >= lqs[wi]:
                        wi, pos = wi + 1, 0
                    continue
                nb = min(HIP_BLOCK_M - na, lqs[wi + 1])
                packed_any = True
                add([ra, pos, na, run[wi + 1], 0], row[0], row[7] * row[9] * PACK_WIDTH)
                wi, pos = (wi + 2, 0) if nb == lqs[wi + 1] else (wi + 1, nb)
    if not packed_any:
        return None
    order = sorted(range(len(tiles)), key=lambda i: keys[i])  # stable
    return torch.tensor([tiles[i] for i in order], dtype=torch.int32).reshape(-1, 5).contiguous()


#: ``kernel="auto"`` runs packed tiles when they remove at least this fraction
#: of the one-window tiles.  The packed form costs more per tile than the
#: one-window form (A/B, one process: c3, 3% fewer tiles, 423 against 391 us;
#: c2, 5% fewer, 238 against 225 us), and wins where the tiles drop by a sixth
#: (the shipped 4x4/r3 geometry: 200 against 240 tiles, 1260 against 1367 us).
PACKED_MIN_SAVING = 0.10


def packed_saving(plan) -> float:
    """Fraction of build_singles' tiles that build_packed removes (0 when the plan
    does not pack); cached in the plan."""
    if "packed_saving" not in plan:
        if "packed_host" not in plan:
            plan["packed_host"] = build_packed(plan)
        host = plan["packed_host"]
        plan["packed_saving"] = 0.0 if host is None else \
            1.0 - host.shape[0] / max(1, build_singles(plan).shape[0])
    return plan["packed_saving"]


def _packed_table(plan, device):
    """build_packed's table on ``device`` (both cached in the plan), or None."""
    if "packed_host" not in plan:
        plan["packed_host"] = build_packed(plan)
    if plan["packed_host"] is None:
        return None
    key = ("packed", device)
    if key not in plan:
        plan[key] = plan["packed_host"].to(device)
    return plan[key]


def shared_fraction(plan, groups: torch.Tensor) -> float:
    """Fraction of the members' KV frames that a pair fetches once for both
    (2 * shared frames / frames of both members, summed over the table): 1.0
    when every pair is the two m-tiles of one window, ~2/3 for pairs of
    neighbouring query frames under a +-1-frame rule, 0 without pairs."""
    p = plan["params"].tolist()
    shared = total = 0
    for r0, _, r1, _ in groups.tolist():
        a0, la = p[r0][6], p[r0][7]
        total += la
        if r1 >= 0:
            a1, lb = p[r1][6], p[r1][7]
            total += lb
            shared += 2 * max(0, min(a0 + la, a1 + lb) - max(a0, a1))
    return shared / total if total else 0.0


def paired_fraction(groups: torch.Tensor) -> float:
    """Fraction of members that share a workgroup with a partner."""
    n = groups.shape[0]
    if n == 0:
        return 0.0
    paired = int((groups[:, 2] >= 0).sum())
    return 2 * paired / (2 * paired + (n - paired))


def _device_tables(plan, device):
    """(params, order) on ``device``, copied once per plan and device."""
    key = ("dev", device)
    tabs = plan.get(key)
    if tabs is None:
        params = plan["params"].to(device)
        order = launch_order(plan).to(device)
        tabs = plan[key] = (params, order)
    return tabs


def run_blockgrid_hip(q, k_ext, v_ext, out, *, plan, f_cur, h, w, n, d,
                      anchor_mode=None, kernel="auto", ring=None, hr_base=None,
                      amax_out=None):
    """Launch the fused window kernel for one sample; writes ``out`` and returns it.

    ``q``/``out``: ``[f_cur*h*w, n, d]``.  ``k_ext``/``v_ext``: the extended KV,
    ``cat([anchor, HR])`` when an anchor is present (``hr_base`` tokens of
    anchor first), else the HR KV alone.  All four must be contiguous with a
    stride-1 head dim, on one device, bf16 or fp16.  The launch is
    asynchronous on the current stream.

    ``kernel``: one of ``"auto"``, ``"grouped"``, ``"solo"``, ``"packed"`` and
    ``"single"``.  ``"auto"`` chooses as follows:
    - plain plans (no anchor prefix, at most 16 KV frames per window) whose
      64-query members pair up sharing at least 90% of their KV frames (the two
      m-tiles of one window, the query tiles of dense attention over the text
      context) run two members per workgroup (``"grouped"``);
    - other plain plans run one member per workgroup: on packed tiles, two
      neighbouring windows to a 64-row tile (``"packed"``), when that removes
      at least ``PACKED_MIN_SAVING`` of the one-window tiles (the 48-query
      windows of the shipped 4x4-block geometry), else one window per tile
      (``"solo"``: c2 and c3);
    - anchored plans run solo (the anchor frames walked after the HR frames)
      when they have at most 16 HR frames and 32 frame slots per window;
    - anything else runs on the single-window kernel (``"single"``).
    Forcing ``"grouped"`` for an anchored plan, ``"solo"`` beyond its limits or
    ``"packed"`` for a plan with nothing to pack raises ``ValueError``.

    ``ring`` = ``(ring_frames, ring_cached, head)``: the HR KV after the anchor
    prefix is an in-place cache (``sr_dit.kv_ring.KVRing``): ``ring_frames``
    slots of ``h*w`` tokens, cached logical frame ``f`` in slot
    ``(head[0] + f) % ring_frames``, then the current chunk's frames.  ``head``
    is a device int32 tensor read by the kernel at launch.  ``hr_base``
    overrides the plan's first HR token (a ring keeps its anchor prefix at a
    fixed size whether or not a call uses it).  ``amax_out`` (device int32
    [1]): receives the bits of max |out| for a per-tensor quantiser of it.
    """
    for name, t in (("q", q), ("k_ext", k_ext), ("v_ext", v_ext), ("out", out)):
        if not t.is_cuda:
            raise RuntimeError(f"run_blockgrid_hip: {name} is not a GPU tensor.")
        if not t.is_contiguous():
            raise ValueError(f"run_blockgrid_hip: {name} must be contiguous.")
        if t.dtype != q.dtype:
            raise ValueError(f"run_blockgrid_hip: {name} dtype {t.dtype} != q dtype {q.dtype}.")
        if t.dim() != 3 or t.shape[1] != n or t.shape[2] != d:
            raise ValueError(f"run_blockgrid_hip: {name} must be [tokens, {n}, {d}], got {tuple(t.shape)}.")
    if q.shape != out.shape or q.shape[0] != f_cur * h * w:
        raise ValueError(f"run_blockgrid_hip: q/out must be [{f_cur * h * w}, {n}, {d}].")
    if k_ext.shape != v_ext.shape:
        raise ValueError("run_blockgrid_hip: k_ext and v_ext shapes differ.")
    params, order = _device_tables(plan, q.device)
    if hr_base is None:
        hr_base = plan.get("hr_base", f_cur * h * w if anchor_mode is not None else 0)
    elif anchor_mode is not None and hr_base < plan.get("hr_base", 0):
        raise ValueError("run_blockgrid_hip: hr_base leaves no room for the anchor prefix.")
    mode = 1 if anchor_mode == "frame" else 0
    if (plan["p_stride"] == P_FRAME) != (mode == 1):
        raise ValueError("run_blockgrid_hip: plan layout does not match anchor_mode.")
    if kernel not in ("auto", "grouped", "solo", "single", "packed"):
        raise ValueError("run_blockgrid_hip: kernel must be auto, grouped, solo, single or packed, "
                         f"got {kernel!r}")
    if kernel == "packed":
        tiles = _packed_table(plan, q.device) if anchor_mode is None else None
        if tiles is None:
            raise ValueError("run_blockgrid_hip: the plan has no windows to pack (plain rows "
                             "without an anchor, at most 16 KV frames, neighbours whose KV "
                             "column union is 32 tokens wide).")
        _lib.window_attn_packed_fwd(
            q, k_ext, v_ext, out, params, tiles, n_w=plan["n_w"], hr_base=hr_base, H=h, W=w,
            n_heads=n, head_dim=d, kv_tokens=k_ext.shape[0], scale=d ** -0.5, ring=ring,
            amax_out=amax_out)
        return out
    if kernel == "grouped" and not groups_supported(plan):
        raise ValueError("run_blockgrid_hip: the grouped kernel needs plain rows without an anchor.")
    if kernel == "solo" and not solo_supported(plan):
        raise ValueError("run_blockgrid_hip: the grouped kernel takes at most 16 HR frames and 32 "
                         "frame slots per window.")
    if kernel == "auto" and not groups_supported(plan) and solo_supported(plan):
        kernel = "solo"
    if kernel == "solo":
        key = ("singles", q.device)
        singles = plan.get(key)
        if singles is None:
            singles = plan[key] = build_singles(plan).to(q.device)
        _lib.window_attn_grouped_fwd(
            q, k_ext, v_ext, out, params, singles, n_w=plan["n_w"], n_groups=singles.shape[0],
            hr_base=hr_base, H=h, W=w, n_heads=n, head_dim=d, kv_tokens=k_ext.shape[0],
            scale=d ** -0.5, ring=ring, amax_out=amax_out, members=1,
            anchor_mode=plan_anchor_mode(plan))
        return out
    use_grouped = False
    if kernel != "single" and groups_supported(plan):
        key = ("groups", q.device)
        groups = plan.get(key)
        if groups is None:
            host = build_groups(plan)
            plan["groups_paired_fraction"] = paired_fraction(host)
            plan["groups_shared_fraction"] = shared_fraction(plan, host)
            plan["mean_kv_tokens"] = mean_kv_tokens(plan)
            groups = plan[key] = host.to(q.device)
        # Pairs that share only part of their KV frames, and unpaired members,
        # run faster one member per workgroup.
        use_grouped = kernel == "grouped" or (plan["groups_paired_fraction"] >= 0.75 and
                                              plan["groups_shared_fraction"] >= 0.9 and
                                              plan["mean_kv_tokens"] >= GROUPED_MIN_KV)
        # Otherwise one member per workgroup: packed tiles where two windows
        # share one (48-query windows of 4x4 blocks), else one window per tile.
        if not use_grouped:
            packs = kernel == "auto" and anchor_mode is None and \
                packed_saving(plan) >= PACKED_MIN_SAVING
            return run_blockgrid_hip(q, k_ext, v_ext, out, plan=plan, f_cur=f_cur, h=h, w=w, n=n,
                                     d=d, anchor_mode=anchor_mode,
                                     kernel="packed" if packs else "solo", ring=ring,
                                     hr_base=hr_base, amax_out=amax_out)
    if use_grouped:
        _lib.window_attn_grouped_fwd(
            q, k_ext, v_ext, out, params, groups, n_w=plan["n_w"], n_groups=groups.shape[0],
            hr_base=hr_base, H=h, W=w, n_heads=n, head_dim=d, kv_tokens=k_ext.shape[0],
            scale=d ** -0.5, ring=ring, amax_out=amax_out)
        return out
    _lib.window_attn_fwd(
        q, k_ext, v_ext, out, params, order,
        n_w=plan["n_w"], m_tiles=kernel_m_tiles(plan), p_stride=plan["p_stride"],
        hr_base=hr_base, H=h, W=w, n_heads=n, head_dim=d,
        kv_tokens=k_ext.shape[0], scale=d ** -0.5, mode=mode, ring=ring, amax_out=amax_out)
    return out
