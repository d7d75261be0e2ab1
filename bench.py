#!/usr/bin/env python
"""TaoMemory operator benchmark on one MI355X.

Headline (``value``): advancing decode tok/s of one request x layer from a
131072-token state, 32 heads x 128, bf16, page memo (BASELINE.json
configs[3]): --warmup untimed single-token steps, then --steps timed ones
(default 16 + 256: the timed steps hold 11 route refreshes and the seal at
position 131327; config.workload states the counts of the run). Each step
is issued by the native C++ driver as direct kernel launches; the graph
preset (both replay mechanisms) is timed on the same steps and reported as
decode_graph. Also
reported: prefill tokens/s of a 16384-token prompt through
tao_attention_prefill, batched streaming decode of 32 ragged
requests (configs[4], decode_batch), a cold-cache decode variant that
cycles 32 independent 128K states (their touched bytes per cycle exceed the
256 MB Infinity Cache), the roofline of the dominant kernels measured live
with HIP events on the launch stream, and the CPU oracle (reference
arithmetic in torch eager) on bounded samples of decode and prefill.

Usage: python bench.py [--gpus 1] [--steps 256] [--warmup 16]
"""
import argparse
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "tao-memory_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "decode tok/s @128K ctx + prefill tokens/s @16K, 1 MI355X; % HBM/MFMA roofline"
HBM_PEAK_GBS = 8000.0
SPIN_CYCLES = 4_000_000        # bounded spin that keeps the queue ahead of the host
STEPS_PER_SPIN = 16
MFMA_BF16_PEAK_TFLOPS = 2500.0
# HBM-side bytes per decode token (decode_units_kernel<128> +
# decode_combine_kernel<128> every token, plus route + fold per refresh and
# fold + epilogue per seal, averaged over the 256-step run; 128K state, H32
# D128, M=34), from two rocprofv3 passes (FETCH_SIZE, then WRITE_SIZE, KiB
# per dispatch) scaled by the same counters over a 256 MiB plain copy
# (FETCH_SIZE reads 0.5000x the copied bytes, WRITE_SIZE 1.0000x); the
# summary and commands are under profiles/.
DECODE_STEP_TRAFFIC_BYTES = 13_570_800


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


class Probe:
    """Records HIP events around every launch a StreamCache makes."""

    def __init__(self, torch):
        self.torch = torch
        self.events = {}
        self.enabled = True

    def __call__(self, name):
        probe = self

        class _Ctx:
            def __enter__(self_inner):
                if probe.enabled:
                    self_inner.start = probe.torch.cuda.Event(enable_timing=True)
                    self_inner.start.record()

            def __exit__(self_inner, *exc):
                if probe.enabled:
                    end = probe.torch.cuda.Event(enable_timing=True)
                    end.record()
                    probe.events.setdefault(name, []).append((self_inner.start, end))
                return False
        return _Ctx()

    def total_ms(self, name):
        return sum(ev[0].elapsed_time(ev[1]) for ev in self.events.get(name, []))

    def count(self, name):
        """Launches (or steps, for grouped entries (start, end, count)) recorded."""
        return sum(ev[2] if len(ev) > 2 else 1 for ev in self.events.get(name, []))

    def reset(self):
        self.events = {}


def make_tokens(torch, tokens, heads, width, seed, device, unit_raw_k=False):
    g = torch.Generator(device=device).manual_seed(seed)
    xs = []
    for i in range(5):
        x = torch.randn((1, tokens, heads, width), generator=g, device=device,
                        dtype=torch.float32)
        if unit_raw_k and i == 4:
            x = x / x.norm(dim=-1, keepdim=True)
        xs.append(x.to(torch.bfloat16))
    fa = torch.randn((heads, width, 3), generator=g, device=device) * 0.02
    fb = torch.randn((heads, width, 3), generator=g, device=device) * 0.02
    return xs, fa, fb


def decode_bytes(cfg, heads, width, selected, position, layer=0):
    """Bytes of the decode step at `position` (selected = route size).

    Returns (reference_basis, own):
    * reference_basis: the per-step algorithmic bytes of the route + selected
      read as the reference defines the step (every selected C matrix and
      its side rows read per token): H*M*(D^2 + 3D)*2 + 2*H*D*2, plus
      H*(P + E)*D*2 on route-refresh steps (P pages, E eligible fines);
    * own: the bytes this build's step moves: the local K/V window, the
      folded route (G^T fp32 + den weights), the local-attention records,
      the token rows and, on refresh steps, the route plus the fold that
      re-reads the selected matrices.
    """
    from tao_attention import schedule
    fines = schedule.fines_at(position, cfg)
    refresh = fines > 0 and schedule.is_turn(position, layer, cfg)
    ref = heads * selected * (width * width + 3 * width) * 2 + 2 * heads * width * 2
    fold = 0
    if refresh:
        completed, pending = divmod(fines, cfg.coarse_group)
        coarse, eligible, _ = schedule.routed_counts(completed, pending, cfg)
        pages = completed + (pending > 0)
        ref += heads * (pages + eligible) * width * 2
        fold = heads * selected * (width * width + 2 * width) * 2 + heads * width * (width + 1) * 4
    keys = schedule.local_len_at(position, cfg) + 1
    local = keys * heads * width * 2 * 2                  # ring K and V
    folded = heads * width * (width + 1) * 4 if fines > 0 else 0
    records = 2 * 16 * heads * (width + 4) * 4            # written, then merged
    tokens = 5 * heads * width * 2 + 3 * heads * width * 2 + heads * width * 2
    own = local + folded + records + tokens + fold
    return ref, own


def decode_loop(torch, state, xs, fa, fb, start, steps):
    """`steps` single-token tao_attention_decode calls; returns (state, seconds).

    Each step's operands are [1, 1, H, D] views taken before the timed
    region: a model hands the layer freshly projected tensors, so the
    caller's own slicing (about 1 us per view) is not part of the step."""
    from tao_attention import tao_attention_decode
    rows = [tuple(x[:, i:i + 1] for x in xs) for i in range(start, start + steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for q, k, v, rq, rk in rows:
        _, state = tao_attention_decode(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb,
                                        alpha=0.5, state=state, position=state.get_pos())
    torch.cuda.synchronize()
    return state, time.perf_counter() - t0


def run_decode(torch, args, device, cfg, heads, width, context, seed, probe):
    """Headline decode: direct launches by the native driver (graph=False).

    The state takes `warmup` untimed decode steps (the first call's one-time
    setup falls there), then `steps` timed ones. The graph preset runs the
    same steps from the same snapshot on its own state, once per replay
    mechanism (reported as decode_graph), and the eager steps are replayed
    once more with the GPU pre-loaded for kernel timing.
    """
    from tao_attention import StreamCache, new_state, tao_attention_decode
    from tao_attention.presets import index_only_page_memo
    total = context + args.steps + args.warmup
    xs, fa, fb = make_tokens(torch, total, heads, width, seed, device)
    state = new_state(0, index_only_page_memo(graph=False))
    state._ingest(*(x[:, :context] for x in xs))
    torch.cuda.synchronize()
    log(f"decode state built: position {state.get_pos()}, route size {state.route_size}")
    snap = state.export()
    graph_snap = dict(snap, config=dict(snap["config"], q1_history_region_graph=True))
    first = context + args.warmup
    state, _ = decode_loop(torch, state, xs, fa, fb, context, args.warmup)
    state, seconds = decode_loop(torch, state, xs, fa, fb, first, args.steps)
    graph = {}
    for replay in ("dispatch", "hipgraph"):
        saved = os.environ.get("TAO_GRAPH_REPLAY")
        os.environ["TAO_GRAPH_REPLAY"] = replay
        try:
            graph_state = StreamCache.from_export(graph_snap)
        finally:
            if saved is None:
                del os.environ["TAO_GRAPH_REPLAY"]
            else:
                os.environ["TAO_GRAPH_REPLAY"] = saved
        graph_state, _ = decode_loop(torch, graph_state, xs, fa, fb, context, args.warmup)
        region = graph_state.history_region
        before = dict(region.counts) if region is not None else {}
        graph_state, graph_seconds = decode_loop(torch, graph_state, xs, fa, fb, first,
                                                 args.steps)
        after = graph_state.history_region.observation()
        timed_counts = {key: after[key] - before.get(key, 0)
                        for key in ("epochs", "eager_warm", "captures", "replays", "id_copies",
                                    "invalidations")}
        graph[replay] = (graph_seconds, timed_counts)
        graph_state.release_execution()
        del graph_state
    del graph_snap
    graph["launch_floor_us"] = graph_launch_floor(torch, device)
    # Device time per step: replay the same steps eagerly on an imported copy
    # with the GPU pre-loaded by a bounded spin kernel, and bracket each group
    # of STEPS_PER_SPIN back-to-back steps with HIP events on the launch
    # stream (no host gaps, no per-step event overhead).
    q, k, v, rq, rk = xs
    timed = StreamCache.from_export(snap)
    del snap
    timed, _ = decode_loop(torch, timed, xs, fa, fb, context, args.warmup)
    steps_bytes = []
    groups = []
    i = first
    while i < first + args.steps:
        torch.cuda._sleep(SPIN_CYCLES)
        start = torch.cuda.Event(enable_timing=True)
        start.record()
        count = min(STEPS_PER_SPIN, first + args.steps - i)
        for _ in range(count):
            sl = slice(i, i + 1)
            _, timed = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                            raw_k=rk[:, sl], fusion_a=fa, fusion_b=fb,
                                            alpha=0.5, state=timed, position=timed.get_pos())
            steps_bytes.append(decode_bytes(cfg, heads, width, timed.route_size, i))
            i += 1
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        groups.append((start, end, count))
    torch.cuda.synchronize()
    probe.events["decode_step"] = groups
    timed.release_execution()
    return state, xs, fa, fb, seconds, graph, steps_bytes


def run_timeline(torch, args, device, cfg, heads, width):
    """Per-phase timeline of the decode step from the kernel's clock stamps.

    The library's diagnostic recorder (tao_step_stamps) has every workgroup
    of an eager decode step write the device's 100 MHz clock at entry, after
    a local unit's scores (its window loads landed), after its record stores
    issued, after their acknowledgement barrier, after its arrival count and,
    for each head's last arrival, after the merge. The steps are the bench's
    timed decode steps, launched back to back behind a bounded spin (as for
    the step kernel's timing), from the same 128K state. Returns the summary
    (medians over the steps of per-launch means, in microseconds)."""
    import numpy as np
    from tao_attention import _hip, new_state, tao_attention_decode
    lib = _hip.lib()
    context = args.context
    total = context + args.warmup + args.steps
    xs, fa, fb = make_tokens(torch, total, heads, width, 4, device)
    state = new_state(0, cfg)
    state._ingest(*(x[:, :context] for x in xs))
    state, _ = decode_loop(torch, state, xs, fa, fb, context, args.warmup)
    nloc, nfine = 768 // 64, width // 32          # local_units(128), fine_units(128)
    grid_max = heads * (nloc + 2 * nfine)
    words = grid_max * 8
    buf = torch.zeros(args.steps, words, dtype=torch.int64, device=device)
    _hip.check(lib.tao_step_stamps(buf.data_ptr(), args.steps, words))
    q, k, v, rq, rk = xs
    first = context + args.warmup
    groups = []
    i = first
    try:
        while i < first + args.steps:
            torch.cuda._sleep(SPIN_CYCLES)
            start = torch.cuda.Event(enable_timing=True)
            start.record()
            count = min(STEPS_PER_SPIN, first + args.steps - i)
            launches0 = lib.tao_step_stamps_count()
            for _ in range(count):
                sl = slice(i, i + 1)
                _, state = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                                raw_k=rk[:, sl], fusion_a=fa, fusion_b=fb,
                                                alpha=0.5, state=state,
                                                position=state.get_pos())
                i += 1
            end = torch.cuda.Event(enable_timing=True)
            end.record()
            groups.append((start, end, launches0, lib.tao_step_stamps_count()))
        torch.cuda.synchronize()
        launches = lib.tao_step_stamps_count()
    finally:
        _hip.check(lib.tao_step_stamps(None, 0, 0))
    if launches != args.steps:
        raise RuntimeError(f"{launches} stamped launches for {args.steps} steps")
    raw = buf.cpu().numpy().view(np.uint64).reshape(args.steps, grid_max, 8)
    if args.timeline_raw:
        np.save(args.timeline_raw, raw)
    ticks_per_us = 100.0                             # s_memrealtime: 100 MHz
    rows = []
    for f in range(args.steps):
        fr = raw[f]
        live = fr[:, 0] != 0
        fr = fr[live]
        t = fr[:, :6].astype(np.int64)
        j = (fr[:, 6] >> np.uint64(32)).astype(np.int64)
        merged = t[:, 5] != 0
        t0 = t[:, 0].min()
        rows.append(dict(t=(t - t0) / ticks_per_us, j=j, merged=merged,
                         u=(fr[:, 6] & np.uint64(0xFFFFFFFF)).astype(np.int64),
                         start=t0, end=t[merged, 5].max(),
                         xcc=(fr[:, 7] >> np.uint64(32)).astype(np.int64),
                         smid=(fr[:, 7] & np.uint64(0xFFFFFFFF)).astype(np.int64)))
    med = lambda xs: float(np.median(np.asarray(xs)))   # noqa: E731

    def phase(sel_fn, a, b):
        return round(med([np.mean(r["t"][sel_fn(r), b] - r["t"][sel_fn(r), a]) for r in rows]), 3)

    local = lambda r: (r["j"] < nloc) & (r["t"][:, 1] != r["t"][:, 2])   # noqa: E731
    empty = lambda r: (r["j"] < nloc) & (r["t"][:, 1] == r["t"][:, 2])   # noqa: E731
    fine = lambda r: r["j"] >= nloc                                       # noqa: E731
    merge = lambda r: r["merged"]                                         # noqa: E731
    gaps = []
    spans = []
    for start, end, a, b in groups:
        for f in range(a + 1, b):
            gaps.append((int(rows[f]["start"]) - int(rows[f - 1]["end"])) / ticks_per_us)
        spans.append(((int(rows[b - 1]["end"]) - int(rows[a]["start"])) / ticks_per_us,
                      start.elapsed_time(end) * 1e3))
    crit, crit_local = [], 0
    for r in rows:
        w = int(np.argmax(np.where(r["merged"], r["t"][:, 5], -1.0)))
        crit.append(r["t"][w])
        crit_local += int(r["j"][w] < nloc)
    crit = np.asarray(crit)
    cus = med([len(set(zip(r["xcc"].tolist(), r["smid"].tolist()))) for r in rows])
    u_of = lambda r: r["u"]                                               # noqa: E731
    one_xcd = sum(int(len(np.unique(r["xcc"][u_of(r) == hh])) == 1)
                  for r in rows for hh in np.unique(u_of(r)))
    head_steps = sum(len(np.unique(u_of(r))) for r in rows)
    summary = {
        "steps": args.steps, "grid": int(len(rows[0]["j"])),
        "clock": "s_memrealtime at 100 MHz (10 ns ticks); medians over the steps of "
                 "per-launch means",
        "stamped_over_event_span": round(sum(a for a, _ in spans) / sum(b for _, b in spans), 4),
        "kernel_span_us": round(med([(r["end"] - r["start"]) / ticks_per_us for r in rows]), 3),
        "launch_gap_us": round(med(gaps), 3) if gaps else None,
        "last_start_us": round(med([r["t"][:, 0].max() for r in rows]), 3),
        "cus_used": cus,
        "heads_on_one_xcd_frac": round(one_xcd / max(head_steps, 1), 4),
        "local_units": {"start_us": round(med([np.mean(r["t"][local(r), 0]) for r in rows]), 3),
                        "loads_and_scores_us": phase(local, 0, 1),
                        "softmax_values_record_us": phase(local, 1, 2),
                        "store_ack_us": phase(local, 2, 3),
                        "arrival_count_us": phase(local, 3, 4),
                        "per_launch": round(med([local(r).sum() for r in rows]), 1)},
        "empty_local_units": {"start_us": round(med([np.mean(r["t"][empty(r), 0])
                                                     if empty(r).any() else 0.0
                                                     for r in rows]), 3),
                              "per_launch": round(med([empty(r).sum() for r in rows]), 1)},
        "fine_units": {"start_us": round(med([np.mean(r["t"][fine(r), 0]) for r in rows]), 3),
                       "read_and_record_us": phase(fine, 0, 2),
                       "store_ack_us": phase(fine, 2, 3),
                       "arrival_count_us": phase(fine, 3, 4),
                       "per_launch": round(med([fine(r).sum() for r in rows]), 1)},
        "merge": {"arrival_us": round(med([np.mean(r["t"][merge(r), 4]) for r in rows]), 3),
                  "merge_us": phase(merge, 4, 5),
                  "last_local_arrival_us": round(med([np.max(r["t"][local(r), 4])
                                                      for r in rows]), 3),
                  "last_fine_arrival_us": round(med([np.max(r["t"][fine(r), 4])
                                                     for r in rows]), 3)},
        "us_per_step_stamped": round(sum(b for _, b in spans) / args.steps, 3),
        "critical_workgroup": {"local_unit_frac": round(crit_local / len(rows), 3),
                               "start_us": round(float(np.median(crit[:, 0])), 3),
                               "arrival_us": round(float(np.median(crit[:, 4])), 3),
                               "end_us": round(float(np.median(crit[:, 5])), 3)},
    }
    return summary


def graph_launch_floor(torch, device, launches=2000):
    """Host cost of one hipGraphLaunch on this runtime: torch.cuda.CUDAGraph
    replays of two one-kernel graphs (a 1,024-element add), alternating as
    the decode graph's two executable graphs do, timed back to back."""
    x = torch.zeros(1024, device=device)
    graphs = []
    side = torch.cuda.Stream(device=device)
    side.wait_stream(torch.cuda.current_stream(device))
    with torch.cuda.stream(side):
        x.add_(1.0)                          # warm the kernel outside capture
    torch.cuda.current_stream(device).wait_stream(side)
    for _ in range(2):
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            x.add_(1.0)
        graphs.append(g)
    for g in graphs:
        g.replay()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(launches):
        graphs[i & 1].replay()
    torch.cuda.synchronize()
    us = (time.perf_counter() - t0) / launches * 1e6
    expect = 2 + launches + 1
    if float(x[0]) != expect:
        raise RuntimeError(f"graph replay count check failed: {float(x[0])} != {expect}")
    del graphs
    return us


def run_cold(torch, args, device, cfg, heads, width, context, n_states, probe):
    """Decode steps cycling through `n_states` independent 128K states, so a
    step's buffers were last touched n_states - 1 steps earlier: with 32
    states the bytes touched per cycle (each state's ring window, folded
    route, records and refresh reads) exceed the 256 MB Infinity Cache. The
    states are imports of one writer-only state (distinct device buffers,
    equal contents); every state decodes its own random tokens."""
    from tao_attention import StreamCache, new_state, tao_attention_decode
    from tao_attention.presets import index_only_page_memo
    xs, fa, fb = make_tokens(torch, context, heads, width, 100, device)
    base = new_state(0, index_only_page_memo(graph=False))
    base._ingest(*xs)
    del xs
    snap = base.export()
    del base
    # Every state is visited at least twice in the timed steps (a state's
    # first visit after the warm-up pass would otherwise be its only one).
    steps = max(args.steps // 2, 2 * n_states)
    per_state = 2 * (steps // n_states + 2) + 2          # token rows both passes read
    states, toks = [], []
    g = torch.Generator(device=device).manual_seed(101)
    for j in range(n_states):
        states.append(StreamCache.from_export(snap))
        toks.append([torch.randn((1, per_state, heads, width), generator=g,
                                 device=device).to(torch.bfloat16) for _ in range(5)])
    del snap
    torch.cuda.synchronize()
    log(f"cold: {n_states} states built")
    for j, st in enumerate(states):        # warm every state
        q, k, v, rq, rk = toks[j]
        _, states[j] = tao_attention_decode(q[:, :1], k[:, :1], v[:, :1], raw_q=rq[:, :1],
                                            raw_k=rk[:, :1], fusion_a=fa, fusion_b=fb,
                                            alpha=0.5, state=st, position=st.get_pos())
    # Each step's [1, 1, H, D] operand views are taken before the timed
    # region, as in decode_loop.
    rows = [tuple(x[:, 1 + i // n_states:2 + i // n_states] for x in toks[i % n_states])
            for i in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        j = i % n_states
        st = states[j]
        q, k, v, rq, rk = rows[i]
        _, states[j] = tao_attention_decode(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa,
                                            fusion_b=fb, alpha=0.5, state=st,
                                            position=st.get_pos())
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    del rows
    # Device time per step, GPU pre-loaded (see run_decode).
    probe.reset()
    groups = []
    base = 1 + steps // n_states + 1
    i = 0
    while i < steps:
        torch.cuda._sleep(SPIN_CYCLES)
        start = torch.cuda.Event(enable_timing=True)
        start.record()
        count = min(STEPS_PER_SPIN, steps - i)
        for _ in range(count):
            j = i % n_states
            st = states[j]
            q, k, v, rq, rk = toks[j]
            t = base + i // n_states
            sl = slice(t, t + 1)
            _, states[j] = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                                raw_k=rk[:, sl], fusion_a=fa, fusion_b=fb,
                                                alpha=0.5, state=st, position=st.get_pos())
            i += 1
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        groups.append((start, end, count))
    torch.cuda.synchronize()
    probe.events["decode_step"] = groups
    sel = states[0].route_size
    for st in states:
        st.release_execution()
    return steps, t1 - t0, sel


def run_batch(torch, args, device, cfg, heads, width, probe):
    """R one-request states at ragged lengths U[16384, 32768]
    (seeded), writer-only; `batch_steps` batched single-token steps
    (tao_attention_decode_batch, one decode step launch pair for all R plus
    the refreshes and seals the cursors hit). Also times the per-request
    loop (tao_attention_decode) on the same states for comparison."""
    import numpy as np
    from tao_attention import new_state, tao_attention_decode, tao_attention_decode_batch
    R, steps, warm = args.batch_requests, args.batch_steps, 4
    lengths = np.random.RandomState(5).randint(16384, 32769, size=R).tolist()
    g = torch.Generator(device=device).manual_seed(11)
    states = []
    for r, n in enumerate(lengths):
        st = new_state(0, cfg)
        xs = [torch.randn((1, n, heads, width), generator=g, device=device).to(torch.bfloat16)
              for _ in range(5)]
        st._ingest(*xs)
        del xs
        states.append(st)
    total = warm + steps + 2 * 8
    toks = [torch.randn((R, total, heads, width), generator=g, device=device).to(torch.bfloat16)
            for _ in range(5)]
    fa = torch.randn((heads, width, 3), generator=g, device=device) * 0.02
    fb = torch.randn((heads, width, 3), generator=g, device=device) * 0.02
    torch.cuda.synchronize()
    log(f"batch: {R} states built, lengths {min(lengths)}..{max(lengths)}")

    def step(t):
        q, k, v, rq, rk = (x[:, t:t + 1] for x in toks)
        return tao_attention_decode_batch(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa,
                                          fusion_b=fb, alpha=0.5, states=states)[0]

    for t in range(warm):
        step(t)
    bytes_per_step = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for t in range(warm, warm + steps):
        bytes_per_step.append(sum(decode_bytes(cfg, heads, width, st.route_size, st.get_pos())[0]
                                  for st in states))
        step(t)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    # Device time per batched step, GPU pre-loaded (see run_decode).
    groups = []
    t = warm + steps
    for _ in range(2):
        torch.cuda._sleep(SPIN_CYCLES)
        start = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(4):
            step(t)
            t += 1
        end = torch.cuda.Event(enable_timing=True)
        end.record()
        groups.append((start, end, 4))
    torch.cuda.synchronize()
    probe.events["batch_step"] = groups
    # The per-request loop on the same states (one tao_attention_decode each).
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    loop_steps = 8
    for _ in range(loop_steps):
        q, k, v, rq, rk = (x[:, t:t + 1] for x in toks)
        for r, st in enumerate(states):
            tao_attention_decode(q[r:r + 1], k[r:r + 1], v[r:r + 1], raw_q=rq[r:r + 1],
                                 raw_k=rk[r:r + 1], fusion_a=fa, fusion_b=fb, alpha=0.5,
                                 state=st, position=st.get_pos())
        t += 1
    torch.cuda.synchronize()
    loop_seconds = time.perf_counter() - t1
    for st in states:
        st.release_execution()
    return {"requests": R, "lengths": [min(lengths), max(lengths)], "steps": steps,
            "seconds": seconds, "bytes_per_step": sum(bytes_per_step) / len(bytes_per_step),
            "loop_tok_s": R * loop_steps / loop_seconds}


def run_model(torch, args, device, cfg):
    """Caller-side whole-model decode: the reference's published benchmark
    shape (12 layers, width 768, 6 heads x 128, vocabulary 32768; RMSNorm,
    RoPE on the normalised q / k, ReLU^2 MLP, untied embeddings) with random
    bf16 weights, one TaoMemory state per layer built writer-only at
    `model_context` tokens, then greedy decode of `model_steps` tokens through
    all 12 layers. Context only: the published whole-model figures are from
    another GPU and model weights."""
    import torch.nn.functional as F
    from tao_attention import WholeStepGraph, new_state, schedule, tao_attention_decode
    L, width, heads, dim, vocab = 12, 768, 6, 128, 32768
    g = torch.Generator(device=device).manual_seed(17)

    def w(*shape):
        return (torch.randn(shape, generator=g, device=device) * 0.02).to(torch.bfloat16)

    embed, unembed = w(vocab, width), w(width, vocab)
    layers = [dict(qkv=w(width, 3 * width), o=w(width, width), up=w(width, 4 * width),
                   down=w(4 * width, width), fa=w(heads, dim, 3).float(),
                   fb=w(heads, dim, 3).float()) for _ in range(L)]
    ctx = args.model_context
    states = []
    for layer in range(L):
        # Layer index l staggers the layer's route refreshes by 2 l tokens
        # (tao_stream.py:202-208), as in the reference's model.
        st = new_state(layer, cfg)
        xs = [torch.randn((1, ctx, heads, dim), generator=g, device=device).to(torch.bfloat16)
              for _ in range(5)]
        st._ingest(*xs)
        del xs
        states.append(st)
    inv = 1.0 / (10000.0 ** (torch.arange(0, dim, 2, device=device).float() / dim))
    span = torch.arange(ctx, ctx + 2 * args.model_steps + 32, device=device).float()[:, None] * inv
    cos_t = torch.cat((span.cos(), span.cos()), -1).to(torch.bfloat16)
    sin_t = torch.cat((-span.sin(), span.sin()), -1).to(torch.bfloat16)

    def rope(x, row):
        # rotate-half RoPE from precomputed tables: x * cos + swap(x) * (-sin, sin)
        return (x * cos_t.index_select(0, row) + x.roll(dim // 2, -1) * sin_t.index_select(0, row))

    def step(token):
        # Positions come from each state's device cursor, so the same step
        # runs eagerly and as a captured whole-step graph.
        x = embed.index_select(0, token.view(1)).view(1, 1, width)
        for lw, st in zip(layers, states):
            row = (st.device_position() - ctx).view(1)
            h = F.rms_norm(x, (width,))
            raw_q, raw_k, v = (h @ lw["qkv"]).view(1, 1, 3, heads, dim).unbind(2)
            q = rope(F.rms_norm(raw_q, (dim,)), row)
            k = rope(F.rms_norm(raw_k, (dim,)), row)
            a, _ = tao_attention_decode(q, k, v, raw_q=raw_q, raw_k=raw_k, fusion_a=lw["fa"],
                                        fusion_b=lw["fb"], alpha=0.5, state=st,
                                        position=st.get_pos())
            x = x + a.reshape(1, 1, width) @ lw["o"]
            h = F.rms_norm(x, (width,))
            x = x + F.relu(h @ lw["up"]).square() @ lw["down"]
        return (F.rms_norm(x, (width,)) @ unembed).view(-1).argmax()

    token = torch.zeros((), dtype=torch.long, device=device)
    for _ in range(8):
        token = step(token)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.model_steps):
        token = step(token)
    torch.cuda.synchronize()
    seconds = time.perf_counter() - t0
    # The same decode continued through one captured graph of the whole
    # step (WholeStepGraph): refresh tokens replay their layers' gated
    # refreshes; seal tokens and refreshes that change a route size run
    # eagerly.
    graph = WholeStepGraph(states)
    for _ in range(8):
        token = graph.step(step, token)
    torch.cuda.synchronize()
    r0, e0 = graph.replays, graph.eager_steps
    p0 = states[0].position
    refresh_tokens = sum(
        any(schedule.fines_at(p, cfg) > 0 and schedule.is_turn(p, st.layer_index, cfg)
            for st in states) for p in range(p0, p0 + args.model_steps))
    seal_tokens = sum(schedule.local_len_at(p, cfg) + 1 == cfg.serve_limit
                      for p in range(p0, p0 + args.model_steps))
    t0 = time.perf_counter()
    for _ in range(args.model_steps):
        token = graph.step(step, token)
    torch.cuda.synchronize()
    graph_seconds = time.perf_counter() - t0
    replays, eager = graph.replays - r0, graph.eager_steps - e0
    graph.release()
    for st in states:
        st.release_execution()
    return {"tok_s": args.model_steps / seconds, "seconds": seconds,
            "graph_tok_s": args.model_steps / graph_seconds, "graph_replays": replays,
            "graph_eager_steps": eager, "refresh_tokens": refresh_tokens,
            "seal_tokens": seal_tokens}


def run_prefill(torch, device, cfg, heads, width, tokens, probe):
    from tao_attention import new_state, schedule, tao_attention_prefill
    from tao_attention.presets import index_only_page_memo
    xs, fa, fb = make_tokens(torch, tokens, heads, width, 3, device, unit_raw_k=True)
    q, k, v, rq, rk = xs
    for _ in range(2):
        warm = new_state(0, index_only_page_memo())
        tao_attention_prefill(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb, alpha=0.5,
                              state=warm, position=0)
        torch.cuda.synchronize()
        del warm
    # Each timed prefill runs the whole prompt on a fresh state (its device
    # buffers allocated inside the timed region); the median of 5 is reported.
    times = []
    for _ in range(5):
        state = new_state(0, index_only_page_memo())
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        _, state = tao_attention_prefill(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb,
                                         alpha=0.5, state=state, position=0)
        torch.cuda.synchronize()
        times.append(time.perf_counter() - t0)
    t1 = time.perf_counter()
    snapshot = state.export()
    torch.cuda.synchronize()
    t2 = time.perf_counter()
    # Kernel timing of the MFMA-bound launches, GPU pre-loaded as for decode.
    probe_state = new_state(0, index_only_page_memo())
    probe_state._probe = probe
    probe_state._launch_prompt_kernels(q, k, v, rq, rk)        # warm
    torch.cuda.synchronize()
    probe.reset()
    for _ in range(3):
        torch.cuda._sleep(SPIN_CYCLES)
        probe_state._launch_prompt_kernels(q, k, v, rq, rk)
    torch.cuda.synchronize()
    probe_state._probe = None
    # Algorithmic MFMA work: causal-aware local attention + writer.
    visible = 0
    for start, width_c in schedule.chunks(0, tokens, cfg):
        ks = start - schedule.local_len_at(start, cfg)
        for p in range(start, start + width_c):
            visible += p - ks + 1
    attn_flops = visible * 4 * width * heads
    fines = schedule.fines_at(tokens, cfg)
    writer_flops = fines * heads * 2 * cfg.fine_tokens * width * width
    times.sort()
    return dict(seconds=times[len(times) // 2], seconds_range=(times[0], times[-1]),
                export_seconds=t2 - t1, attn_flops=attn_flops,
                writer_flops=writer_flops, fines=fines, snapshot_fines=snapshot["state_version"])


def run_full_sequence(torch, args, device):
    """configs[1] shape: tao_attention over B2 x T8192 x H12 x D64 bf16 with
    TaoConfig() (coarse value branch on), every query routing itself. Returns
    seconds per forward call and per forward + backward (gradients of q, k, v,
    raw_q, raw_k, fusion_a, fusion_b and alpha, as configs[1] names), each the
    mean of event-bracketed timed calls."""
    from tao_attention import TaoConfig, tao_attention
    b, t, h, d = 2, args.full_sequence_tokens, 12, 64
    g = torch.Generator(device=device).manual_seed(11)
    xs = [torch.randn(b, t, h, d, generator=g, device=device).to(torch.bfloat16)
          for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=g, device=device) * 0.02
    fb = torch.randn(h, d, 3, generator=g, device=device) * 0.02
    q, k, v, rq, rk = xs
    cfg = TaoConfig()

    def call():
        return tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb,
                             alpha=0.5, config=cfg)

    with torch.no_grad():
        for _ in range(2):
            call()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        runs = 5
        start.record()
        for _ in range(runs):
            call()
        end.record()
        torch.cuda.synchronize()
    seconds = start.elapsed_time(end) / runs * 1e-3
    # forward + backward (gradients of q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha)
    leaves = [x.detach().requires_grad_(True) for x in xs]
    fa_l, fb_l = fa.detach().requires_grad_(True), fb.detach().requires_grad_(True)
    alpha_l = torch.tensor(0.5, requires_grad=True)    # host scalar: no per-step sync
    grad = torch.randn(b, t, h, d, generator=g, device=device).to(torch.bfloat16)

    def step():
        out = tao_attention(*leaves[:3], raw_q=leaves[3], raw_k=leaves[4], fusion_a=fa_l,
                            fusion_b=fb_l, alpha=alpha_l, config=cfg)
        return torch.autograd.grad(out, leaves + [fa_l, fb_l, alpha_l], grad)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    start.record()
    for _ in range(runs):
        step()
    end.record()
    torch.cuda.synchronize()
    train_seconds = start.elapsed_time(end) / runs * 1e-3
    return dict(seconds=seconds, train_seconds=train_seconds, batch=b, tokens=t, heads=h,
                width=d)


def config0_inputs(torch, device):
    """B1 x T2048 x H4 x D64 fp32, q/k/v/raw_q/raw_k N(0,1) from seed
    0 with RoPE applied by the caller to q and k, fusion_a/b N(0, 0.02)."""
    b, t, h, d = 1, 2048, 4, 64
    g = torch.Generator().manual_seed(0)
    xs = [torch.randn(b, t, h, d, generator=g) for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=g) * 0.02
    fb = torch.randn(h, d, 3, generator=g) * 0.02
    inv = 10000.0 ** (-torch.arange(0, d // 2, dtype=torch.float64) * 2 / d)
    ang = torch.arange(t, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat((ang.cos(), ang.cos()), -1)[None, :, None, :]
    sin = torch.cat((ang.sin(), ang.sin()), -1)[None, :, None, :]
    for i in (0, 1):
        x = xs[i]
        rot = torch.cat((-x[..., d // 2:], x[..., :d // 2]), -1)
        xs[i] = (x.double() * cos + rot.double() * sin).float()
    return [x.to(device) for x in xs], fa.to(device), fb.to(device)


def run_full_sequence_f32(torch, device):
    """configs[0] on the GPU: tao_attention forward with fp32 operands and
    index_only_page_memo(graph=False); mean of 10 event-bracketed calls."""
    from tao_attention import tao_attention
    from tao_attention.presets import index_only_page_memo
    xs, fa, fb = config0_inputs(torch, device)
    cfg = index_only_page_memo(graph=False)

    def call():
        return tao_attention(*xs[:3], raw_q=xs[3], raw_k=xs[4], fusion_a=fa, fusion_b=fb,
                             alpha=0.5, config=cfg)

    with torch.no_grad():
        for _ in range(2):
            call()
        torch.cuda.synchronize()
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        runs = 10
        start.record()
        for _ in range(runs):
            call()
        end.record()
        torch.cuda.synchronize()
    return start.elapsed_time(end) / runs * 1e-3


def cpu_full_sequence_f32(torch, runs=3):
    """configs[0] as defined: the oracle's full-sequence forward (torch eager,
    fp32) on the host cores; 1 warm-up, then the median of `runs`."""
    from oracle import tao_oracle as O
    from tao_attention.presets import index_only_page_memo
    xs, fa, fb = config0_inputs(torch, torch.device("cpu"))
    geo = O.Geometry.from_config(index_only_page_memo(graph=False))
    O.training_forward(*xs, fa, fb, 0.5, geo)
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        O.training_forward(*xs, fa, fb, 0.5, geo)
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2]


def run_writers(torch, device):
    """The non-preset writers' operators at the configs[2] block shape: the
    62 sealed 256-token blocks of a 16K prefill, H32, D128, taken as one batch
    of association_statistics + association_matrix (the regularized writer's
    seal work of that prefill), and selected_fine_numerator over 4096 queries
    with M = 18 of those 62 fines. Event-timed means of 5 calls after 2."""
    from tao_attention.association_writer import association_matrix, association_statistics
    from tao_attention.indirect_fine import selected_fine_numerator
    blocks, t, h, d = 62, 256, 32, 128
    g = torch.Generator(device=device).manual_seed(13)
    k = torch.randn(blocks, t, h, d, generator=g, device=device).to(torch.bfloat16)
    v = torch.randn(blocks, t, h, d, generator=g, device=device).to(torch.bfloat16)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def timed(fn, runs=5):
        for _ in range(2):
            fn()
        torch.cuda.synchronize()
        start.record()
        for _ in range(runs):
            fn()
        end.record()
        torch.cuda.synchronize()
        return start.elapsed_time(end) / runs * 1e-3

    with torch.no_grad():
        stats_s = timed(lambda: association_statistics(k, v))
        gram, cross = association_statistics(k, v)
        solve_s = timed(lambda: association_matrix(gram, cross, unchecked=True))
        bank = association_matrix(gram, cross, unchecked=True).unsqueeze(0).permute(0, 2, 1, 3, 4)
        bank = bank.contiguous()                                   # [1, H, 62, D, D]
        q, m = 4096, 18
        channel = (torch.randn(1, q, h, m, d, generator=g, device=device) * 0.1).to(torch.bfloat16)
        ids = torch.argsort(torch.rand(q * h, blocks, generator=g, device=device),
                            dim=-1)[:, :m].reshape(1, q, h, m)   # distinct ids per query
        read_s = timed(lambda: selected_fine_numerator(channel, ids, bank))
    stats_flops = blocks * h * 2 * (2 * t * d * d)          # U^T U and U^T V
    read_flops = q * h * m * 2 * d * d
    read_bytes = h * blocks * d * d * 2 + q * h * m * (d * 2 + 8) + q * h * d * 2
    return {
        "workload": "62 blocks x 256 tokens x H32 x D128 bf16 (configs[2] seals); selected "
                    "numerator 4096 queries x H32 x M18 over those 62 fines",
        "statistics_ms": round(stats_s * 1e3, 4),
        "statistics_tflops": round(stats_flops / stats_s / 1e12, 1),
        "cholesky_solve_ms": round(solve_s * 1e3, 4),
        "solves": blocks * h,
        "selected_numerator_ms": round(read_s * 1e3, 4),
        "selected_numerator_tflops": round(read_flops / read_s / 1e12, 1),
        "selected_numerator_GBs": round(read_bytes / read_s / 1e9, 1)}


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_cores():
    """Threads for the CPU baseline: the CPUs this process may run on, capped
    by OMP_NUM_THREADS when the environment sets it (the GPU box's share)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    cap = os.environ.get("OMP_NUM_THREADS")
    if cap and cap.isdigit() and int(cap) > 0:
        n = min(n, int(cap))
    return max(1, n)


def cpu_prefill_baseline(torch, tokens, width, sample_heads, heads, runs=3):
    """Oracle prefill (torch eager on the host) of a `tokens`-token prompt
    (configs[2] inputs: N(0,1), unit-norm raw_k rows) at `sample_heads` of the
    `heads` heads: every head's work is independent and identical in kind, so
    the H32 rate is the sample's tokens/s x sample_heads / heads. One warm-up
    on 1024 tokens, then the median of `runs` runs."""
    from oracle import tao_oracle as O
    from tao_attention.presets import index_only_page_memo
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(1, tokens, sample_heads, width, generator=g) for _ in range(5)]
    xs[4] = xs[4] / xs[4].norm(dim=-1, keepdim=True)
    xs = [x.to(torch.bfloat16) for x in xs]
    fa = torch.randn(sample_heads, width, 3, generator=g) * 0.02
    fb = torch.randn(sample_heads, width, 3, generator=g) * 0.02
    geo = O.Geometry.from_config(index_only_page_memo())
    O.OracleStream(0, geo).prefill(*(x[:, :1024] for x in xs), fa, fb, 0.5)
    times = []
    for _ in range(runs):
        ora = O.OracleStream(0, geo)
        t0 = time.perf_counter_ns()
        ora.prefill(*xs, fa, fb, 0.5)
        times.append((time.perf_counter_ns() - t0) * 1e-9)
    times.sort()
    sec = times[len(times) // 2]
    return {"tok_s": tokens / sec * sample_heads / heads,
            "sample": f"median of {runs} oracle prefills of the full {tokens}-token prompt at "
                      f"H{sample_heads} D{width} ({sec:.2f} s each, after a 1024-token warm-up), "
                      f"scaled to H{heads} by x{sample_heads}/{heads} (heads are independent); "
                      f"CPU {cpu_model()}"}


def cpu_baseline(torch, state, xs, fa, fb, steps, runs=3):
    """Oracle decode (torch eager on the host) from the GPU state's snapshot.

    One warm-up decode, then `runs` runs of `steps` single-token decodes each
    (the state advances through all of them); returns the median tok/s.
    """
    from oracle import tao_oracle as O
    snap = state.export()
    cpu = {}
    for key, value in snap.items():
        cpu[key] = value
    cpu["local"] = tuple(t.cpu() for t in snap["local"])
    cpu["packed_fine_c"] = snap["packed_fine_c"].cpu()
    cpu["pages"] = [(pz.cpu(), None, fz.cpu()) for pz, _, fz in snap["pages"]]
    cpu["pending_z"] = [z.cpu() for z in snap["pending_z"]]
    cpu["route_ids"] = tuple(t.cpu() for t in snap["route_ids"])
    del snap
    ora = O.OracleStream.from_export(cpu, 0)
    toks = [x[:, :1 + runs * steps].cpu() for x in xs]
    fa_c, fb_c = fa.cpu(), fb.cpu()
    ora.decode(*(t[:, :1] for t in toks), fa_c, fb_c, 0.5)       # warm-up
    rates = []
    for r in range(runs):
        t0 = time.perf_counter_ns()
        for i in range(1 + r * steps, 1 + (r + 1) * steps):
            ora.decode(*(t[:, i:i + 1] for t in toks), fa_c, fb_c, 0.5)
        rates.append(steps / ((time.perf_counter_ns() - t0) * 1e-9))
    rates.sort()
    return rates[len(rates) // 2], steps


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--context", type=int, default=131072)
    ap.add_argument("--prefill-tokens", type=int, default=16384)
    ap.add_argument("--cold-states", type=int, default=32)
    ap.add_argument("--cpu-steps", type=int, default=64)
    ap.add_argument("--cpu-prefill-heads", type=int, default=4)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-cold", action="store_true")
    ap.add_argument("--no-prefill", action="store_true")
    ap.add_argument("--batch-requests", type=int, default=32)
    ap.add_argument("--batch-steps", type=int, default=128)
    ap.add_argument("--no-batch", action="store_true")
    ap.add_argument("--model-context", type=int, default=131072)
    ap.add_argument("--model-steps", type=int, default=128)
    ap.add_argument("--no-model", action="store_true")
    ap.add_argument("--full-sequence-tokens", type=int, default=8192)
    ap.add_argument("--no-full-sequence", action="store_true")
    ap.add_argument("--no-writers", action="store_true")
    ap.add_argument("--timeline", action="store_true",
                    help="only the decode step's per-phase clock-stamp timeline (diagnostic: "
                         "prints its summary as the JSON line instead of the bench result)")
    ap.add_argument("--timeline-raw", default=None,
                    help="with --timeline: also save the raw stamp frames (uint64 "
                         "[steps, workgroups, 8]) to this .npy path")
    ap.add_argument("--calibrate-copy-mib", type=int, default=0,
                    help="after the run, copy a buffer of this many MiB 4 times (a plain "
                         "copy kernel of known size, to scale rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU: the TaoMemory operator path has no "
              "multi-GPU mode in this build (heads and requests would shard with no "
              "exchange); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch
    from tao_attention import _hip
    from tao_attention.presets import index_only_page_memo
    _hip.lib()
    device = torch.device("cuda:0")
    cfg = index_only_page_memo(graph=False)
    heads, width = 32, 128
    probe = Probe(torch)
    if args.timeline:
        log("decode timeline: building 128K state")
        summary = run_timeline(torch, args, device, cfg, heads, width)
        print(json.dumps({"decode_timeline": summary, "context": args.context,
                          "heads": heads, "head_dim": width}), flush=True)
        return

    log("decode: building 128K state")
    state, xs, fa, fb, seconds, graph, steps_bytes = run_decode(
        torch, args, device, cfg, heads, width, args.context, 4, probe)
    from tao_attention import schedule
    first, last = args.context + args.warmup, args.context + args.warmup + args.steps
    refreshes = schedule.count_turns(first, last, 0, cfg)
    seals = schedule.fines_at(last, cfg) - schedule.fines_at(first, cfg)
    window = (f"{args.steps} single-token steps timed (positions {first}..{last - 1}, after "
              f"{args.warmup} untimed warm-up steps from {args.context}): {refreshes} route "
              f"refreshes and {seals} seal{'s' if seals != 1 else ''} inside the timed steps")
    tok_s = args.steps / seconds
    n_step = probe.count("decode_step")
    step_ms = probe.total_ms("decode_step") / max(n_step, 1)
    alg_bytes = sum(b for b, _ in steps_bytes) / len(steps_bytes)
    own_bytes = sum(o for _, o in steps_bytes) / len(steps_bytes)
    achieved = alg_bytes / (step_ms * 1e-3) / 1e9
    log(f"decode: {tok_s:.1f} tok/s (graph preset: dispatch replay "
        f"{args.steps / graph['dispatch'][0]:.1f}, hipGraph replay "
        f"{args.steps / graph['hipgraph'][0]:.1f}), step kernel {step_ms * 1e3:.2f} us, "
        f"{achieved:.0f} GB/s")
    result = {
        "metric": METRIC,
        "value": round(tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(seconds / args.steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic N(0,1) bf16 operands (seeded); state built writer-only",
        "config": {"workload": f"configs[3]: advancing decode of one request x layer from a "
                               f"{args.context}-token state, H32 D128; {window}; "
                               "index_only_page_memo(graph=False): each step is issued by "
                               "the native C++ driver as direct launches (the graph preset "
                               "is timed on the same steps as decode_graph)",
                   "context": args.context, "heads": heads, "head_dim": width,
                   "selected_fines": state.route_size, "timed_refreshes": refreshes,
                   "timed_seals": seals},
        "roofline": {"bound": "hbm", "kernel": "decode_step_kernel<128> per step (one launch: the units and the last workgroup's merge per head), with the %d route refreshes (route_refresh_kernel + fold_kernel) and %d seals (writer + epilogue + fold) of the timed steps amortised" % (refreshes, seals),
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4),
                     "traffic": DECODE_STEP_TRAFFIC_BYTES if args.context == 131072 else None,
                     "kernel_us": round(step_ms * 1e3, 3),
                     "algorithmic_bytes_per_launch": int(alg_bytes),
                     "algorithmic_basis": "reference step: H*M*(D^2+3D)*2 + 2*H*D*2 per token, "
                                          "+ H*(P+E)*D*2 on refresh steps",
                     "own_bytes_per_step": int(own_bytes),
                     "own_GBs": round(own_bytes / (step_ms * 1e-3) / 1e9, 1)},
        "decode_graph": {"preset": "index_only_page_memo(graph=True)",
                         "replay": "dispatch (default): the epoch's recorded step "
                                   "arguments dispatched directly",
                         "tok_s": round(args.steps / graph["dispatch"][0], 2),
                         "ms_per_step": round(graph["dispatch"][0] / args.steps * 1e3, 4),
                         "timed_steps": graph["dispatch"][1],
                         "hipgraph": {"replay": "TAO_GRAPH_REPLAY=hipgraph: per token one "
                                                "hipGraphExecKernelNodeSetParams + "
                                                "hipGraphLaunch of the one-node step graph "
                                                "(two executable graphs alternating)",
                                      "tok_s": round(args.steps / graph["hipgraph"][0], 2),
                                      "ms_per_step": round(graph["hipgraph"][0] / args.steps
                                                           * 1e3, 4),
                                      "timed_steps": graph["hipgraph"][1],
                                      "launch_floor_us": round(graph["launch_floor_us"], 2),
                                      "launch_floor": "host us per torch.cuda.CUDAGraph.replay "
                                                      "of a one-kernel graph (two graphs "
                                                      "alternating), the runtime's floor under "
                                                      "any per-token graph replay"}},
    }
    if not args.no_cold:
        log("cold decode: building states")
        del xs
        steps, cold_s, cold_sel = run_cold(torch, args, device, cfg, heads, width,
                                           args.context, args.cold_states, probe)
        cold_ms = probe.total_ms("decode_step") / max(probe.count("decode_step"), 1)
        cold_bytes, cold_own = decode_bytes(cfg, heads, width, cold_sel, args.context + 9)
        result["decode_cold"] = {
            "states": args.cold_states, "tok_s": round(steps / cold_s, 2),
            "kernel_us": round(cold_ms * 1e3, 3),
            "achieved_GBs": round(cold_bytes / (cold_ms * 1e-3) / 1e9, 1),
            "touched_bytes_per_cycle": int(cold_own * args.cold_states),
            "timed_steps": steps, "visits_per_state": steps // args.cold_states,
            "note": "timed steps cycle through independent 128K states (no refresh in these "
                    "steps), each state visited visits_per_state times after a warm-up "
                    "visit; a cycle touches touched_bytes_per_cycle bytes (each state's ring "
                    "window, folded route and records), above the 256 MB Infinity Cache when "
                    "it exceeds 268435456"}
        log(f"cold: {steps / cold_s:.1f} tok/s, kernel {cold_ms * 1e3:.2f} us")
        xs = None
    if not args.no_prefill:
        log("prefill 16K")
        pre = run_prefill(torch, device, cfg, heads, width, args.prefill_tokens, probe)
        attn_ms = probe.total_ms("local_attention") / max(probe.count("local_attention"), 1)
        writer_ms = probe.total_ms("writer") / max(probe.count("writer"), 1)
        flops = pre["attn_flops"] + pre["writer_flops"]
        tflops = flops / ((attn_ms + writer_ms) * 1e-3) / 1e12
        result["prefill_tokens_per_s"] = round(args.prefill_tokens / pre["seconds"], 1)
        result["prefill"] = {
            "tokens": args.prefill_tokens, "seconds": round(pre["seconds"], 5),
            "timing": "median of 5 prefills, each on a fresh state (allocation included)",
            "seconds_range": [round(x, 5) for x in pre["seconds_range"]],
            "export_seconds": round(pre["export_seconds"], 5)}
        result["roofline_prefill"] = {
            "bound": "mfma", "kernels": "local_attn_kernel<128> + writer_kernel<128>",
            "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "traffic": None,
            "attention_ms": round(attn_ms, 4), "writer_ms": round(writer_ms, 4),
            "algorithmic_gflop": round(flops / 1e9, 2)}
        log(f"prefill: {result['prefill_tokens_per_s']} tok/s, mfma {tflops:.1f} TFLOP/s")
    if not args.no_batch:
        log("batched decode: building states")
        bt = run_batch(torch, args, device, cfg, heads, width, probe)
        b_ms = probe.total_ms("batch_step") / max(probe.count("batch_step"), 1)
        b_tok_s = bt["requests"] * bt["steps"] / bt["seconds"]
        b_achieved = bt["bytes_per_step"] / (b_ms * 1e-3) / 1e9
        result["decode_batch"] = {
            "workload": "configs[4]: %d one-request states (lengths U[16384,32768], seed 5; "
                        "%d..%d), H32 D128, index_only_page_memo; %d batched single-token "
                        "steps through tao_attention_decode_batch" % (
                            bt["requests"], bt["lengths"][0], bt["lengths"][1], bt["steps"]),
            "tok_s": round(b_tok_s, 1),
            "ms_per_step": round(bt["seconds"] / bt["steps"] * 1e3, 4),
            "kernel_us_per_step": round(b_ms * 1e3, 2),
            "achieved_GBs": round(b_achieved, 1),
            "frac": round(b_achieved / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_step": int(bt["bytes_per_step"]),
            "algorithmic_basis": "sum over requests of the reference step (as roofline)",
            "per_request_loop_tok_s": round(bt["loop_tok_s"], 1)}
        log(f"batched decode: {b_tok_s:.1f} tok/s, step {b_ms * 1e3:.1f} us, "
            f"{b_achieved:.0f} GB/s; per-request loop {bt['loop_tok_s']:.1f} tok/s")
    if not args.no_model:
        log("whole-model decode: building 12 layer states")
        md = run_model(torch, args, device, cfg)
        result["model_decode"] = {
            "model": "12 layers, width 768, 6 heads x 128, vocabulary 32768 (the reference's "
                     "published benchmark shape), random bf16 weights, batch 1",
            "context": args.model_context, "steps": args.model_steps,
            "tok_s": round(md["tok_s"], 1),
            "whole_step_graph_tok_s": round(md["graph_tok_s"], 1),
            "whole_step_graph_tokens": {"replayed": md["graph_replays"],
                                        "eager (seal / route-size change / warm-up before a "
                                        "capture)": md["graph_eager_steps"],
                                        "with a refresh in some layer": md["refresh_tokens"],
                                        "with a seal": md["seal_tokens"]},
            "layer_indices": "0..11: layer l refreshes at first_fine + 2 l + 24 k "
                             "(tao_stream.py:202-208), so about half the tokens carry a "
                             "refresh in some layer",
            "note": "caller-side greedy decode through all 12 layers (eager, then the same "
                    "decode continued through one captured graph of the whole step, "
                    "WholeStepGraph; index_only_page_memo); the reference publishes 107.192 "
                    "tok/s (memo) and "
                    "123.816 tok/s (memo + regional graph) at 128K for its trained model on an "
                    "RTX 4090 (docs/benchmarks.md:94): context, not a like-for-like baseline"}
        log(f"whole-model decode: {md['tok_s']:.1f} tok/s eager, {md['graph_tok_s']:.1f} tok/s "
            f"whole-step graph at {args.model_context} context")
    if not args.no_full_sequence:
        log("full-sequence read (tao_attention forward, configs[1] shape)")
        fs = run_full_sequence(torch, args, device)
        result["full_sequence_forward"] = {
            "workload": "configs[1] shape: tao_attention B%d x T%d x H%d x D%d bf16, "
                        "TaoConfig() (coarse values on), every query routes itself; synthetic "
                        "N(0,1) operands; the backward takes the gradients of q, k, v, raw_q, "
                        "raw_k, fusion_a, fusion_b and alpha"
                        % (fs["batch"], fs["tokens"], fs["heads"], fs["width"]),
            "ms": round(fs["seconds"] * 1e3, 4),
            "tokens_per_s": round(fs["batch"] * fs["tokens"] / fs["seconds"], 1),
            "forward_backward_ms": round(fs["train_seconds"] * 1e3, 4),
            "forward_backward_tokens_per_s": round(fs["batch"] * fs["tokens"] /
                                                   fs["train_seconds"], 1)}
        log(f"full-sequence forward: {fs['seconds'] * 1e3:.3f} ms, "
            f"{fs['batch'] * fs['tokens'] / fs['seconds']:.1f} tok/s; forward + backward "
            f"{fs['train_seconds'] * 1e3:.3f} ms")
    if not args.no_full_sequence:
        log("fp32 full-sequence forward (configs[0])")
        f32_s = run_full_sequence_f32(torch, device)
        result["full_sequence_f32"] = {
            "workload": "configs[0]: tao_attention forward B1 x T2048 x H4 x D64 fp32, "
                        "index_only_page_memo(graph=False), seed 0, RoPE on q/k; fp32 "
                        "semantics: every bf16 rounding point of the bf16 path rounds to fp32",
            "ms": round(f32_s * 1e3, 4), "tokens_per_s": round(2048 / f32_s, 1)}
        log(f"fp32 forward: {f32_s * 1e3:.3f} ms")
    if not args.no_writers:
        log("non-preset writer operators (configs[2] block shape)")
        result["writers"] = run_writers(torch, device)
        log(f"writers: {result['writers']}")
    if not args.no_cpu_baseline:
        log("cpu baseline (oracle, torch eager on host cores)")
        cores = cpu_cores()
        torch.set_num_threads(cores)
        xs_cpu, _, _ = make_tokens(torch, 1 + 3 * args.cpu_steps, heads, width, 7, device)
        cpu_tok_s, sample = cpu_baseline(torch, state, xs_cpu, fa, fb, args.cpu_steps)
        result["cpu_baseline"] = {
            "value": round(cpu_tok_s, 4), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"median of 3 runs of {sample} single-token decodes (after 1 warm-up) "
                      f"of the oracle (torch eager) from the GPU state's snapshot at position "
                      f"{state.get_pos()} (H32 D128); torch.set_num_threads({cores}) = the "
                      f"CPUs this process may run on (sched_getaffinity, capped by "
                      f"OMP_NUM_THREADS when set); CPU {cpu_model()}; torch {torch.__version__}"}
        log(f"cpu baseline: {cpu_tok_s:.3f} tok/s on {cores} threads")
        if not args.no_prefill:
            pre_cpu = cpu_prefill_baseline(torch, args.prefill_tokens, width,
                                           args.cpu_prefill_heads, heads)
            result["cpu_baseline_prefill"] = {
                "value": round(pre_cpu["tok_s"], 2), "unit": "tokens/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": pre_cpu["sample"]}
            log(f"cpu prefill baseline: {pre_cpu['tok_s']:.1f} tokens/s (H32-equivalent)")
        if not args.no_full_sequence:
            f32_cpu = cpu_full_sequence_f32(torch)
            result["cpu_baseline_full_sequence_f32"] = {
                "value": round(2048 / f32_cpu, 1), "unit": "tokens/s",
                "cores": torch.get_num_threads(), "kind": "port",
                "sample": f"configs[0] as defined (B1 x T2048 x H4 x D64 fp32): median of 3 "
                          f"oracle forwards after 1 warm-up, {f32_cpu:.3f} s each; CPU "
                          f"{cpu_model()}"}
            log(f"cpu configs[0] baseline: {f32_cpu:.3f} s per forward")
    state.release_execution()
    if args.calibrate_copy_mib:
        n = args.calibrate_copy_mib * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device=device)
        dst = torch.empty_like(src)
        for _ in range(4):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["copy_calibration"] = {"bytes_read": n * 4, "bytes_written": n * 4, "copies": 4}
        del src, dst
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
