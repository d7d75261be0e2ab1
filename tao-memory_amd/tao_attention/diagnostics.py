"""Closed-form diagnostics counters of one request x layer (host code).

The reference's StreamCache.bytes() (tao_stream.py:988-1094) reports
counters that its process() (:919-986) and _read_progressive / _read_reused
(:162-230, :236-374) update per chunk and per route segment. Every one of
them is a function of the call sequence: chunk boundaries, route turns,
sealed fines and route sizes are closed forms of the cursor (schedule.py).
StreamCache keeps a log of its calls and evaluates the counters here on
demand, so the per-token decode path does no bookkeeping for them.

Log entries:
  ("call", pos0, tokens, route_size)  one call of tokens > 1 (the reference's
                                       chunk loop, allow_page_memo False)
  ("run", pos0, n, route_size)        n consecutive one-token calls from pos0
                                       (allow_page_memo True); n = None for
                                       the open run, ending at the cursor
  ("release", pos0, 0, 0)             release_execution (drops the memo)
route_size is the state's route size when the entry begins.
"""

import numpy as np

from . import schedule


def _is_turn(p, layer, config):
    first = config.first_fine
    first_turn = first + config.layer_stagger * layer
    return (p == first) | ((p >= first_turn) & ((p - first_turn) % config.route_period == 0))


def _fines(p, config):
    limit = config.serve_limit
    return np.where(p < limit, 0, (p - limit) // config.fine_tokens + 1)


def _local_len(p, config):
    limit = config.serve_limit
    return np.where(p < limit, p, config.local_keep + (p - limit) % config.fine_tokens)


class _Counts:
    def __init__(self):
        self.coarse_matrix_contractions = 0
        self.fine_matrix_contractions = 0
        self.fine_candidate_scores = 0
        self.route_query_heads = 0
        self.route_selection_calls = 0
        self.pending_only_fine_present_query_heads = 0
        self.fused_fine_calls = 0
        self.peak_local_length_tokens = 0
        self.peak_logical_cache_bytes = 0
        self.peak_physical_cache_tensor_bytes = 0
        self.memo = False


def _history_bytes(completed, pending, B, H, D, config):
    """LayerState.logical_bytes (tao_stream.py:518-527), vectorised."""
    elements = (completed * (config.coarse_group + 1) + pending) * (D * D + D)
    if config.coarse_index_only:
        elements = elements - completed * D * D
    return elements * B * H * 2


def pending_writer_parts(B, H, D, config):
    """Bytes of each fp32 pending sum config's writer holds
    (tao_stream.py:463-478): gram and cross [B, H, D, D] (regularized and
    feature-mass writers), cross, mass and square mass (structured), mass
    (feature writers); none for the softmax writer."""
    dd, d = B * H * D * D * 4, B * H * D * 4
    writer = config.fine_writer
    return {"gram": dd if writer in ("regularized_association",
                                     "feature_mass_association") else 0,
            "cross": dd if writer != "softmax" else 0,
            "mass": d if writer in ("feature_mass_association",
                                    "structured_gram_association") else 0,
            "square": d if writer == "structured_gram_association" else 0}


def pending_present(fines, config):
    """Whether the pending sums exist after `fines` seals: from the first
    seal until a completed page drops them, which only the page-value branch
    does (never in the index-only preset, tao_stream.py:486-497)."""
    fines = np.asarray(fines, dtype=np.int64)
    return (fines > 0) & ((fines % config.coarse_group > 0) | config.coarse_index_only)


def _pending_writer_bytes(fines, B, H, D, config):
    """LayerState.pending_writer_bytes (tao_stream.py:514-516) after `fines`
    seals."""
    total = sum(pending_writer_parts(B, H, D, config).values())
    return np.where(pending_present(fines, config), total, 0)


def _segment(c, positions, widths, single, route_size, layer, B, H, D, config):
    """Account the chunks starting at `positions` (widths `widths`); `single`
    marks one-token calls. Returns the route size after the last chunk."""
    p = np.asarray(positions, dtype=np.int64)
    w = np.asarray(widths, dtype=np.int64)
    if p.size == 0:
        return route_size
    group = config.coarse_group
    f = _fines(p, config)
    completed, pending = f // group, f % group
    pairs = {int(x): schedule.routed_counts(int(x) // group, int(x) % group, config)
             for x in np.unique(f)}
    eligible = np.array([pairs[int(x)][1] for x in f], dtype=np.int64)
    selected = np.array([pairs[int(x)][2] for x in f], dtype=np.int64)
    qh = B * w * H
    if not config.coarse_index_only:
        c.coarse_matrix_contractions += int((qh * completed).sum())
    has = f > 0
    # Route turns inside each chunk [p, p + w): at most one per chunk start for
    # the one-token chunks; multi-token chunks count theirs in closed form.
    turns = np.zeros_like(p)
    first_turn_off = np.full_like(p, -1)
    if (w == 1).all():
        on = _is_turn(p, layer, config) & has
        turns = on.astype(np.int64)
        first_turn_off = np.where(on, 0, -1)
    for i in (np.nonzero(has)[0] if not (w == 1).all() else ()):
        s, width = int(p[i]), int(w[i])
        t = s if schedule.is_turn(s, layer, config) else schedule.next_turn(s, layer, config)
        n = 0
        first = -1
        while t < s + width:
            if first < 0:
                first = t - s
            n += 1
            t = schedule.next_turn(t, layer, config)
        turns[i], first_turn_off[i] = n, first
    rq = turns * B * H
    c.route_query_heads += int(rq.sum())
    c.route_selection_calls += int((turns * B).sum())
    c.fine_candidate_scores += int((rq * eligible).sum())
    # Route size of each chunk's first segment: the size after the last
    # earlier chunk that refreshed (or the carried size).
    refreshed = turns > 0
    idx = np.where(refreshed, np.arange(p.size), -1)
    last = np.maximum.accumulate(idx)
    prev_last = np.concatenate(([-1], last[:-1]))
    m_prev = np.where(prev_last >= 0, selected[np.maximum(prev_last, 0)], route_size)
    n_before = np.where(refreshed, first_turn_off, w)
    contr = B * H * (n_before * m_prev + (w - n_before) * selected)
    c.fine_matrix_contractions += int(contr[has].sum())
    # One _read_reused call per route segment of a chunk with history.
    segments = np.where(refreshed, turns + (first_turn_off > 0), 1)
    c.fused_fine_calls += int(segments[has].sum())
    c.pending_only_fine_present_query_heads += int(
        (qh * ((pending > 0) & (completed == 0))).sum())
    all_k = _local_len(p, config) + w
    c.peak_local_length_tokens = max(c.peak_local_length_tokens, int(all_k.max()))
    hist = _history_bytes(completed, pending, B, H, D, config)
    key = B * all_k * H * D * 2
    logical, physical = hist + 2 * key, hist + 3 * key
    if config.fine_writer != "softmax":
        # The pending statistic sums (tao_stream.py:953-958, 969-978):
        # counted before the chunk and, at a seal, after it (the first sums
        # of a new page; the pre-seal peak stays when a page drops them).
        logical = logical + _pending_writer_bytes(f, B, H, D, config)
        physical = physical + _pending_writer_bytes(f, B, H, D, config)
        sealed = all_k == config.serve_limit
        f1 = f + sealed
        after = (_history_bytes(f1 // group, f1 % group, B, H, D, config)
                 + _pending_writer_bytes(f1, B, H, D, config))
        keep = B * config.local_keep * H * D * 2
        logical = np.where(sealed, np.maximum(logical, after + 2 * keep), logical)
        physical = np.where(sealed, np.maximum(physical, after + 3 * keep), physical)
    c.peak_logical_cache_bytes = max(c.peak_logical_cache_bytes, int(logical.max()))
    c.peak_physical_cache_tensor_bytes = max(c.peak_physical_cache_tensor_bytes,
                                             int(physical.max()))
    # Page-normalisation memo: built by a non-refresh one-token read with
    # history (memo preset, index-only), dropped by a seal after the read.
    memo_cfg = config.q1_page_normalization_memo and config.coarse_index_only
    build = single & has & ~refreshed if memo_cfg else np.zeros_like(has)
    seal = all_k == config.serve_limit
    last_build = int(np.nonzero(build)[0].max()) if build.any() else -1
    last_seal = int(np.nonzero(seal)[0].max()) if seal.any() else -1
    if last_build > last_seal:
        c.memo = True
    elif last_seal >= 0:
        c.memo = False
    return int(selected[last[-1]]) if last[-1] >= 0 else route_size


def counters(config, layer, B, H, D, log, position):
    """Counters of the logged calls; `position` closes an open run."""
    c = _Counts()
    for kind, pos0, n, route_size in log:
        if kind == "release":
            c.memo = False
            continue
        if kind == "run":
            count = (position - pos0) if n is None else n
            pos = np.arange(pos0, pos0 + count, dtype=np.int64)
            _segment(c, pos, np.ones_like(pos), np.ones(pos.size, dtype=bool), route_size,
                     layer, B, H, D, config)
        else:
            ch = schedule.chunks(pos0, n, config)
            _segment(c, [s for s, _ in ch], [w for _, w in ch], np.zeros(len(ch), dtype=bool),
                     route_size, layer, B, H, D, config)
    return c


def memo_bytes(present, completed, pending, B, H, D):
    """Bytes of the memo tuple (pending z, page z, page weights), bf16."""
    if not present:
        return 0
    pages = completed + (pending > 0)
    return B * H * D * 2 * (pending + 2 * pages)
