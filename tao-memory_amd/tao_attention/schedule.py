"""Closed forms of the streaming schedule (host-side integers).

All of the reference's lifecycle is a function of the causal cursor: the
local window grows to ``serve_limit`` then seals its oldest ``fine_tokens``
block (tao_stream.py:914-917, 959-967), so the local length, the number of
sealed fines and the chunk boundaries follow from the position alone. Route
refreshes follow tao_stream.py:202-210 and the selected counts
tao_stream.py:29-37.
"""


def local_len_at(position, config):
    """Exact-local tokens held before the token at ``position`` is appended."""
    limit = config.serve_limit
    if position < limit:
        return position
    return config.local_keep + (position - limit) % config.fine_tokens


def fines_at(position, config):
    """Sealed fine memories after ``position`` tokens have been processed."""
    limit = config.serve_limit
    if position < limit:
        return 0
    return (position - limit) // config.fine_tokens + 1


def next_chunk(position, desired, config):
    """StreamCache.next_chunk (tao_stream.py:914-917)."""
    return min(desired, config.fine_tokens,
               config.serve_limit - local_len_at(position, config))


def chunks(position, tokens, config):
    """[(start, width)] of the reference's prefill loop (operator.py:100-127)."""
    out = []
    start = position
    end = position + tokens
    while start < end:
        width = next_chunk(start, end - start, config)
        out.append((start, width))
        start += width
    return out


def seals_in(start, width, config):
    """True if processing [start, start + width) ends with a seal."""
    return local_len_at(start, config) + width == config.serve_limit


def is_turn(position, layer, config):
    """Route refresh at ``position`` for ``layer`` (tao_stream.py:202-208)."""
    first = config.first_fine
    first_turn = first + config.layer_stagger * layer
    return position == first or (
        position >= first_turn
        and (position - first_turn) % config.route_period == 0)


def next_turn(position, layer, config):
    """First refresh strictly after ``position`` (tao_stream.py:209-210)."""
    first_turn = config.first_fine + config.layer_stagger * layer
    if position < first_turn:
        return first_turn
    period = config.route_period
    return first_turn + period * ((position - first_turn) // period + 1)


def routed_counts(completed, pending, config):
    """(coarse pages, eligible fines, selected M), tao_stream.py:29-37."""
    group = config.coarse_group
    coarse_budget = config.budget(group * completed)
    coarse = min(completed, (2 * coarse_budget + group - 1) // group)
    eligible = group * coarse + pending
    return coarse, eligible, min(eligible, config.budget(group * completed + pending))


def sub_chunks(start, width, layer, config):
    """[(start, count, refresh)] route segments of one chunk (:205-223)."""
    out = []
    offset = 0
    while offset < width:
        absolute = start + offset
        count = min(width - offset, next_turn(absolute, layer, config) - absolute)
        out.append((absolute, count, is_turn(absolute, layer, config)))
        offset += count
    return out


def count_turns(lo, hi, layer, config):
    """Number of refresh positions in [lo, hi) (closed form of is_turn)."""
    if hi <= lo:
        return 0
    first = config.first_fine
    first_turn = first + config.layer_stagger * layer
    period = config.route_period
    count = 0
    if lo <= first < hi and first < first_turn:
        count += 1
    start = max(lo, first_turn)
    if start < hi:
        k0 = -(-(start - first_turn) // period)
        k1 = (hi - 1 - first_turn) // period
        count += max(0, k1 - k0 + 1)
    return count

