"""TaoMemory CPU oracle: the reference's inference arithmetic restated in torch.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker or the timed CPU baseline; the product never routes through it.

Every function cites the reference file:line it restates (paths relative to
the reference repository root). Tensors are CPU, layout [B, T, H, D] for
token streams, [B, H, S, D] for per-fine descriptors, [B, H, S, D, D] for the
fine-memory bank. Rounding points follow the reference's torch/Triton casts;
see ``oracle/numerics.py`` for the three backend choices fixed here.

Pinning (tests/test_oracle.py): closed forms for the schedule and budget;
torch's own bf16 ``logsumexp``/``softmax`` for the composite ops; fp64 brute
force for writer, read, local attention and fusion; stable-argsort brute force
for routing; invariants (decode == 1-token prefill, chunked == whole prefill,
export/import equality, banks independent of queries).
"""

import math

import torch

from .numerics import (BF16, F32, exp32, fold_sum, log32, logsumexp,
                       quarter_sum, rnd, softmax)

NEG_INF = float("-inf")


# ----------------------------------------------------------------------------
# Closed forms: config.py:54-60, tao_stream.py:29-37, 196-211, 914-917
# ----------------------------------------------------------------------------

class Geometry:
    """Geometry fields of the reference TaoConfig (config.py:7-19)."""

    def __init__(self, fine_tokens=256, local_keep=512, coarse_group=8,
                 route_period=24, layer_stagger=2, budget_root_scale=2,
                 budget_offset=2, coarse_index_only=True, page_memo=False):
        self.fine_tokens = fine_tokens
        self.local_keep = local_keep
        self.coarse_group = coarse_group
        self.route_period = route_period
        self.layer_stagger = layer_stagger
        self.budget_root_scale = budget_root_scale
        self.budget_offset = budget_offset
        self.coarse_index_only = coarse_index_only
        self.page_memo = page_memo            # q1_page_normalization_memo

    @classmethod
    def from_config(cls, config):
        return cls(config.fine_tokens, config.local_keep, config.coarse_group,
                   config.route_period, config.layer_stagger,
                   config.budget_root_scale, config.budget_offset,
                   config.coarse_index_only, config.q1_page_normalization_memo)

    @property
    def serve_limit(self):
        return self.local_keep + self.fine_tokens

    def budget(self, count):
        """config.py:54-60: min(n, ceil(sqrt(scale*n)) + offset)."""
        if count <= 0:
            return 0
        root = math.isqrt(self.budget_root_scale * count)
        if root * root < self.budget_root_scale * count:
            root += 1
        return min(count, root + self.budget_offset)

    def routed_counts(self, completed, pending):
        """tao_stream.py:29-37 -> (coarse pages, eligible fines, selected M)."""
        group = self.coarse_group
        coarse_budget = self.budget(group * completed)
        coarse = min(completed, (2 * coarse_budget + group - 1) // group)
        eligible = group * coarse + pending
        selected = min(eligible, self.budget(group * completed + pending))
        return coarse, eligible, selected

    def is_turn(self, position, layer):
        """tao_stream.py:202-208: route refresh positions of one layer."""
        first = self.serve_limit
        first_turn = first + self.layer_stagger * layer
        return position == first or (
            position >= first_turn
            and (position - first_turn) % self.route_period == 0)

    def next_turn(self, position, layer):
        """tao_stream.py:209-210: next refresh strictly after ``position``."""
        first_turn = self.serve_limit + self.layer_stagger * layer
        if position < first_turn:
            return first_turn
        period = self.route_period
        return first_turn + period * ((position - first_turn) // period + 1)


# ----------------------------------------------------------------------------
# Writer and page summaries: tao_stream.py:56-77, 478-501
# ----------------------------------------------------------------------------

def seal_softmax(raw_k, v):
    """Softmax fine writer for one block, tao_stream.py:66-77.

    raw_k, v: [B, F, H, D] (F = fine_tokens). Returns z [B, H, D] and
    C [B, H, D, D] in raw_k's dtype. Per channel: m = max_t k,
    e = r(exp(r(k - m))), Z = r(sum_t e), P = r(e / Z),
    z = r(m + r(log Z)), C = r(P^T V) with fp32 accumulation.
    """
    dtype = raw_k.dtype
    top = raw_k.amax(dim=1, keepdim=True)
    shifted = rnd(raw_k.to(F32) - top.to(F32), dtype)
    e = rnd(exp32(shifted.to(F32)), dtype)
    total = rnd(quarter_sum(e, 1), dtype)                    # [B, H, D]
    prob = rnd(e.to(F32) / total.unsqueeze(1).to(F32), dtype)  # [B, F, H, D]
    z = rnd(top.squeeze(1).to(F32) + rnd(log32(total.to(F32)), dtype).to(F32),
            dtype)
    c = torch.einsum("bthd,bthe->bhde", prob.to(torch.float64),
                     v.to(torch.float64))
    return z, rnd(c, dtype)


def page_summary(z_group):
    """Completed page / pending-page descriptor r(logsumexp over fines).

    z_group: [B, H, n, D] -> [B, H, D]; tao_stream.py:283, 412, 485.
    """
    return logsumexp(z_group, 2)


def segment_weights(fine_z, page_z_of_fine):
    """sw = r(exp(r(z - pz))), tao_stream.py:349 / query_fresh_fine.py:38-39."""
    dtype = fine_z.dtype
    diff = rnd(fine_z.to(F32) - page_z_of_fine.to(F32), dtype)
    return rnd(exp32(diff.to(F32)), dtype)


def page_coarse_matrix(z_group, page_z, c_group):
    """Coarse value matrix of a completed page (non-index-only), :486-499.

    weight = r(exp(r(z - page_z))); page_C = r(sum_s weight[s,d] C_s[d,e]).
    """
    weight = segment_weights(z_group, page_z.unsqueeze(2))     # [B,H,8,D]
    pc = torch.einsum("bhsd,bhsde->bhde", weight.to(torch.float64),
                      c_group.to(torch.float64))
    return rnd(pc, z_group.dtype)


# ----------------------------------------------------------------------------
# Routing and the selected read: tao_stream.py:253-374, query_fresh_fine.py
# ----------------------------------------------------------------------------

def topk_oldest(scores, count):
    """tao_stream.py:50-53: stable descending order, first ``count``."""
    return scores.argsort(dim=-1, descending=True, stable=True)[
        ..., :min(count, scores.shape[-1])]


def query_weights(raw_q):
    """h = r(softmax_D(raw_q)), tao_stream.py:253-254 / :421."""
    return softmax(raw_q, -1)


def page_weights(page_z):
    """pw = r(softmax over pages), page_z [B, H, P, D], tao_stream.py:291/414."""
    return softmax(page_z, 2)


def page_values(h, pw):
    """hv = r(h * pw): [B, Q, H, D] x [B, H, P, D] -> [B, Q, H, P, D] (:298)."""
    return rnd(h.unsqueeze(3).to(F32) * pw.unsqueeze(1).to(F32), h.dtype)


def route(hv_anchor, fine_sw, completed, pending, geometry):
    """Routing refresh from one anchor query, tao_stream.py:310-357.

    hv_anchor: [B, H, P, D] (P = completed + (pending > 0)).
    fine_sw:   [B, H, S, D] segment weights of every sealed fine.
    Returns (chosen_page [B, H, coarse] int64 ascending,
             selected_id [B, H, M] int64 in score order, scores dict).
    """
    b, heads, _, d = hv_anchor.shape
    dtype = hv_anchor.dtype
    group = geometry.coarse_group
    coarse, _, fine_count = geometry.routed_counts(completed, pending)
    pages, ids = [], []
    chosen = torch.zeros((b, heads, 0), dtype=torch.int64)
    page_mass = None
    if coarse:
        page_mass = rnd(fold_sum(hv_anchor[:, :, :completed], -1), dtype)
        chosen = topk_oldest(page_mass, coarse).sort(-1).values
        segment = torch.arange(group)
        pages.append(chosen.unsqueeze(-1).expand(b, heads, coarse, group)
                     .reshape(b, heads, coarse * group))
        ids.append((chosen.unsqueeze(-1) * group + segment)
                   .reshape(b, heads, coarse * group))
    if pending:
        pend = torch.arange(pending).view(1, 1, pending).expand(b, heads, pending)
        pages.append(torch.full_like(pend, completed))
        ids.append(completed * group + pend)
    cand_page = torch.cat(pages, -1)
    cand_id = torch.cat(ids, -1)
    e = cand_id.shape[-1]
    hv_c = torch.gather(hv_anchor, 2, cand_page.unsqueeze(-1).expand(b, heads, e, d))
    sw_c = torch.gather(fine_sw, 2, cand_id.unsqueeze(-1).expand(b, heads, e, d))
    channel = rnd(hv_c.to(F32) * sw_c.to(F32), dtype)
    mass = rnd(fold_sum(channel, -1), dtype)
    order = topk_oldest(mass, fine_count)
    selected = cand_id.gather(-1, order)
    return chosen, selected, {"page_mass": page_mass, "mass": mass,
                              "candidates": cand_id}


def selected_read(hv, fine_sw, selected, bank_c, group):
    """query_fresh_fine.py:8-75: fine = r(r(num) / den).

    hv [B, Q, H, P, D]; fine_sw [B, H, S, D]; selected [B, H, M];
    bank_c [B, H, S, D, D]. ch = r(hv[page] * sw); num = r(sum_m ch @ C)
    (fp64 here; fp32 in the reference, so parity is to tolerance);
    den = r(sum_m r(sum_d ch)); returns (fine [B,Q,H,D], ch [B,Q,H,M,D]).
    """
    b, q, heads, _, d = hv.shape
    dtype = hv.dtype
    m = selected.shape[-1]
    page = selected // group
    hv_sel = torch.gather(hv, 3, page[:, None, :, :, None].expand(b, q, heads, m, d))
    sw_sel = torch.gather(fine_sw, 2, selected.unsqueeze(-1).expand(b, heads, m, d))
    ch = rnd(hv_sel.to(F32) * sw_sel.unsqueeze(1).to(F32), dtype)  # [B,Q,H,M,D]
    c_sel = torch.gather(bank_c, 2, selected[..., None, None].expand(b, heads, m, d, d))
    num = torch.einsum("bqhmd,bhmde->bqhe", ch.to(torch.float64),
                       c_sel.to(torch.float64))
    num = rnd(num, dtype)
    per_slot = rnd(fold_sum(ch, -1), dtype)                 # [B,Q,H,M]
    den = rnd(fold_sum(per_slot, -1), dtype)                # [B,Q,H]
    fine = rnd(num.to(F32) / den.unsqueeze(-1).to(F32), dtype)
    return fine, ch


FEATURE_WRITERS = ("feature_mass_association", "structured_gram_association")


def mass_descriptor(mass):
    """Descriptor of an fp32 feature mass: r(log mass), the fp32 log rounded
    once more to bf16 (tao_stream.py:60-65, 280-283, 483)."""
    return rnd(log32(mass.float()), torch.bfloat16)


def feature_read(h, read_z, matrices):
    """Numerator-only mixture read of the feature writers (tao_stream.py:
    301-305, 362-367): coef = feature_read_coefficients(h, z) per query and
    matrix, out = r(sum_p sum_d coef[p, d] M_p[d, e]) with no denominator.
    h [B, Q, H, D]; read_z [B, H, P, D]; matrices [B, H, P, D, D]."""
    from . import writers as W
    coef = W.feature_read_coefficients(h, read_z.unsqueeze(1))       # [B,Q,H,P,D]
    out = torch.einsum("bqhpd,bhpde->bqhe", coef.to(torch.float64),
                       matrices.to(torch.float64))
    return rnd(out, h.dtype)


def coarse_read(h, page_z_completed, page_c):
    """Coarse value read (non-index-only), tao_stream.py:299-305."""
    dtype = h.dtype
    weight = softmax(page_z_completed, 2)
    hv = page_values(h, weight)
    out = torch.einsum("bthpd,bhpde->bthe", hv.to(torch.float64),
                       page_c.to(torch.float64))
    return rnd(out, dtype)


# ----------------------------------------------------------------------------
# Fusion: fusion_pointwise.py:10-117, operator.py:86-97
# ----------------------------------------------------------------------------

def fusion(raw_q, local, coarse, fine, fusion_a, fusion_b, alpha,
           coarse_on, fine_on, arith=BF16):
    """Three-branch presence-aware fusion with every cast explicit.

    Streaming (arith=bf16): the kernel math is bf16 regardless of the stream
    dtype (Triton casts, fusion_pointwise.py:103-121, 151-166); results are
    stored in raw_q's dtype. tao_attention's _fuse_training (operator.py:
    21-38) rounds every torch op to the operand dtype instead: arith =
    raw_q.dtype (the two agree for bf16 operands).
    """
    dtype = raw_q.dtype
    q = raw_q.to(F32)
    a = rnd(fusion_a.to(F32), arith).to(F32)                # [H, D, 3]
    bias = rnd(fusion_b.to(F32), arith).to(F32)
    present = int(coarse_on) + int(fine_on)
    local_bias = rnd(torch.tensor(math.log(present) if present else 0.0,
                                  dtype=torch.float64), arith).to(F32)
    scores = []
    for branch in range(3):
        prod = rnd(a[..., branch] * q, arith).to(F32)
        s = rnd(prod + bias[..., branch], arith)
        if branch == 0:
            s = rnd(s.to(F32) + local_bias, arith)
        if (branch == 1 and not coarse_on) or (branch == 2 and not fine_on):
            s = torch.full_like(s, NEG_INF)
        scores.append(s)
    score = rnd(torch.stack(scores, -1), dtype)            # stored in dtype
    rho = rnd(softmax(score, -1), dtype)                    # F.softmax + .to
    gain = rnd(torch.tensor(2 * alpha, dtype=torch.float64), dtype).to(F32)
    rl, rc, rf = (rho[..., i].to(F32) for i in range(3))
    local_twice = rnd(2.0 * local.to(F32), arith).to(F32)
    coarse_scaled = rnd(gain * coarse.to(F32), arith).to(F32)
    fine_scaled = rnd(gain * fine.to(F32), arith).to(F32)
    lt = rnd(rl * local_twice, arith).to(F32)
    ct = rnd(rc * coarse_scaled, arith).to(F32)
    ft = rnd(rf * fine_scaled, arith).to(F32)
    first = rnd(lt + ct, arith).to(F32)
    return rnd(rnd(first + ft, arith), dtype)


# ----------------------------------------------------------------------------
# Local attention: flash_attention.py:16-37 (SDPA, scale 1/sqrt(D))
# ----------------------------------------------------------------------------

def local_attention(q, k, v):
    """Suffix-aligned causal attention in fp64, rounded once to q's dtype.

    Square -> causal, Tq == 1 -> all keys, else query row i sees keys
    col <= Tk - Tq + i: one formula covers the reference's three SDPA modes.
    """
    tq, tk, d = q.shape[1], k.shape[1], q.shape[-1]
    s = torch.einsum("bqhd,bkhd->bhqk", q.to(torch.float64), k.to(torch.float64))
    s = s / math.sqrt(d)
    rows = tk - tq + torch.arange(tq)
    allowed = torch.arange(tk)[None, :] <= rows[:, None]
    s = s.masked_fill(~allowed, NEG_INF)
    p = torch.softmax(s, -1)
    out = torch.einsum("bhqk,bkhd->bqhd", p, v.to(torch.float64))
    return rnd(out, q.dtype)


# ----------------------------------------------------------------------------
# Streaming state: tao_stream.py:126-527 (LayerState), 790-986 (StreamCache)
# ----------------------------------------------------------------------------

class OracleStream:
    """One request x layer streaming state (softmax writer).

    Semantic content equals the reference StreamCache: local exact window,
    sealed fine z / C, completed page summaries, route ids, position.
    """

    def __init__(self, layer_index, geometry=None, writer="softmax"):
        self.layer = layer_index
        self.g = geometry or Geometry()
        self.writer = writer           # a TaoConfig.fine_writer
        self.pending_gram = self.pending_cross = None
        self.pending_mass = self.pending_square = None   # feature writers
        self.position = 0
        self.local = None            # (k, v, raw_k) [B, n, H, D]
        self.fine_z = []             # [B, H, D] per sealed fine
        self.fine_c = []             # [B, H, D, D]
        self.page_z = []             # completed pages [B, H, D]
        self.page_c = []             # completed pages [B, H, D, D] (non-index-only)
        self.route_ids = None        # (chosen [B,1,H,K'], selected [B,1,H,M])
        self.state_version = 0
        self.route_refreshes = 0
        self.fine_seal_events = 0
        self._bank = None            # stacked fine_c, rebuilt after a seal
        # Diagnostics counters of StreamCache.bytes() (tao_stream.py:
        # 1044-1094), updated where the reference updates them.
        self.diag = dict(coarse_matrix_contractions=0, fine_matrix_contractions=0,
                         fine_candidate_scores=0, route_query_heads=0,
                         route_selection_calls=0, pending_only_fine_present_query_heads=0,
                         fused_fine_calls=0, peak_local_length_tokens=0,
                         peak_logical_cache_bytes=0, peak_physical_cache_tensor_bytes=0)
        self.memo = False            # page_normalization_memo is not None
        self.last_route_queries = 0
        self.last_fine_contractions = 0

    # -- state views ------------------------------------------------------
    @property
    def completed(self):
        return len(self.page_z)

    @property
    def pending(self):
        return len(self.fine_z) - self.completed * self.g.coarse_group

    def page_descriptors(self):
        """page_z over completed pages plus the pending summary (:267-290):
        r(logsumexp) of the pending fines' z, or for the feature writers
        r(log) of their summed feature mass (:280-283)."""
        parts = list(self.page_z)
        if self.pending:
            if self.writer in FEATURE_WRITERS:
                parts.append(mass_descriptor(self.pending_mass))
            else:
                start = self.completed * self.g.coarse_group
                parts.append(page_summary(torch.stack(self.fine_z[start:], 2)))
        return torch.stack(parts, 2)

    def fine_segment_weights(self, page_z):
        z = torch.stack(self.fine_z, 2)                       # [B,H,S,D]
        page_of = torch.arange(z.shape[2]) // self.g.coarse_group
        return segment_weights(z, page_z.index_select(2, page_of))

    # -- lifecycle --------------------------------------------------------
    def next_chunk(self, desired):
        """tao_stream.py:914-917."""
        current = 0 if self.local is None else self.local[0].shape[1]
        return min(desired, self.g.fine_tokens, self.g.serve_limit - current)

    def seal(self, raw_k, v):
        """tao_stream.py:435-512 for the softmax writer and, with
        writer="regularized_association", the association value matrices
        (:56-77) and pending statistic sums (:463-499): C = association_matrix
        of the block's statistics; the statistics add to the pending sums in
        seal order; a completed page's matrix is association_matrix of the
        sums, which then restart (never, index-only, as in the reference)."""
        if self.writer in FEATURE_WRITERS:
            self._seal_feature(raw_k, v)
            return
        z, c = seal_softmax(raw_k, v)
        if self.writer == "regularized_association":
            from . import writers as W
            gram, cross = W.association_statistics(raw_k, v)
            c = W.association_matrix(gram, cross)[1]
            if self.pending_gram is None:
                self.pending_gram, self.pending_cross = gram, cross
            else:
                self.pending_gram = self.pending_gram + gram
                self.pending_cross = self.pending_cross + cross
        self.fine_z.append(z)
        self.fine_c.append(c)
        self._bank = None
        self.state_version += 1
        group = self.g.coarse_group
        if self.pending == group:
            start = self.completed * group
            zs = torch.stack(self.fine_z[start:], 2)
            pz = page_summary(zs)
            self.page_z.append(pz)
            if not self.g.coarse_index_only and self.writer == "regularized_association":
                from . import writers as W
                self.page_c.append(W.association_matrix(self.pending_gram,
                                                        self.pending_cross)[1])
                self.pending_gram = self.pending_cross = None
            elif not self.g.coarse_index_only:
                self.page_c.append(page_coarse_matrix(
                    zs, pz, torch.stack(self.fine_c[start:], 2)))

    def _seal_feature(self, raw_k, v):
        """_seal for the feature writers (tao_stream.py:56-65) and their
        pending sums and page descriptors (:463-499): z = r(log mass); C =
        association_matrix (feature mass) or structured_matrix (structured
        Gram) of the block's statistics; the fp32 mass (and the gram /
        square mass and cross) add up in seal order; a completed page's z is
        r(log) of the summed mass. With page values the page's matrix comes
        from the summed statistics, and the sums then restart; index-only,
        they never restart (the reference clears them only in its page-value
        branch, :488-497), so page z and the pending descriptor are r(log) of
        the mass summed over every fine sealed so far."""
        from . import writers as W
        if self.writer == "structured_gram_association":
            square, cross, mass = W.structured_statistics(raw_k, v)
            c = W.structured_matrix(square, cross, mass, self.g.fine_tokens)[1]
            self.pending_square = square if self.pending_square is None else \
                self.pending_square + square
        else:
            gram, cross, mass = W.association_statistics(raw_k, v, with_mass=True)
            c = W.association_matrix(gram, cross)[1]
            self.pending_gram = gram if self.pending_gram is None else self.pending_gram + gram
        self.pending_cross = cross if self.pending_cross is None else self.pending_cross + cross
        self.pending_mass = mass if self.pending_mass is None else self.pending_mass + mass
        self.fine_z.append(mass_descriptor(mass))
        self.fine_c.append(c.to(raw_k.dtype))
        self._bank = None
        self.state_version += 1
        group = self.g.coarse_group
        if self.pending == group:
            self.page_z.append(mass_descriptor(self.pending_mass))
            if not self.g.coarse_index_only:
                if self.writer == "structured_gram_association":
                    pc = W.structured_matrix(self.pending_square, self.pending_cross,
                                             self.pending_mass, self.g.fine_tokens * group)[1]
                else:
                    pc = W.association_matrix(self.pending_gram, self.pending_cross)[1]
                self.page_c.append(pc.to(raw_k.dtype))
                self.pending_gram = self.pending_cross = None
                self.pending_mass = self.pending_square = None

    def logical_bytes(self, b, heads, d):
        """LayerState.logical_bytes (tao_stream.py:518-527), bf16."""
        count = self.completed * (self.g.coarse_group + 1) + self.pending
        elements = count * (d * d + d)
        if self.g.coarse_index_only:
            elements -= self.completed * d * d
        return elements * b * heads * 2

    def pending_writer_bytes(self):
        """LayerState.pending_writer_bytes (tao_stream.py:514-516): the
        pending gram, cross, feature mass and square mass sums the writer
        holds, counted at the reference's fp32 (4 bytes an element; the
        oracle holds gram and cross in fp64)."""
        return sum(t.numel() * 4 for t in (self.pending_gram, self.pending_cross,
                                           self.pending_mass, self.pending_square)
                   if t is not None)

    def release_execution(self):
        """StreamCache.release_execution (:838-844): drops the memo."""
        self.memo = False

    def read(self, raw_q, allow_page_memo=False):
        """LayerState._read_progressive + _read_reused (:196-374)."""
        b, t, heads, d = raw_q.shape
        self.last_route_queries = 0            # LayerState.read (:162-164)
        self.last_fine_contractions = 0
        if not self.fine_z:
            zero = torch.zeros_like(raw_q)
            return zero, zero, False, False
        page_z = self.page_descriptors()
        pw = page_weights(page_z)
        sw = self.fine_segment_weights(page_z)
        if self._bank is None or self._bank.shape[2] != len(self.fine_c):
            self._bank = torch.stack(self.fine_c, 2)
        bank = self._bank
        h = query_weights(raw_q)
        hv = page_values(h, pw)                               # [B,T,H,P,D]
        coarse_on = bool(self.page_z) and not self.g.coarse_index_only
        feature = self.writer in FEATURE_WRITERS
        if coarse_on and feature:
            coarse = feature_read(h, page_z[:, :, :self.completed],
                                  torch.stack(self.page_c, 2))
        elif coarse_on:
            coarse = coarse_read(h, page_z[:, :, :self.completed],
                                 torch.stack(self.page_c, 2))
        else:
            coarse = torch.zeros_like(raw_q)
        fine = torch.empty_like(raw_q)
        offset = 0
        while offset < t:
            absolute = self.position + offset
            refresh = self.g.is_turn(absolute, self.layer)
            count = min(t - offset, self.g.next_turn(absolute, self.layer) - absolute)
            if refresh:
                chosen, selected, _ = route(hv[:, offset], sw, self.completed,
                                            self.pending, self.g)
                self.route_ids = (chosen.unsqueeze(1), selected.unsqueeze(1))
                self.route_refreshes += 1
                self.last_route_queries += b * heads                  # :215-216
            elif (allow_page_memo and t == 1 and self.g.page_memo
                  and self.g.coarse_index_only):
                self.memo = True                                      # :292-295
            self.last_fine_contractions += b * count * heads * self.route_ids[1].shape[-1]
            self.diag["fused_fine_calls"] += 1                        # :244, :370
            sel = self.route_ids[1][:, 0]
            if feature:
                b_, heads_, m_ = sel.shape
                z_all = torch.stack(self.fine_z, 2)
                z_sel = torch.gather(z_all, 2, sel.unsqueeze(-1).expand(b_, heads_, m_, d))
                c_sel = torch.gather(bank, 2, sel[..., None, None].expand(b_, heads_, m_, d, d))
                part = feature_read(h[:, offset:offset + count], z_sel, c_sel)
            else:
                part, _ = selected_read(hv[:, offset:offset + count], sw, sel, bank,
                                        self.g.coarse_group)
            fine[:, offset:offset + count] = part
            offset += count
        return coarse, fine, coarse_on, True

    def process(self, raw_q, raw_k, q, k, v, allow_page_memo=False):
        """StreamCache.process (:919-979): local, read, then seal at 768."""
        if self.local is None:
            all_k, all_v, all_raw = k, v, raw_k
        else:
            all_k = torch.cat((self.local[0], k), 1)
            all_v = torch.cat((self.local[1], v), 1)
            all_raw = torch.cat((self.local[2], raw_k), 1)
        if all_k.shape[1] > self.g.serve_limit:
            raise ValueError("chunk crosses a fine seal boundary")
        local = local_attention(q, all_k, all_v)
        b, t, heads, d = raw_q.shape
        query_heads = b * t * heads
        _, eligible, _ = self.g.routed_counts(self.completed, self.pending)
        if not self.g.coarse_index_only:
            self.diag["coarse_matrix_contractions"] += query_heads * self.completed
        coarse, fine, c_on, f_on = self.read(raw_q, allow_page_memo)
        if self.pending and not self.completed:
            self.diag["pending_only_fine_present_query_heads"] += query_heads
        self.diag["fine_matrix_contractions"] += self.last_fine_contractions
        self.diag["route_query_heads"] += self.last_route_queries
        self.diag["route_selection_calls"] += self.last_route_queries // heads
        self.diag["fine_candidate_scores"] += self.last_route_queries * eligible
        self.diag["peak_local_length_tokens"] = max(self.diag["peak_local_length_tokens"],
                                                    all_k.shape[1])
        history = self.logical_bytes(b, heads, d) + self.pending_writer_bytes()   # :953-958
        key_bytes = all_k.numel() * 2
        self._preseal = (history + 2 * key_bytes, history + 3 * key_bytes)
        if all_k.shape[1] == self.g.serve_limit:
            self.memo = False                                         # :445-449
            self.fine_seal_events += 1
            ft, keep = self.g.fine_tokens, self.g.local_keep
            self.seal(all_raw[:, :ft], all_v[:, :ft])
            self.local = (all_k[:, -keep:].clone(), all_v[:, -keep:].clone(),
                          all_raw[:, -keep:].clone())
        else:
            self.local = (all_k, all_v, all_raw)
        if self.writer != "softmax":
            # :969-978: the first pending sums of a new page count in the
            # peak; the pre-seal peak stays when a completed page drops them.
            after = self.logical_bytes(b, heads, d) + self.pending_writer_bytes()
            local_bytes = self.local[0].numel() * 2
            self._preseal = (max(self._preseal[0], after + 2 * local_bytes),
                             max(self._preseal[1], after + 3 * local_bytes))
        return local, coarse, fine, c_on, f_on

    def prefill(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
                position=None):
        """operator.py:70-127: split at next_chunk, fuse each chunk."""
        if position is not None and position != self.position:
            raise ValueError("position must match this request's causal cursor")
        outputs = []
        start = 0
        single = q.shape[1] == 1          # allow_page_memo (operator.py:80-83)
        while start < q.shape[1]:
            width = self.next_chunk(q.shape[1] - start)
            end = start + width
            local, coarse, fine, c_on, f_on = self.process(
                raw_q[:, start:end], raw_k[:, start:end], q[:, start:end],
                k[:, start:end], v[:, start:end], allow_page_memo=single)
            # StreamCache.advance (:981-986)
            self.diag["peak_logical_cache_bytes"] = max(self.diag["peak_logical_cache_bytes"],
                                                        self._preseal[0])
            self.diag["peak_physical_cache_tensor_bytes"] = max(
                self.diag["peak_physical_cache_tensor_bytes"], self._preseal[1])
            if c_on or f_on:
                out = fusion(raw_q[:, start:end], local, coarse, fine,
                             fusion_a, fusion_b, alpha, c_on, f_on)
            else:
                out = local
            outputs.append(out)
            self.position += width
            start = end
        return torch.cat(outputs, 1)

    def decode(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
               position=None):
        """operator.py:130-138."""
        if q.shape[1] != 1:
            raise ValueError("decode accepts exactly one new query/key/value")
        return self.prefill(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
                            position)

    def export(self, config=None, layer_index=None):
        """Snapshot in the reference's schema (tao_stream.py:853-877): every key
        the reference writes; config is the TaoConfig.export() dict the
        snapshot declares (default: this geometry with the memo and graph
        flags off), layer_index defaults to this stream's layer."""
        group = self.g.coarse_group
        if config is None:
            g = self.g
            config = dict(fine_tokens=g.fine_tokens, local_keep=g.local_keep,
                          coarse_group=g.coarse_group, route_period=g.route_period,
                          layer_stagger=g.layer_stagger, budget_root_scale=g.budget_root_scale,
                          budget_offset=g.budget_offset, fine_writer=self.writer,
                          coarse_index_only=g.coarse_index_only,
                          q1_page_normalization_memo=False, q1_history_region_graph=False)
        packed = torch.stack(self.fine_c, 2) if self.fine_c else None
        z = self.fine_z
        pages = []
        for index, pz in enumerate(self.page_z):
            pc = self.page_c[index] if self.page_c else None
            pages.append((pz.clone(), None if pc is None else pc.clone(),
                          torch.stack(z[index * group:(index + 1) * group], 2)))
        pending = [zz.clone() for zz in z[self.completed * group:]]
        f32 = lambda t: None if t is None else t.to(torch.float32).clone()
        return {
            "layer_index": self.layer if layer_index is None else layer_index,
            "config": dict(config),
            "route_interval": 2,
            "fusion_mode": "pointwise",
            "fused_fine": True,
            "position": self.position,
            "local": None if self.local is None else tuple(t.clone() for t in self.local),
            "packed_fine_c": packed,
            "pages": pages,
            "pending_z": pending,
            "pending_square_mass": f32(self.pending_square),
            "pending_mass": f32(self.pending_mass),
            "pending_gram": f32(self.pending_gram),
            "pending_cross": f32(self.pending_cross),
            "route_ids": None if self.route_ids is None else tuple(t.clone() for t in self.route_ids),
            "route_key": None,
            "state_version": self.state_version,
            "route_refreshes": self.route_refreshes,
            "fine_seal_events": self.fine_seal_events,
        }

    @classmethod
    def from_export(cls, saved, layer_index, geometry=None):
        """Restore from a snapshot dict (tao_stream.py:879-912)."""
        state = cls(layer_index, geometry,
                    writer=saved.get("config", {}).get("fine_writer", "softmax"))
        if saved.get("pending_gram") is not None:
            state.pending_gram = saved["pending_gram"].double().clone()
        if saved.get("pending_cross") is not None:
            state.pending_cross = saved["pending_cross"].double().clone()
        if saved.get("pending_square_mass") is not None:
            state.pending_square = saved["pending_square_mass"].float().clone()
        if saved.get("pending_mass") is not None:
            state.pending_mass = saved["pending_mass"].float().clone()
        group = state.g.coarse_group
        state.position = saved["position"]
        state.local = (None if saved["local"] is None
                       else tuple(t.clone() for t in saved["local"]))
        packed = saved["packed_fine_c"]
        for index, (pz, pc, fz) in enumerate(saved["pages"]):
            state.page_z.append(pz.clone())
            if pc is not None:
                state.page_c.append(pc.clone())
            for j in range(group):
                state.fine_z.append(fz[:, :, j].clone())
                state.fine_c.append(packed[:, :, index * group + j].clone())
        offset = len(saved["pages"]) * group
        for j, z in enumerate(saved["pending_z"]):
            state.fine_z.append(z.clone())
            state.fine_c.append(packed[:, :, offset + j].clone())
        state.route_ids = (None if saved["route_ids"] is None
                           else tuple(t.clone() for t in saved["route_ids"]))
        state.state_version = saved["state_version"]
        state.route_refreshes = saved["route_refreshes"]
        state.fine_seal_events = saved["fine_seal_events"]
        return state



# ----------------------------------------------------------------------------
# Full-sequence read: operator.py:21-52 (tao_attention, _fuse_training),
# tao_stream.py:530-787 (read_training and its helpers)
# ----------------------------------------------------------------------------

def training_forward(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
                     geometry=None, return_routes=False, writer="softmax"):
    """tao_attention forward with fresh routing at every query.

    Restates read_training (tao_stream.py:668-757) with route_interval=1 and
    _fuse_training (operator.py:21-38):
      * local: tile t = tokens [F t, min(T, F t + F)) attends suffix-causally
        to keys [max(0, F t - keep), end) (_local_training_corrected_4k,
        :760-787, and its ragged fallback :763-775 are the same windows);
      * tile t reads the first max(0, t - keep / F) sealed fines (:734);
        fines come from _seal_training_all (:80-123, the softmax writer per
        block), page summaries from _training_metadata / _tile_metadata
        (:530-593: logsumexp over the 8 fines of a completed page, over the
        first `pending` fines of the pending page);
      * every query routes itself (_read_training_group, :596-665: the same
        candidate construction, segment weights and stable top-k as the
        streaming refresh) and reads its own selection
        (selected_read.py:156-173: fine = r(r(num) / r(den)));
      * coarse read of completed pages when not index-only (:609-615);
      * fusion with coarse presence pos >= first_coarse and not index-only,
        fine presence pos >= first_fine, output = local where neither is
        present (operator.py:46-52, 21-38).
    Tiles are evaluated one at a time; the reference's stacking of up to 8
    tiles with equal (completed, pending?, M, length) on the batch axis
    (:700-748) changes no value.

    writer="regularized_association" keeps the softmax writer's z and read
    and replaces the value matrices (tao_stream.py:72-74, 80-123, 565-569):
    C_f = association_matrix(association_statistics(block f)) and, for a
    completed page, association_matrix of the in-order sums of its fines'
    statistics (oracle/writers.py).

    The feature writers (index-only) follow _seal_training_all's feature
    branches and _training_metadata (tao_stream.py:80-97, 543-549): z = r(log
    mass), C from association_matrix / structured_matrix of the block, page
    z = r(log) of the in-order mass sums, and each query's read the
    numerator-only mixture over its selection (:656-662).

    Returns out [B, T, H, D] (and, with return_routes, a dict tile -> selected
    ids [B, Q, H, M] in score order).
    """
    g = geometry or Geometry()
    b, total, heads, d = q.shape
    ft, keep, group = g.fine_tokens, g.local_keep, g.coarse_group
    local = torch.empty_like(q)
    for start in range(0, total, ft):
        end = min(total, start + ft)
        k0 = max(0, start - keep)
        local[:, start:end] = local_attention(q[:, start:end], k[:, k0:end], v[:, k0:end])
    routes = {}
    n_tiles = -(-total // ft)
    lag = keep // ft                                     # config.visibility_tiles
    visible_max = max(0, n_tiles - 1 - lag)
    if total <= g.serve_limit or visible_max == 0:       # :682-688
        return (local, routes) if return_routes else local
    zs, cs, stats, masses = [], [], [], []
    feature = writer in FEATURE_WRITERS
    for f in range(visible_max):
        kb, vb = raw_k[:, f * ft:(f + 1) * ft], v[:, f * ft:(f + 1) * ft]
        if feature:
            from . import writers as W
            if writer == "structured_gram_association":
                square, cross, mass = W.structured_statistics(kb, vb)
                c = W.structured_matrix(square, cross, mass, ft)[1].to(kb.dtype)
                stats.append((square, cross))
            else:
                gram, cross, mass = W.association_statistics(kb, vb, with_mass=True)
                c = W.association_matrix(gram, cross)[1].to(kb.dtype)
                stats.append((gram, cross))
            z = mass_descriptor(mass)
            masses.append(mass)
        else:
            z, c = seal_softmax(kb, vb)
        if writer == "regularized_association":
            from . import writers as W
            stats.append(W.association_statistics(kb, vb))
            c = W.association_matrix(*stats[-1])[1]
        zs.append(z)
        cs.append(c)
    fine_z = torch.stack(zs, 2)                          # [B, H, S, D]
    bank = torch.stack(cs, 2)                            # [B, H, S, D, D]
    full_pages = visible_max // group
    def mass_sum(lo, hi):
        total = masses[lo]
        for i in range(lo + 1, hi):
            total = total + masses[i]
        return total

    if feature:
        page_z_full = [mass_descriptor(mass_sum(p * group, (p + 1) * group))
                       for p in range(full_pages)]
    else:
        page_z_full = [page_summary(fine_z[:, :, p * group:(p + 1) * group])
                       for p in range(full_pages)]
    page_c_full = []
    if not g.coarse_index_only and feature:
        from . import writers as W
        for p in range(full_pages):
            first = sum(stats[p * group + i][0] for i in range(group))
            cross = sum(stats[p * group + i][1] for i in range(group))
            if writer == "structured_gram_association":
                pc = W.structured_matrix(first, cross, mass_sum(p * group, (p + 1) * group),
                                         ft * group)[1]
            else:
                pc = W.association_matrix(first, cross)[1]
            page_c_full.append(pc.to(raw_k.dtype))
    elif not g.coarse_index_only and writer == "regularized_association":
        from . import writers as W
        for p in range(full_pages):
            gram = sum(stats[p * group + i][0] for i in range(group))
            cross = sum(stats[p * group + i][1] for i in range(group))
            page_c_full.append(W.association_matrix(gram, cross)[1])
    elif not g.coarse_index_only:
        page_c_full = [page_coarse_matrix(fine_z[:, :, p * group:(p + 1) * group],
                                          page_z_full[p], bank[:, :, p * group:(p + 1) * group])
                       for p in range(full_pages)]
    first_coarse = keep + group * ft                     # config.py:47-48
    out = local.clone()
    for tile in range(n_tiles):
        start = tile * ft
        end = min(total, start + ft)
        visible = max(0, tile - lag)
        if not visible:
            continue
        completed, pending = divmod(visible, group)
        parts = list(page_z_full[:completed])
        if pending and feature:
            parts.append(mass_descriptor(mass_sum(completed * group, visible)))
        elif pending:
            parts.append(page_summary(fine_z[:, :, completed * group:visible]))
        page_z = torch.stack(parts, 2)
        pw = page_weights(page_z)
        page_of = torch.arange(visible) // group
        sw = segment_weights(fine_z[:, :, :visible], page_z.index_select(2, page_of))
        h = query_weights(raw_q[:, start:end])
        hv = page_values(h, pw)                          # [B, Q, H, P, D]
        nq = end - start
        flat = hv.reshape(b * nq, heads, *hv.shape[3:])
        sw_flat = sw.unsqueeze(1).expand(b, nq, *sw.shape[1:]).reshape(b * nq, *sw.shape[1:])
        _, selected, _ = route(flat, sw_flat, completed, pending, g)
        selected = selected.reshape(b, nq, heads, -1)    # [B, Q, H, M]
        routes[tile] = selected
        fine = torch.empty_like(raw_q[:, start:end])
        tile_bank = bank[:, :, :visible]
        for i in range(nq):
            if feature:
                sel = selected[:, i]                     # [B, H, M]
                m_ = sel.shape[-1]
                z_sel = torch.gather(fine_z[:, :, :visible], 2,
                                     sel.unsqueeze(-1).expand(b, heads, m_, d))
                c_sel = torch.gather(tile_bank, 2, sel[..., None, None].expand(b, heads, m_, d, d))
                part = feature_read(h[:, i:i + 1], z_sel, c_sel)
            else:
                part, _ = selected_read(hv[:, i:i + 1], sw, selected[:, i], tile_bank, group)
            fine[:, i:i + 1] = part
        coarse_on = start >= first_coarse and not g.coarse_index_only
        fine_on = start >= g.serve_limit                 # first_fine
        if coarse_on and feature:
            coarse = feature_read(h, page_z[:, :, :completed],
                                  torch.stack(page_c_full[:completed], 2))
        elif coarse_on:
            coarse = coarse_read(h, page_z[:, :, :completed],
                                 torch.stack(page_c_full[:completed], 2))
        else:
            coarse = torch.zeros_like(fine)
        if coarse_on or fine_on:
            out[:, start:end] = fusion(raw_q[:, start:end], local[:, start:end], coarse,
                                       fine, fusion_a, fusion_b, alpha, coarse_on, fine_on,
                                       arith=raw_q.dtype)
    return (out, routes) if return_routes else out


def training_forward_smooth(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, routes,
                            geometry=None, intermediates=None, writer="softmax"):
    """training_forward's function without bf16 rounding, for gradients.

    Same steps as training_forward (local attention per tile, the softmax
    writer, page logsumexps, page softmax, segment weights, h, hv, the
    selected read num / den, the coarse read, the three-branch fusion with
    presence masks), evaluated in the inputs' dtype (fp64 in the tests), with
    every query's selection fixed to `routes` (tile -> ids [B, Q, H, M]): the
    reference's selection has no derivative (tao_stream.py:647-650), so the
    gradient of tao_attention is the gradient of this function at the bf16
    forward's selections. Differentiable by torch autograd. A dict
    `intermediates` receives the fine descriptors "fine_z" [B, H, S, D] and
    the bank "bank" [B, H, S, D, D] (C[d][e]), to take gradients at them.

    writer="regularized_association" keeps the softmax writer's z and takes
    C_f = solve(G + tr(G)/D I, X) with G = U^T U, X = U^T V, U = softmax_D(raw_k)
    of the block (association_writer.py:11-32 without its bf16 casts), and a
    completed page's matrix from the sums of its fines' G and X,
    differentiable through the solves.

    The feature writers (tao_stream.py:56-65, 543-549, 600-662) take
    z_f = log(m_f) with m_f = sum_t U_t, C_f from the solve (feature mass)
    or structured_matrix of the block's statistics (structured Gram), page
    z = log of the summed masses and page C from the summed statistics; a
    query's fine read is the mixture sum_m w_m h C_m with
    w_m = (h . exp z_m) / sum_m' (h . exp z_m') over its selection, and its
    coarse read the same mixture over the completed pages (no denominator).
    """
    if writer in FEATURE_WRITERS:
        return _feature_forward_smooth(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
                                       routes, geometry or Geometry(), writer, intermediates)
    g = geometry or Geometry()
    b, total, heads, d = q.shape
    ft, keep, group = g.fine_tokens, g.local_keep, g.coarse_group
    parts = []
    for start in range(0, total, ft):
        end = min(total, start + ft)
        k0 = max(0, start - keep)
        s = torch.einsum("bqhd,bkhd->bhqk", q[:, start:end], k[:, k0:end]) / math.sqrt(d)
        rows = (end - k0) - (end - start) + torch.arange(end - start)
        allowed = torch.arange(end - k0)[None, :] <= rows[:, None]
        p = torch.softmax(s.masked_fill(~allowed, NEG_INF), -1)
        parts.append(torch.einsum("bhqk,bkhd->bqhd", p, v[:, k0:end]))
    local = torch.cat(parts, 1)
    n_tiles = -(-total // ft)
    lag = keep // ft
    visible_max = max(0, n_tiles - 1 - lag)
    if total <= g.serve_limit or visible_max == 0:
        return local
    zs, cs, grams, crosses = [], [], [], []
    for f in range(visible_max):
        kb, vb = raw_k[:, f * ft:(f + 1) * ft], v[:, f * ft:(f + 1) * ft]
        zs.append(torch.logsumexp(kb, 1))                           # [B, H, D]
        if writer == "regularized_association":
            u = torch.softmax(kb, -1)                               # over channels
            gram = torch.einsum("bthd,bthe->bhde", u, u)
            cross = torch.einsum("bthd,bthe->bhde", u, vb)
            ridge = gram.diagonal(dim1=-2, dim2=-1).sum(-1) / d
            system = gram + ridge[..., None, None] * torch.eye(d, dtype=gram.dtype)
            cs.append(torch.linalg.solve(system, cross))
            grams.append(gram)
            crosses.append(cross)
        else:
            cs.append(torch.einsum("bthd,bthe->bhde", torch.softmax(kb, 1), vb))
    fine_z = torch.stack(zs, 2)
    bank = torch.stack(cs, 2)
    if intermediates is not None:
        intermediates["fine_z"], intermediates["bank"] = fine_z, bank
    full = visible_max // group
    pz_full = [torch.logsumexp(fine_z[:, :, p * group:(p + 1) * group], 2) for p in range(full)]
    pc_full = []
    if not g.coarse_index_only and writer == "regularized_association":
        for p in range(full):
            gram = sum(grams[p * group + i] for i in range(group))
            cross = sum(crosses[p * group + i] for i in range(group))
            ridge = gram.diagonal(dim1=-2, dim2=-1).sum(-1) / d
            system = gram + ridge[..., None, None] * torch.eye(d, dtype=gram.dtype)
            pc_full.append(torch.linalg.solve(system, cross))
    elif not g.coarse_index_only:
        for p in range(full):
            w = torch.exp(fine_z[:, :, p * group:(p + 1) * group] - pz_full[p].unsqueeze(2))
            pc_full.append(torch.einsum("bhsd,bhsde->bhde", w, bank[:, :, p * group:(p + 1) * group]))
    first_coarse = keep + group * ft
    gain = 2.0 * alpha
    outs = [local[:, :min(total, (lag + 1) * ft)]]
    for tile in range(lag + 1, n_tiles):
        start, end = tile * ft, min(total, tile * ft + ft)
        visible = tile - lag
        completed, pending = divmod(visible, group)
        pz = list(pz_full[:completed])
        if pending:
            pz.append(torch.logsumexp(fine_z[:, :, completed * group:visible], 2))
        page_z = torch.stack(pz, 2)                                 # [B, H, P, D]
        pw = torch.softmax(page_z, 2)
        page_of = torch.arange(visible) // group
        sw = torch.exp(fine_z[:, :, :visible] - page_z[:, :, page_of])
        rq = raw_q[:, start:end]
        h = torch.softmax(rq, -1)                                   # [B, Q, H, D]
        hv = h.unsqueeze(3) * pw.unsqueeze(1)                       # [B, Q, H, P, D]
        sel = routes[tile]
        mask = torch.zeros((*sel.shape[:3], visible), dtype=h.dtype)
        mask.scatter_(-1, sel, 1.0)
        a = hv[:, :, :, page_of] * sw.unsqueeze(1) * mask.unsqueeze(-1)   # [B, Q, H, V, D]
        num = torch.einsum("bqhvd,bhvde->bqhe", a, bank[:, :, :visible])
        fine = num / a.sum((-1, -2)).unsqueeze(-1)
        coarse_on = start >= first_coarse and not g.coarse_index_only
        if coarse_on:
            cw = torch.softmax(page_z[:, :, :completed], 2)
            coarse = torch.einsum("bqhd,bhpd,bhpde->bqhe", h, cw,
                                  torch.stack(pc_full[:completed], 2))
        else:
            coarse = torch.zeros_like(fine)
        present = 1 + int(coarse_on)
        scores = []
        for branch in range(3):
            s = fusion_a[..., branch] * rq + fusion_b[..., branch]
            if branch == 0:
                s = s + math.log(present)
            if branch == 1 and not coarse_on:
                s = torch.full_like(s, NEG_INF)
            scores.append(s)
        rho = torch.softmax(torch.stack(scores, -1), -1)
        lo = local[:, start:end]
        outs.append(rho[..., 0] * 2 * lo + rho[..., 1] * gain * coarse + rho[..., 2] * gain * fine)
    return torch.cat(outs, 1)


def _smooth_local(q, k, v, g):
    """Per-tile suffix-causal local attention without rounding (the local
    part of training_forward_smooth)."""
    b, total, heads, d = q.shape
    ft, keep = g.fine_tokens, g.local_keep
    parts = []
    for start in range(0, total, ft):
        end = min(total, start + ft)
        k0 = max(0, start - keep)
        s = torch.einsum("bqhd,bkhd->bhqk", q[:, start:end], k[:, k0:end]) / math.sqrt(d)
        rows = (end - k0) - (end - start) + torch.arange(end - start)
        allowed = torch.arange(end - k0)[None, :] <= rows[:, None]
        p = torch.softmax(s.masked_fill(~allowed, NEG_INF), -1)
        parts.append(torch.einsum("bhqk,bkhd->bqhd", p, v[:, k0:end]))
    return torch.cat(parts, 1)


def _smooth_mixture(h, z, matrices, mask=None):
    """sum_m w_m sum_d h[d] M_m[d][e] with w_m = (h . exp z_m) / sum over the
    (masked) items; h [B, Q, H, D], z [B, H, P, D], matrices [B, H, P, D, D],
    mask [B, Q, H, P] or None (every item)."""
    mass = torch.einsum("bqhd,bhpd->bqhp", h, torch.exp(z))
    if mask is not None:
        mass = mass * mask
    w = mass / mass.sum(-1, keepdim=True)
    return torch.einsum("bqhp,bqhd,bhpde->bqhe", w, h, matrices)


def _feature_forward_smooth(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, routes, g,
                            writer, intermediates):
    """training_forward_smooth for the feature writers (see there)."""
    from . import writers as W
    b, total, heads, d = q.shape
    ft, keep, group = g.fine_tokens, g.local_keep, g.coarse_group
    local = _smooth_local(q, k, v, g)
    n_tiles = -(-total // ft)
    lag = keep // ft
    visible_max = max(0, n_tiles - 1 - lag)
    if total <= g.serve_limit or visible_max == 0:
        return local
    structured = writer == "structured_gram_association"
    zs, cs, firsts, crosses, masses = [], [], [], [], []
    for f in range(visible_max):
        kb, vb = raw_k[:, f * ft:(f + 1) * ft], v[:, f * ft:(f + 1) * ft]
        u = torch.softmax(kb, -1)                                   # over channels
        mass = u.sum(1)                                             # [B, H, D]
        cross = torch.einsum("bthd,bthe->bhde", u, vb)
        if structured:
            first = (u * u).sum(1)
            cs.append(W.structured_matrix(first, cross, mass, ft)[0])
        else:
            first = torch.einsum("bthd,bthe->bhde", u, u)
            ridge = first.diagonal(dim1=-2, dim2=-1).sum(-1) / d
            system = first + ridge[..., None, None] * torch.eye(d, dtype=first.dtype)
            cs.append(torch.linalg.solve(system, cross))
        zs.append(torch.log(mass))
        firsts.append(first)
        crosses.append(cross)
        masses.append(mass)
    fine_z = torch.stack(zs, 2)
    bank = torch.stack(cs, 2)
    if intermediates is not None:
        intermediates["fine_z"], intermediates["bank"] = fine_z, bank
    full = visible_max // group
    pz_full, pc_full = [], []
    for p in range(full):
        idx = range(p * group, (p + 1) * group)
        mass = sum(masses[i] for i in idx)
        pz_full.append(torch.log(mass))
        if g.coarse_index_only:
            continue
        first = sum(firsts[i] for i in idx)
        cross = sum(crosses[i] for i in idx)
        if structured:
            pc_full.append(W.structured_matrix(first, cross, mass, ft * group)[0])
        else:
            ridge = first.diagonal(dim1=-2, dim2=-1).sum(-1) / d
            system = first + ridge[..., None, None] * torch.eye(d, dtype=first.dtype)
            pc_full.append(torch.linalg.solve(system, cross))
    first_coarse = keep + group * ft
    gain = 2.0 * alpha
    outs = [local[:, :min(total, (lag + 1) * ft)]]
    for tile in range(lag + 1, n_tiles):
        start, end = tile * ft, min(total, tile * ft + ft)
        visible = tile - lag
        completed = visible // group
        rq = raw_q[:, start:end]
        h = torch.softmax(rq, -1)
        sel = routes[tile]
        mask = torch.zeros((*sel.shape[:3], visible), dtype=h.dtype)
        mask.scatter_(-1, sel, 1.0)
        fine = _smooth_mixture(h, fine_z[:, :, :visible], bank[:, :, :visible], mask)
        coarse_on = start >= first_coarse and not g.coarse_index_only
        if coarse_on:
            coarse = _smooth_mixture(h, torch.stack(pz_full[:completed], 2),
                                     torch.stack(pc_full[:completed], 2))
        else:
            coarse = torch.zeros_like(fine)
        present = 1 + int(coarse_on)
        scores = []
        for branch in range(3):
            s = fusion_a[..., branch] * rq + fusion_b[..., branch]
            if branch == 0:
                s = s + math.log(present)
            if branch == 1 and not coarse_on:
                s = torch.full_like(s, NEG_INF)
            scores.append(s)
        rho = torch.softmax(torch.stack(scores, -1), -1)
        lo = local[:, start:end]
        outs.append(rho[..., 0] * 2 * lo + rho[..., 1] * gain * coarse + rho[..., 2] * gain * fine)
    return torch.cat(outs, 1)
