"""Pins the CPU oracle (CPU only).

The reference ships no golden vectors (its only test, tests/gpu_sanity.py,
asserts finiteness and self-consistency), so each oracle function is checked
against something independent of its own formula: closed forms and the
survey's derived table, torch's own bf16 ops (the reference's third-party
arithmetic), fp64 brute force, stable-sort brute force and streaming
invariants. Each check is chosen so a plausible restatement mistake (wrong
softmax axis, dropped rounding, off-by-one window, unstable tie order) fails.
"""
import math

import pytest
import torch

from oracle import numerics as N
from oracle import tao_oracle as O

BF16 = torch.bfloat16


# --------------------------------------------------------------- closed forms
def test_budget_matches_ceil_sqrt_definition():
    g = O.Geometry()
    for n in range(0, 5000):
        if n == 0:
            assert g.budget(0) == 0
            continue
        root = math.ceil(math.sqrt(2 * n) - 1e-12)
        while root * root < 2 * n:
            root += 1
        while (root - 1) * (root - 1) >= 2 * n:
            root -= 1
        assert g.budget(n) == min(n, root + 2)
    assert (g.budget(510), g.budget(62), g.budget(126)) == (34, 14, 18)


@pytest.mark.parametrize("context,expect", [
    (2048, (0, 6, 6)), (8192, (3, 30, 10)), (16384, (4, 38, 14)),
    (32768, (5, 46, 18)), (131072, (9, 78, 34)),
])
def test_routed_counts_table(context, expect):
    """Derived counts table: pages/pending after `context` tokens."""
    g = O.Geometry()
    fines = (context - g.serve_limit) // g.fine_tokens + 1
    completed, pending = divmod(fines, g.coarse_group)
    assert g.routed_counts(completed, pending) == expect


def test_turn_schedule():
    g = O.Geometry()
    turns0 = [p for p in range(700, 900) if g.is_turn(p, 0)]
    assert turns0 == [768, 792, 816, 840, 864, 888]
    turns5 = [p for p in range(700, 900) if g.is_turn(p, 5)]
    assert turns5 == [768, 778, 802, 826, 850, 874, 898]
    for layer in (0, 3):
        for p in range(700, 1000):
            nt = g.next_turn(p, layer)
            assert nt > p and g.is_turn(nt, layer) or nt == 768 + 2 * layer
            assert not any(g.is_turn(x, layer) and x >= 768 + 2 * layer
                           for x in range(p + 1, nt))


# ------------------------------------------------------- torch's own bf16 ops
@pytest.mark.parametrize("shape,dim", [((4, 32, 8, 128), 2), ((3, 16, 6, 64), 2),
                                       ((2, 8, 64, 128), 2), ((5, 7, 3), 1)])
def test_logsumexp_is_torch_bf16_composite(shape, dim):
    torch.manual_seed(1)
    x = (torch.randn(shape) * 3).to(BF16)
    assert torch.equal(N.logsumexp(x, dim), torch.logsumexp(x, dim=dim))


def test_logsumexp_single_rounding_would_fail():
    """The composite's intermediate roundings are observable (not a no-op)."""
    torch.manual_seed(2)
    x = (torch.randn(4, 32, 8, 128) * 3).to(BF16)
    single = torch.logsumexp(x.float(), dim=2).to(BF16)
    assert (single != N.logsumexp(x, 2)).float().mean() > 0.01


@pytest.mark.parametrize("shape,dim", [((64, 32, 128), -1), ((2, 32, 64, 128), 2),
                                       ((2, 8, 9, 64), 2)])
def test_softmax_matches_torch_bf16_within_one_ulp(shape, dim):
    torch.manual_seed(3)
    x = (torch.randn(shape) * 2).to(BF16)
    a, b = torch.softmax(x, dim=dim), N.softmax(x, dim)
    diff = (N.bf16_bits(a) - N.bf16_bits(b)).abs()
    assert diff.max() <= 1
    assert (diff > 0).float().mean() < 1e-3


def test_fold_sum_is_butterfly_order():
    torch.manual_seed(4)
    for n in (1, 3, 8, 64, 100, 128, 200):
        x = torch.randn(5, n) * torch.logspace(-3, 3, n)
        got = N.fold_sum(x, -1)
        for row in range(5):
            vals = [torch.tensor(v, dtype=torch.float32) for v in x[row].tolist()]
            width = 1
            while width < n:
                width *= 2
            vals += [torch.tensor(0.0)] * (width - n)
            while len(vals) > 1:
                half = len(vals) // 2
                vals = [vals[i] + vals[i + half] for i in range(half)]
            assert got[row].item() == vals[0].item()


# ------------------------------------------------------------ fp64 brute force
def test_writer_against_fp64():
    torch.manual_seed(5)
    k = torch.randn(1, 256, 3, 32).to(BF16)
    v = torch.randn(1, 256, 3, 32).to(BF16)
    z, c = O.seal_softmax(k, v)
    kd, vd = k.double(), v.double()
    z_ref = torch.logsumexp(kd, dim=1)                       # over tokens
    p_ref = torch.softmax(kd, dim=1)
    c_ref = torch.einsum("bthd,bthe->bhde", p_ref, vd)
    torch.testing.assert_close(z.double(), z_ref, atol=2e-2, rtol=1e-2)
    torch.testing.assert_close(c.double(), c_ref, atol=2e-3, rtol=2e-2)
    # Softmax over channels instead of tokens must not pass.
    p_bad = torch.softmax(kd, dim=-1)
    c_bad = torch.einsum("bthd,bthe->bhde", p_bad, vd)
    assert (c.double() - c_bad).abs().max() > 1e-2


def test_read_against_fp64():
    torch.manual_seed(6)
    b, q, h, p, s, d, m = 1, 3, 2, 3, 20, 16, 5
    hv = (torch.rand(b, q, h, p, d) / d).to(BF16)
    sw = torch.rand(b, h, s, d).to(BF16)
    bank = torch.randn(b, h, s, d, d).to(BF16)
    sel = torch.stack([torch.randperm(s)[:m] for _ in range(h)])[None]
    fine, ch = O.selected_read(hv, sw, sel, bank, group=8)
    ref = torch.zeros(b, q, h, d, dtype=torch.float64)
    for hh in range(h):
        num = torch.zeros(q, d, dtype=torch.float64)
        den = torch.zeros(q, 1, dtype=torch.float64)
        for slot in range(m):
            fid = sel[0, hh, slot].item()
            weight = hv[0, :, hh, fid // 8].double() * sw[0, hh, fid].double()
            num += weight @ bank[0, hh, fid].double()
            den += weight.sum(-1, keepdim=True)
        ref[0, :, hh] = num / den
    torch.testing.assert_close(fine.double(), ref, atol=2e-2, rtol=2e-2)


def test_local_attention_against_sdpa_modes():
    torch.manual_seed(7)
    import torch.nn.functional as F
    for tq, tk in ((8, 8), (1, 20), (5, 20)):
        q = torch.randn(1, tq, 2, 16).to(BF16)
        k = torch.randn(1, tk, 2, 16).to(BF16)
        v = torch.randn(1, tk, 2, 16).to(BF16)
        got = O.local_attention(q, k, v)
        qt, kt, vt = (t.double().transpose(1, 2) for t in (q, k, v))
        if tq == tk:
            ref = F.scaled_dot_product_attention(qt, kt, vt, is_causal=True)
        elif tq == 1:
            ref = F.scaled_dot_product_attention(qt, kt, vt)
        else:
            rows = tk - tq + torch.arange(tq)
            mask = torch.arange(tk)[None, :] <= rows[:, None]
            ref = F.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask)
        torch.testing.assert_close(got.double(), ref.transpose(1, 2), atol=1e-2, rtol=1e-2)


def test_fusion_closed_form():
    """Coarse absent: out = 2*rho0*local + 2*alpha*rho2*fine, rho = softmax(s0, s2)."""
    torch.manual_seed(8)
    h, d = 2, 16
    raw_q = torch.randn(1, 4, h, d).to(BF16)
    local = torch.randn(1, 4, h, d).to(BF16)
    fine = torch.randn(1, 4, h, d).to(BF16)
    a = torch.randn(h, d, 3) * 0.5
    bias = torch.randn(h, d, 3) * 0.5
    alpha = 0.5
    out = O.fusion(raw_q, local, torch.zeros_like(local), fine, a, bias, alpha, False, True)
    s0 = a[..., 0].double() * raw_q.double() + bias[..., 0].double()
    s2 = a[..., 2].double() * raw_q.double() + bias[..., 2].double()
    r0 = torch.sigmoid(s0 - s2)
    ref = 2 * r0 * local.double() + 2 * alpha * (1 - r0) * fine.double()
    torch.testing.assert_close(out.double(), ref, atol=5e-2, rtol=3e-2)


def _three_branch_closed_form(raw_q, local, coarse, fine, a, bias, alpha, local_bias):
    """fp64: rho = softmax(s0 + local_bias, s1, s2), s_i = a_i q + b_i;
    out = 2 rho0 local + 2 alpha (rho1 coarse + rho2 fine)."""
    q = raw_q.double()
    s = [a[..., i].double() * q + bias[..., i].double() for i in range(3)]
    s[0] = s[0] + local_bias
    rho = torch.softmax(torch.stack(s, -1), -1)
    return (2 * rho[..., 0] * local.double()
            + 2 * alpha * (rho[..., 1] * coarse.double() + rho[..., 2] * fine.double()))


def test_fusion_three_branch_closed_form():
    """Coarse and fine present (fusion_pointwise.py:10-47, 50-92; the local
    score carries log(#present history branches) = log 2): the oracle equals
    the closed form within bf16 rounding, and the same closed form without
    the local bias, or with the coarse and fine operands swapped, is far from
    it, so a dropped bias or a transposed branch would fail this test."""
    torch.manual_seed(9)
    h, d, t = 3, 32, 6
    raw_q = torch.randn(1, t, h, d).to(BF16)
    local, coarse, fine = (torch.randn(1, t, h, d).to(BF16) for _ in range(3))
    a = torch.randn(h, d, 3) * 0.5
    bias = torch.randn(h, d, 3) * 0.5
    alpha = 0.75
    out = O.fusion(raw_q, local, coarse, fine, a, bias, alpha, True, True).double()
    # The oracle rounds a and b to bf16 before use (fusion_pointwise.py:103-108).
    a16, b16 = a.to(BF16).float(), bias.to(BF16).float()
    ref = _three_branch_closed_form(raw_q, local, coarse, fine, a16, b16, alpha, math.log(2))
    torch.testing.assert_close(out, ref, atol=5e-2, rtol=3e-2)
    no_bias = _three_branch_closed_form(raw_q, local, coarse, fine, a16, b16, alpha, 0.0)
    swapped = _three_branch_closed_form(raw_q, local, fine, coarse, a16, b16, alpha, math.log(2))
    for wrong in (no_bias, swapped):
        assert (out - wrong).abs().max().item() > 0.2
    # Coarse present, fine absent: one history branch, so the local bias is
    # log 1 = 0 (fusion_pointwise.py:99-100) and the fine branch drops out.
    only_coarse = O.fusion(raw_q, local, coarse, fine, a, bias, alpha, True, False).double()
    s = [a16[..., i].double() * raw_q.double() + b16[..., i].double() for i in (0, 1)]
    rho = torch.softmax(torch.stack(s, -1), -1)
    ref1 = 2 * rho[..., 0] * local.double() + 2 * alpha * rho[..., 1] * coarse.double()
    torch.testing.assert_close(only_coarse, ref1, atol=5e-2, rtol=3e-2)


def test_normalisation_properties():
    """Segment weights of a page sum to one (pz = logsumexp of the page's z);
    page weights sum to one over pages, h over channels; hv is the rounded
    product of the matching page row. A sign flip in z - pz, a softmax over
    the wrong axis or a mis-broadcast page index fails one of these."""
    torch.manual_seed(11)
    b, h, pages, d = 1, 3, 4, 16
    z = (torch.randn(b, h, pages * 8, d) * 2).to(BF16)
    pz = torch.stack([O.page_summary(z[:, :, 8 * p:8 * p + 8]) for p in range(pages)], 2)
    sw = O.segment_weights(z, pz.repeat_interleave(8, dim=2))
    sums = sw.double().reshape(b, h, pages, 8, d).sum(3)
    torch.testing.assert_close(sums, torch.ones_like(sums), atol=3e-2, rtol=0)
    assert (sw.double() <= 1.0 + 1e-2).all()
    exact = torch.logsumexp(z.double().reshape(b, h, pages, 8, d), 3)
    torch.testing.assert_close(pz.double(), exact, atol=3e-2, rtol=1e-2)
    pw = O.page_weights(pz)
    torch.testing.assert_close(pw.double().sum(2), torch.ones(b, h, d, dtype=torch.float64),
                               atol=3e-2, rtol=0)
    raw_q = torch.randn(b, 2, h, d).to(BF16)
    hq = O.query_weights(raw_q)
    torch.testing.assert_close(hq.double().sum(-1), torch.ones(b, 2, h, dtype=torch.float64),
                               atol=3e-2, rtol=0)
    hv = O.page_values(hq, pw)
    assert hv.shape == (b, 2, h, pages, d)
    for qi in range(2):
        for p in range(pages):
            ref = (hq[0, qi].double() * pw[0, :, p].double())
            torch.testing.assert_close(hv[0, qi, :, p].double(), ref, atol=0, rtol=2 ** -8)


# ------------------------------------------------------------------- routing
def _sorted_topk(scores, count):
    order = sorted(range(len(scores)), key=lambda i: (-scores[i], i))
    return order[:count]


def test_route_against_stable_sort_brute_force():
    torch.manual_seed(9)
    g = O.Geometry()
    completed, pending = 9, 5
    b, h, d = 1, 3, 16
    pages = completed + 1
    s = completed * 8 + pending
    # Quantised values create many exact bf16 ties.
    hv = (torch.randint(1, 4, (b, h, pages, d)).float() / 64).to(BF16)
    sw = (torch.randint(1, 4, (b, h, s, d)).float() / 4).to(BF16)
    chosen, selected, info = O.route(hv, sw, completed, pending, g)
    coarse, eligible, m = g.routed_counts(completed, pending)
    assert chosen.shape[-1] == coarse and selected.shape[-1] == m
    for hh in range(h):
        pm = [N.rnd(N.fold_sum(hv[0, hh, p], -1)).float().item() for p in range(completed)]
        want_pages = sorted(_sorted_topk(pm, coarse))
        assert chosen[0, hh].tolist() == want_pages
        cands = [p * 8 + j for p in want_pages for j in range(8)]
        cands += [completed * 8 + j for j in range(pending)]
        scores = []
        for fid in cands:
            page = min(fid // 8, completed)
            ch = N.rnd(hv[0, hh, page].float() * sw[0, hh, fid].float())
            scores.append(N.rnd(N.fold_sum(ch, -1)).float().item())
        want = [cands[i] for i in _sorted_topk(scores, m)]
        assert selected[0, hh].tolist() == want
        assert len(set(want)) == m


# ---------------------------------------------------------------- streaming
def _stream_inputs(tokens, heads=2, width=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(1, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    return xs, fa, fb


def _run(stream, xs, fa, fb, splits, alpha=0.5):
    q, k, v, rq, rk = xs
    outs = []
    start = 0
    for width in splits:
        sl = slice(start, start + width)
        if width == 1:
            outs.append(stream.decode(q[:, sl], k[:, sl], v[:, sl], rq[:, sl], rk[:, sl],
                                      fa, fb, alpha, position=start))
        else:
            outs.append(stream.prefill(q[:, sl], k[:, sl], v[:, sl], rq[:, sl], rk[:, sl],
                                       fa, fb, alpha, position=start))
        start += width
    return torch.cat(outs, 1)


def test_stream_local_only_before_first_fine():
    xs, fa, fb = _stream_inputs(800)
    s = O.OracleStream(0)
    out = _run(s, xs, fa, fb, [800])
    q, k, v = xs[:3]
    for end in (256, 512, 768):
        start = end - 256
        lo = max(0, end - 768)
        ref = O.local_attention(q[:, start:end], k[:, lo:end], v[:, lo:end])
        assert torch.equal(out[:, start:end], ref)
    assert not torch.equal(out[:, 768:800], O.local_attention(q[:, 768:800], k[:, 256:800], v[:, 256:800]))


def test_stream_chunking_invariance_and_decode_equals_prefill():
    xs, fa, fb = _stream_inputs(1400, seed=1)
    whole = _run(O.OracleStream(1), xs, fa, fb, [1400])
    calls = _run(O.OracleStream(1), xs, fa, fb, [256, 256, 300, 100, 400, 88])
    torch.testing.assert_close(whole, calls, atol=0, rtol=0)
    mixed = _run(O.OracleStream(1), xs, fa, fb, [1300] + [1] * 100)
    torch.testing.assert_close(whole, mixed, atol=0, rtol=0)


def test_stream_export_import_continues_identically():
    xs, fa, fb = _stream_inputs(1500, seed=2)
    a = O.OracleStream(0)
    _run(a, xs, fa, fb, [1200])
    snap = a.export()
    b = O.OracleStream.from_export(snap, 0)
    rest = [t[:, 1200:] for t in xs]
    q, k, v, rq, rk = rest
    out_a = a.prefill(q, k, v, rq, rk, fa, fb, 0.5)
    out_b = b.prefill(q, k, v, rq, rk, fa, fb, 0.5)
    assert torch.equal(out_a, out_b)
    assert a.position == b.position == 1500


def test_banks_depend_only_on_raw_k_and_v():
    xs, fa, fb = _stream_inputs(1300, seed=3)
    ys = [t.clone() for t in xs]
    ys[0] = torch.randn_like(ys[0].float()).to(BF16)   # q
    ys[3] = torch.randn_like(ys[3].float()).to(BF16)   # raw_q
    a, b = O.OracleStream(0), O.OracleStream(0)
    _run(a, xs, fa, fb, [1300])
    _run(b, ys, fa, fb, [1300])
    assert len(a.fine_z) == len(b.fine_z) == 3
    for x, y in zip(a.fine_z + a.fine_c, b.fine_z + b.fine_c):
        assert torch.equal(x, y)


def test_stream_rejects_contract_violations():
    xs, fa, fb = _stream_inputs(10)
    s = O.OracleStream(0)
    q, k, v, rq, rk = xs
    with pytest.raises(ValueError):
        s.prefill(q, k, v, rq, rk, fa, fb, 0.5, position=3)
    with pytest.raises(ValueError):
        s.decode(q[:, :2], k[:, :2], v[:, :2], rq[:, :2], rk[:, :2], fa, fb, 0.5)


# ------------------------------------------------------------ coarse branch
def test_page_coarse_matrix_against_fp64():
    """page_C[d, e] = sum_s exp(z_s[d] - pz[d]) C_s[d, e] (tao_stream.py:486-499).
    Weights index the row d of each C_s: weighting columns instead, or using
    exp(pz - z), fails the fp64 comparison; identical fine matrices must come
    back unchanged because a page's segment weights sum to one per row."""
    torch.manual_seed(12)
    b, h, d = 1, 2, 16
    z = (torch.randn(b, h, 8, d) * 2).to(BF16)
    c = torch.randn(b, h, 8, d, d).to(BF16)
    pz = O.page_summary(z)
    pc = O.page_coarse_matrix(z, pz, c)
    w = torch.exp(z.double() - torch.logsumexp(z.double(), 2, keepdim=True))
    ref = torch.einsum("bhsd,bhsde->bhde", w, c.double())
    torch.testing.assert_close(pc.double(), ref, atol=3e-2, rtol=2e-2)
    bad = torch.einsum("bhse,bhsde->bhde", w, c.double())
    assert (pc.double() - bad).abs().max() > 5e-2
    same = c[:, :, :1].expand(b, h, 8, d, d).contiguous()
    pc_same = O.page_coarse_matrix(z, pz, same)
    torch.testing.assert_close(pc_same.double(), same[:, :, 0].double(), atol=0, rtol=3e-2)


def test_coarse_read_against_fp64():
    """coarse = sum_p softmax_p(page_z)[d] h[d] page_C_p[d, :] (tao_stream.py:299-305);
    one completed page reduces to h @ page_C."""
    torch.manual_seed(13)
    b, t, h, p, d = 1, 3, 2, 4, 16
    pz = (torch.randn(b, h, p, d) * 2).to(BF16)
    pc = torch.randn(b, h, p, d, d).to(BF16)
    hq = O.query_weights(torch.randn(b, t, h, d).to(BF16))
    out = O.coarse_read(hq, pz, pc)
    w = torch.softmax(pz.double(), 2)                              # [b,h,p,d]
    ref = torch.einsum("bthd,bhpd,bhpde->bthe", hq.double(), w, pc.double())
    torch.testing.assert_close(out.double(), ref, atol=2e-2, rtol=2e-2)
    wrong_axis = torch.softmax(pz.double(), 3)
    bad = torch.einsum("bthd,bhpd,bhpde->bthe", hq.double(), wrong_axis, pc.double())
    assert (out.double() - bad).abs().max() > 2e-2
    one = O.coarse_read(hq, pz[:, :, :1], pc[:, :, :1])
    torch.testing.assert_close(one.double(), torch.einsum("bthd,bhde->bthe", hq.double(),
                                                          pc[:, :, 0].double()),
                               atol=1e-2, rtol=2e-2)


def test_stream_coarse_branch_switches_on_at_first_coarse():
    """DEFAULT_CONFIG geometry (coarse_index_only=False): identical to the
    index-only stream until the first page completes (first_coarse = 2560),
    different afterwards; chunking and decode still give identical outputs."""
    xs, fa, fb = _stream_inputs(2700, seed=4)
    values = O.Geometry(coarse_index_only=False)
    with_values = _run(O.OracleStream(0, values), xs, fa, fb, [2700])
    index_only = _run(O.OracleStream(0), xs, fa, fb, [2700])
    assert torch.equal(with_values[:, :2560], index_only[:, :2560])
    assert not torch.equal(with_values[:, 2560:], index_only[:, 2560:])
    calls = _run(O.OracleStream(0, values), xs, fa, fb, [1000, 1500, 60, 1] + [1] * 139)
    torch.testing.assert_close(with_values, calls, atol=0, rtol=0)
    s = O.OracleStream(0, values)
    _run(s, xs, fa, fb, [2700])
    snap = s.export()
    assert len(snap["pages"]) == 1 and snap["pages"][0][1] is not None
    assert snap["pages"][0][1].shape == (1, 2, 16, 16)


@pytest.mark.parametrize("coarse,memo", [(False, True), (True, False), (False, False)])
def test_diagnostics_counters_match_reference_accounting(coarse, memo):
    """The product's closed-form diagnostics (tao_attention.diagnostics, from a
    call log) equal the oracle's restatement of the reference's per-chunk and
    per-segment accounting (tao_stream.py:162-230, 919-986) over random mixes
    of prefill calls, one-token runs and releases."""
    import random
    from tao_attention import TaoConfig, diagnostics
    cfg = TaoConfig(coarse_index_only=not coarse, q1_page_normalization_memo=memo)
    layer, heads, width, total = 1, 2, 16, 2900
    rng = random.Random(3 + 2 * coarse + memo)
    xs, fa, fb = _stream_inputs(total, heads=heads, width=width, seed=5)
    s = O.OracleStream(layer, O.Geometry.from_config(cfg))
    log, pos = [], 0
    while pos < total:
        route = 0 if s.route_ids is None else s.route_ids[1].shape[-1]
        if rng.random() < 0.5:
            n = min(rng.randint(1, 40), total - pos)
            for i in range(n):
                if not (log and log[-1][0] == "run" and log[-1][1] + log[-1][2] == pos + i):
                    log.append(["run", pos + i, 0, route if i == 0 else
                                s.route_ids[1].shape[-1]])
                log[-1][2] += 1
                q, k, v, rq, rk = (t[:, pos + i:pos + i + 1] for t in xs)
                s.prefill(q, k, v, rq, rk, fa, fb, 0.5)
        else:
            n = min(rng.randint(2, 700), total - pos)
            log.append(["call", pos, n, route])
            q, k, v, rq, rk = (t[:, pos:pos + n] for t in xs)
            s.prefill(q, k, v, rq, rk, fa, fb, 0.5)
        pos += n
        if rng.random() < 0.1:
            s.release_execution()
            log.append(["release", pos, 0, 0])
    c = diagnostics.counters(cfg, layer, 1, heads, width, [tuple(e) for e in log], pos)
    for key, value in s.diag.items():
        assert getattr(c, key) == value, key
    assert c.memo == s.memo
    assert s.diag["fine_matrix_contractions"] > 0 and s.diag["route_query_heads"] > 0
    if coarse:
        assert s.diag["coarse_matrix_contractions"] > 0


# ------------------------------------------------------------- full sequence

def _brute_local(q, k, v, tile=256, keep=512):
    """Per-query fp64 softmax over keys [max(0, tile_start - keep), i]."""
    b, t, heads, d = q.shape
    out = torch.empty(b, t, heads, d, dtype=torch.float64)
    for i in range(t):
        lo = max(0, (i // tile) * tile - keep)
        s = torch.einsum("bhd,bkhd->bhk", q[:, i].double(), k[:, lo:i + 1].double()) / math.sqrt(d)
        out[:, i] = torch.einsum("bhk,bkhd->bhd", torch.softmax(s, -1), v[:, lo:i + 1].double())
    return out.to(q.dtype)


def test_training_forward_short_prefix_is_exact_local_attention():
    """Below first_fine the full-sequence read is the tiled local attention
    (read_training :682-688, _local_training_corrected_4k ragged fallback)."""
    xs, fa, fb = _stream_inputs(700, seed=8)
    q, k, v, rq, rk = xs
    out = O.training_forward(q, k, v, rq, rk, fa, fb, 0.5, O.Geometry())
    torch.testing.assert_close(out, _brute_local(q, k, v), atol=1e-2, rtol=0)
    xs, fa, fb = _stream_inputs(1100, seed=9)
    q, k, v, rq, rk = xs
    out = O.training_forward(q, k, v, rq, rk, fa, fb, 0.5, O.Geometry())
    torch.testing.assert_close(out[:, :768], _brute_local(q, k, v)[:, :768], atol=1e-2, rtol=0)


@pytest.mark.parametrize("index_only,tokens", [(True, 2100), (False, 2900)])
def test_training_forward_is_the_stream_refreshing_at_every_query(index_only, tokens):
    """read_training(route_interval=1) equals the streaming read with a route
    refresh at every query: the stream's local ring equals the tile windows,
    its epoch at a chunk equals tile - 2 visible fines, and routing, read,
    coarse read and fusion presence are the same functions. A stream with
    route_period=1 therefore gives identical bits; with the default period
    only the first refresh position agrees."""
    xs, fa, fb = _stream_inputs(tokens, seed=7)
    q, k, v, rq, rk = xs
    g = O.Geometry(coarse_index_only=index_only)
    out, routes = O.training_forward(q, k, v, rq, rk, fa, fb, 0.5, g, return_routes=True)
    every = O.Geometry(coarse_index_only=index_only, route_period=1)
    assert torch.equal(out, _run(O.OracleStream(0, every), xs, fa, fb, [tokens]))
    streamed = _run(O.OracleStream(0, g), xs, fa, fb, [tokens])
    assert torch.equal(out[:, :769], streamed[:, :769])
    assert not torch.equal(out[:, 769:], streamed[:, 769:])
    # route invariants: M unique ids among the tile's eligible candidates
    for tile, sel in routes.items():
        visible = tile - 2
        completed, pending = divmod(visible, 8)
        _, _, m = g.routed_counts(completed, pending)
        assert sel.shape[-1] == m
        assert int(sel.min()) >= 0 and int(sel.max()) < visible
        srt = sel.sort(-1).values
        assert bool((srt[..., 1:] != srt[..., :-1]).all())


@pytest.mark.parametrize("index_only,tokens", [(True, 1400), (False, 2700)])
def test_training_smooth_forward_is_the_rounded_forward(index_only, tokens):
    """The fp64 function the gradients are taken of equals the bf16 forward to
    bf16 tolerance at the forward's own selections, and autograd through it
    reaches every operand (tao_attention's differentiable inputs,
    tests/gpu_sanity.py:28-34 of the reference)."""
    xs, fa, fb = _stream_inputs(tokens, seed=11)
    g = O.Geometry(coarse_index_only=index_only)
    out, routes = O.training_forward(*xs, fa, fb, 0.5, g, return_routes=True)
    leaves = [x.double().requires_grad_(True) for x in xs]
    fa64, fb64 = fa.double().requires_grad_(True), fb.double().requires_grad_(True)
    smooth = O.training_forward_smooth(*leaves, fa64, fb64, 0.5, routes, g)
    torch.testing.assert_close(smooth.float(), out.float(), atol=3e-2, rtol=3e-2)
    grads = torch.autograd.grad(smooth.square().sum(), leaves + [fa64, fb64])
    for gr in grads:
        assert torch.isfinite(gr).all() and gr.abs().sum() > 0


@pytest.mark.parametrize("writer", ["feature_mass_association", "structured_gram_association"])
@pytest.mark.parametrize("index_only,tokens", [(True, 1400), (False, 2700)])
def test_training_smooth_forward_feature_writers(writer, index_only, tokens):
    """The feature writers' fp64 function (log-mass z, solve / structured
    matrices, mixture reads) equals their bf16 forward to bf16 tolerance at
    its selections (with the coarse mixture past first_coarse = 2560), and
    autograd reaches every operand; the softmax writer's smooth function at
    the same selections does not match (so the writer branch is taken)."""
    xs, fa, fb = _stream_inputs(tokens, seed=13)
    g = O.Geometry(coarse_index_only=index_only)
    out, routes = O.training_forward(*xs, fa, fb, 0.5, g, return_routes=True, writer=writer)
    leaves = [x.double().requires_grad_(True) for x in xs]
    fa64, fb64 = fa.double().requires_grad_(True), fb.double().requires_grad_(True)
    smooth = O.training_forward_smooth(*leaves, fa64, fb64, 0.5, routes, g, writer=writer)
    torch.testing.assert_close(smooth.float(), out.float(), atol=3e-2, rtol=3e-2)
    soft = O.training_forward_smooth(*(x.double() for x in xs), fa.double(), fb.double(), 0.5,
                                     routes, g)
    tail = slice(768, None)
    assert (soft[:, tail] - smooth[:, tail].detach()).abs().max() > 0.1
    grads = torch.autograd.grad(smooth.square().sum(), leaves + [fa64, fb64])
    for gr in grads:
        assert torch.isfinite(gr).all() and gr.abs().sum() > 0


@pytest.mark.parametrize("tokens,index_only", [(1300, True), (2900, False)])
def test_training_forward_fp32_matches_fp64_at_its_routes(tokens, index_only):
    """The fp32 semantics of tao_attention (every rounding point at fp32):
    training_forward on fp32 operands agrees with the independent fp64
    evaluation training_forward_smooth at the fp32 forward's own routes to
    fp32 accuracy (1e-5), pages, coarse read and both fusion biases
    included; and the bf16 and fp32 runs of the same inputs differ by bf16
    rounding only. A dropped term, a wrong index or a bf16 rounding left in
    the fp32 path would exceed 1e-5."""
    g = O.Geometry(coarse_index_only=index_only)
    gen = torch.Generator().manual_seed(5)
    h, d = 2, 16
    xs = [torch.randn(1, tokens, h, d, generator=gen) for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=gen) * 0.02
    fb = torch.randn(h, d, 3, generator=gen) * 0.02
    out, routes = O.training_forward(*xs, fa, fb, 0.5, g, return_routes=True)
    assert out.dtype == torch.float32
    smooth = O.training_forward_smooth(*(x.double() for x in xs), fa.double(), fb.double(), 0.5,
                                       routes, g)
    assert (out.double() - smooth).abs().max() < 1e-5
    low = O.training_forward(*(x.to(torch.bfloat16) for x in xs), fa, fb, 0.5, g)
    assert (low.double() - smooth).abs().max() > 1e-3
