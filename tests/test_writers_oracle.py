"""Pins for the non-preset writer oracle (oracle/writers.py), CPU only.

Each check uses a method independent of the restated formula: numpy's LU
solve for the Cholesky path, the dense matrix behind the structured writer's
two Sherman-Morrison steps, invariants of the statistics, brute-force loops
and one-hot channels for the selected numerator.
"""
import pytest
import torch

from oracle import writers as W

BF16 = torch.bfloat16


def kv(n, t, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(n, t, h, d, generator=g) * 2).to(BF16)
    v = torch.randn(n, t, h, d, generator=g).to(BF16)
    return k, v


@pytest.mark.parametrize("d", [8, 64])
def test_association_statistics_invariants(d):
    k, v = kv(2, 256, 3, d, 1)
    gram, cross, mass = W.association_statistics(k, v, with_mass=True)
    u = W.feature_simplex(k)
    assert torch.equal(u, u.to(BF16).double())                  # u is bf16-valued
    assert torch.allclose(gram, gram.transpose(-1, -2))
    assert torch.all(torch.linalg.eigvalsh(gram) > -1e-9)
    trace = gram.diagonal(dim1=-2, dim2=-1).sum(-1)
    assert torch.allclose(trace, (u * u).sum(-1).sum(1), rtol=1e-12)
    # each softmax row sums to 1 before its bf16 rounding (2^-9 per element)
    assert torch.allclose(mass.sum(-1), torch.full_like(mass.sum(-1), 256.0), rtol=4e-3)
    # sum_d cross[d][e] = sum_t (sum_d u[t][d]) v[t][e]
    row = u.sum(-1)                                             # [N, T, H]
    want = torch.einsum("nth,nthe->nhe", row, v.double())
    assert torch.allclose(cross.sum(-2), want, rtol=1e-10, atol=1e-10)
    square, cross2, mass2 = W.structured_statistics(k, v)
    assert torch.equal(cross2, cross) and torch.equal(mass2, mass)
    assert mass.dtype == square.dtype == torch.float32
    assert torch.allclose(square.double(), gram.diagonal(dim1=-2, dim2=-1), rtol=256 * 2 ** -24)


@pytest.mark.parametrize("d", [64, 128])
def test_feature_simplex_and_mass_orders(d):
    """The fp32 orders this build fixes for u and the feature mass, against
    what the reference's arithmetic admits: u within one bf16 ulp of the
    fp64 softmax rounded once (equal almost everywhere: only values whose
    fp32 evaluation lands across a rounding boundary differ); the mass is
    the fp32 left-to-right token sum (numpy's float32 cumsum, an
    independent sequential sum, equals it bit for bit) and lies within
    256 fp32 roundings of the exact sum."""
    import numpy as np
    k, v = kv(2, 256, 3, d, 9)
    u = W.feature_simplex(k)
    exact = torch.softmax(k.double(), -1)
    ref = exact.to(BF16).double()
    ulp = 2.0 ** (torch.floor(torch.log2(exact)) - 7)
    assert ((u - ref).abs() <= ulp).all()
    assert (u != ref).double().mean() < 1e-3
    if d == 128:
        # the group/pair order matters: a plain left-to-right sum over all D
        # channels gives a different u on some rows
        x = k.float()
        e = torch.exp(x.double() - x.amax(-1, keepdim=True).double()).float()
        flat = torch.zeros(e.shape[:-1])
        for j in range(d):
            flat = flat + e[..., j]
        assert not torch.equal((e / flat.unsqueeze(-1)).to(BF16).double(), u)
    mass = W.association_statistics(k, v, with_mass=True)[2]       # [N, H, D]
    ut = u.float().transpose(1, 2).numpy()                         # [N, H, T, D]
    seq = np.cumsum(ut, axis=2, dtype=np.float32)[:, :, -1]
    assert np.array_equal(mass.numpy(), seq)
    exact_mass = u.transpose(1, 2).sum(-2)
    assert ((mass.double() - exact_mass).abs() <= 256 * 2 ** -24 * exact_mass).all()


@pytest.mark.parametrize("d", [8, 64])
def test_association_matrix_against_dense_solve(d):
    k, v = kv(3, 256, 2, d, 2)
    gram, cross = W.association_statistics(k, v)
    solution, c = W.association_matrix(gram, cross)
    system = W.regularised_system(gram)
    # ridge = mean diagonal (a dropped /D or a missing ridge fails here)
    ridge = system.diagonal(dim1=-2, dim2=-1) - gram.diagonal(dim1=-2, dim2=-1)
    assert torch.allclose(ridge, gram.diagonal(dim1=-2, dim2=-1).mean(-1, keepdim=True)
                          .expand_as(ridge))
    dense = W.dense_solve(system, cross)
    assert torch.allclose(solution, dense, rtol=1e-9, atol=1e-9)
    assert torch.allclose(system @ solution, cross, rtol=1e-9, atol=1e-9)
    assert c.dtype == BF16 and torch.equal(c, solution.to(BF16))


def test_chronological_sum_order():
    x = torch.randn(2, 3, 5, 4, 4, dtype=torch.float32)
    total = W.chronological_sum(x)
    want = x[:, :, 0]
    for i in range(1, 5):
        want = want + x[:, :, i]
    assert torch.equal(total, want)
    assert torch.allclose(total, x.double().sum(2).float(), atol=1e-5)


@pytest.mark.parametrize("zero_variance", [False, True])
def test_structured_matrix_against_dense_inverse(zero_variance):
    d, count = 16, 256
    k, v = kv(2, count, 2, d, 3)
    square, cross, mass = W.structured_statistics(k, v)
    if zero_variance:
        # identical tokens: var = 0 exactly, the rank-one var term drops out
        k = k[:, :1].expand(-1, count, -1, -1)
        square, cross, mass = W.structured_statistics(k, v)
        mass = square.sqrt() * count          # force square * count == mass^2
        square = mass * mass / count
    result, c = W.structured_matrix(square, cross, mass, count)
    system = W.structured_system(square, mass, count)
    dense = W.dense_solve(system, cross)
    assert torch.allclose(result, dense, rtol=1e-8, atol=1e-10)
    assert torch.equal(c, result.to(BF16))


def test_feature_read_coefficients_mixture():
    g = torch.Generator().manual_seed(4)
    h = torch.softmax(torch.randn(2, 5, 3, 16, generator=g), -1).to(BF16)
    z = torch.randn(2, 5, 3, 6, 16, generator=g).to(BF16)
    out = W.feature_read_coefficients(h, z)
    mass = (h.double().unsqueeze(-2) * z.double().exp()).sum(-1)
    mixture = mass / mass.sum(-1, keepdim=True)
    assert torch.allclose(mixture.sum(-1), torch.ones_like(mixture.sum(-1)))
    ratio = out.double() / h.double().unsqueeze(-2)
    assert torch.allclose(ratio, mixture.unsqueeze(-1).expand_as(ratio), rtol=8e-3)
    # a broadcast read_z (one row for every query) equals the expanded one
    zb = z[:, :1]
    assert torch.equal(W.feature_read_coefficients(h, zb),
                       W.feature_read_coefficients(h, zb.expand_as(z)))


def test_selected_numerator_brute_force_and_one_hot():
    g = torch.Generator().manual_seed(5)
    b, q, h, m, d, s = 4, 3, 2, 5, 8, 7
    channel = torch.randn(b, q, h, m, d, generator=g).to(BF16)
    ids = torch.randint(0, s, (b, q, h, m), generator=g)
    bank = torch.randn(2, h, s, d, d, generator=g).to(BF16)      # shared by b % 2
    out = W.selected_fine_numerator(channel, ids, bank)
    assert torch.equal(out, W.selected_fine_numerator_loop(channel, ids, bank))
    # one-hot channel picks row d0 of the selected C
    onehot = torch.zeros(b, q, h, 1, d)
    onehot[..., 3] = 1
    pick = W.selected_fine_numerator(onehot.to(BF16), ids[..., :1], bank)
    for bi in range(b):
        for qi in range(q):
            for hi in range(h):
                assert torch.equal(pick[bi, qi, hi], bank[bi % 2, hi, ids[bi, qi, hi, 0], 3])


def test_selected_numerator_backward_brute_force():
    g = torch.Generator().manual_seed(6)
    b, q, h, m, d, s = 2, 3, 2, 4, 8, 5
    channel = torch.randn(b, q, h, m, d, generator=g).to(BF16)
    ids = torch.randint(0, s, (b, q, h, m), generator=g)
    bank = torch.randn(1, h, s, d, d, generator=g).to(BF16)
    grad = torch.randn(b, q, h, d, generator=g).to(BF16)
    dch, dc = W.selected_fine_numerator_backward(channel, ids, bank, grad)
    # autograd of the fp64 contraction gives the same adjoints up to the casts
    ch = channel.double().requires_grad_()
    cb = bank.double().requires_grad_()
    gathered = cb[0][torch.arange(h)[None, None, :, None], ids]
    out = torch.einsum("bqhmd,bqhmde->bqhe", ch, gathered)
    out.backward(grad.double())
    assert torch.allclose(dch.double(), ch.grad, rtol=8e-3, atol=1e-6)
    # per-batch bf16 partials, then a bf16 total: a few bf16 ulps of the largest term
    assert (dc.double() - cb.grad).abs().max() <= 2e-2 * cb.grad.abs().max()
    # a mistake in the shared-bank index (b % BB) or the id routing is O(1)
    assert not torch.allclose(dc.double(), cb.grad.roll(1, 2), atol=0.5)


def test_oracle_stream_regularized_writer_pages_and_pending():
    """OracleStream with the regularized writer: fine C = association_matrix
    of the block's statistics; a completed page's C equals association_matrix
    of the statistics of its 2048 tokens taken at once (the statistics are
    sums over tokens, so the in-order sum of its eight fines' must agree);
    the pending sums restart after a page with page values and keep summing
    index-only; export carries them."""
    from oracle import tao_oracle as O
    g = torch.Generator().manual_seed(7)
    t, h, d = 2900, 2, 8
    xs = [torch.randn(1, t, h, d, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=g) * 0.02
    fb = torch.randn(h, d, 3, generator=g) * 0.02
    for index_only in (False, True):
        s = O.OracleStream(0, O.Geometry(coarse_index_only=index_only),
                           writer="regularized_association")
        pos = 0
        while pos < t:
            w = s.next_chunk(t - pos)
            s.prefill(*(x[:, pos:pos + w] for x in xs), fa, fb, 0.5)
            pos += w
        rk, v = xs[4], xs[2]
        fines = len(s.fine_z)
        assert fines == 8 + 1
        for f in (0, 5, 8):
            blk = slice(f * 256, (f + 1) * 256)
            want = W.association_matrix(*W.association_statistics(rk[:, blk], v[:, blk]))[1]
            assert torch.equal(s.fine_c[f], want)
        page = W.association_statistics(rk[:, :2048], v[:, :2048])
        if index_only:
            assert s.page_c == []
            total = W.association_statistics(rk[:, :fines * 256], v[:, :fines * 256])
            assert torch.allclose(s.pending_gram, total[0], rtol=1e-12, atol=1e-12)
        else:
            want = W.association_matrix(*page)[1]
            assert (s.page_c[0].double() - want.double()).abs().max() <= \
                2 ** -8 * want.double().abs().max()
            last = W.association_statistics(rk[:, 2048:2304], v[:, 2048:2304])
            assert torch.allclose(s.pending_gram, last[0], rtol=1e-12, atol=1e-12)
        snap = s.export()
        assert snap["config"]["fine_writer"] == "regularized_association"
        assert snap["pending_gram"].dtype == torch.float32
        back = O.OracleStream.from_export(snap, 0, O.Geometry(coarse_index_only=index_only))
        assert back.writer == "regularized_association"
        assert torch.equal(back.pending_gram.float(), snap["pending_gram"])


@pytest.mark.parametrize("index_only", [False, True])
def test_regularized_writer_peak_counts_pending_sums(index_only):
    """The pending gram/cross sums enter the peak cache bytes
    (tao_stream.py:953-958, 969-978), in the oracle and in the product's
    closed-form diagnostics. Closed form at B1 H2 D128 for a 768-token
    prefill: the third 256-token chunk seals the first fine; before it the
    peak is 2 x 768 key rows, after it one fine's bytes + the fp32 sums +
    2 x 512 key rows, which is larger:
      before = 2 * 768 * H * D * 2                         = 786432
      after  = (D*D + D) * H * 2 + 2 * H * D * D * 4 + 2 * 512 * H * D * 2
             = 66048 + 262144 + 524288                      = 852480
    Physical counts three key rows, and there the pre-seal figure stays:
      max(3 * 768 * H * D * 2, 66048 + 262144 + 3 * 512 * H * D * 2)
      = max(1179648, 1114624)."""
    from oracle import tao_oracle as O
    from tao_attention import TaoConfig, diagnostics
    h, d, t = 2, 128, 768
    g = torch.Generator().manual_seed(3)
    xs = [torch.randn(1, t, h, d, generator=g).to(BF16) for _ in range(5)]
    fa = torch.zeros(h, d, 3)
    s = O.OracleStream(0, O.Geometry(coarse_index_only=index_only),
                       writer="regularized_association")
    s.prefill(*xs, fa, fa, 0.5)
    assert s.pending_writer_bytes() == 2 * h * d * d * 4
    assert s.diag["peak_logical_cache_bytes"] == 852480
    assert s.diag["peak_physical_cache_tensor_bytes"] == 1179648
    soft = O.OracleStream(0, O.Geometry(coarse_index_only=index_only))
    soft.prefill(*xs, fa, fa, 0.5)
    assert soft.diag["peak_logical_cache_bytes"] == 786432
    cfg = TaoConfig(fine_writer="regularized_association", coarse_index_only=index_only)
    c = diagnostics.counters(cfg, 0, 1, h, d, [("call", 0, t, 0)], t)
    assert (c.peak_logical_cache_bytes, c.peak_physical_cache_tensor_bytes) == (
        s.diag["peak_logical_cache_bytes"], s.diag["peak_physical_cache_tensor_bytes"])


@pytest.mark.parametrize("writer", ["feature_mass_association", "structured_gram_association"])
def test_oracle_stream_feature_writers(writer):
    """OracleStream with a feature writer (tao_stream.py:56-65, 280-305,
    362-367, 463-499) over 17 fines (two completed pages and a pending
    fine), pinned by checks that do not restate it:
    - a fine's z is within half a bf16 ulp of the log of the block's exact
      (fp64) mass, which sums to the block length over the channels;
    - the mass runs: index-only the reference never clears pending_mass
      (:488-497), so page p's z and the pending descriptor are the log of
      the mass of every fine so far; with page values each page's run
      restarts. Each descriptor is within one bf16 ulp of the log of the
      exact mass of its run, equals r(log) of numpy's float32 running sum of
      the fines' masses bit for bit, and lies far (about log 2) from the
      log of the other rule's run, so either rule's mistake fails;
    - the page matrices (non-index-only) are the writer's matrix of each
      page's 2048 tokens' statistics taken at once;
    - export -> import -> 300 more tokens equals the uninterrupted stream;
    - the fine read of a query against one selected fine is r(h @ C): the
      mixture of one matrix is 1;
    - with two fines whose z are equal the read is the plain mean of the
      two matrices' reads (mixture 1/2 each)."""
    import numpy as np
    from oracle import tao_oracle as O
    g = torch.Generator().manual_seed(11)
    t, extra, h, d = 5000, 300, 2, 8
    xs = [torch.randn(1, t + extra, h, d, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=g) * 0.02
    fb = torch.randn(h, d, 3, generator=g) * 0.02

    def run(s, lo, hi):
        pos, outs = lo, []
        while pos < hi:
            w = s.next_chunk(hi - pos)
            outs.append(s.prefill(*(x[:, pos:pos + w] for x in xs), fa, fb, 0.5))
            pos += w
        return torch.cat(outs, 1)

    def near(z, exact_log):        # within one bf16 ulp of the exact log
        return ((z.double() - exact_log).abs() <= 2 ** -7 * exact_log.abs()).all()

    for index_only in (False, True):
        geo = O.Geometry(coarse_index_only=index_only)
        s = O.OracleStream(0, geo, writer=writer)
        run(s, 0, t)
        rk, v = xs[4], xs[2]
        assert len(s.fine_z) == 17 and len(s.page_z) == 2
        masses, exact = [], []
        for f in range(17):
            blk = slice(f * 256, (f + 1) * 256)
            masses.append(W.association_statistics(rk[:, blk], v[:, blk], with_mass=True)[2])
            exact.append(W.feature_simplex(rk[:, blk]).sum(1))             # fp64 [1, H, D]
            assert torch.allclose(exact[f].sum(-1), torch.full_like(exact[f].sum(-1), 256.0),
                                  rtol=4e-3)
            assert ((s.fine_z[f].double() - exact[f].log()).abs()
                    <= 2 ** -8 * exact[f].log().abs()).all()
        stacked = np.stack([m.numpy() for m in masses])                     # [F, 1, H, D]

        def descriptor(first, last):   # r(log) of numpy's float32 running sum
            run_sum = np.cumsum(stacked[first:last + 1], axis=0, dtype=np.float32)[-1]
            return torch.from_numpy(np.log(run_sum.astype(np.float64))).float().to(BF16)

        def exact_log(first, last):
            return sum(exact[first:last + 1]).log()

        desc = s.page_descriptors()                                         # [1, H, 3, D]
        for p, (lo, hi) in enumerate(((0, 7), (8, 15), (16, 16))):
            first = 0 if index_only else lo
            z = s.page_z[p] if p < 2 else desc[:, :, 2]
            assert torch.equal(z, descriptor(first, hi))
            assert near(z, exact_log(first, hi))
            if p:
                other = lo if index_only else 0
                assert (z.double() - exact_log(other, hi)).abs().min() > 0.3
        if index_only:
            assert s.page_c == []
        else:
            for p in range(2):
                tok = slice(p * 2048, (p + 1) * 2048)
                if writer == "structured_gram_association":
                    sq, cross, mass = W.structured_statistics(rk[:, tok], v[:, tok])
                    want = W.structured_matrix(sq, cross, mass, 2048)[1]
                else:
                    want = W.association_matrix(*W.association_statistics(rk[:, tok],
                                                                         v[:, tok]))[1]
                assert (s.page_c[p].double() - want.double()).abs().max() <= \
                    2 ** -7 * want.double().abs().max()
        snap = s.export(config=None)
        assert snap["pending_mass"] is not None and snap["pending_mass"].dtype == torch.float32
        assert (snap["pending_square_mass"] is None) == (writer == "feature_mass_association")
        assert (snap["pending_gram"] is None) == (writer == "structured_gram_association")
        back = O.OracleStream.from_export(snap, 0, geo)
        assert torch.equal(run(back, t, t + extra), run(s, t, t + extra))
        assert all(torch.equal(a, b) for a, b in zip(back.page_z, s.page_z))
        # the mixture read against hand-picked fines
        hq = O.query_weights(xs[3][:, :1])                          # [1, 1, H, D]
        z_all, c_all = torch.stack(s.fine_z, 2), torch.stack(s.fine_c, 2)
        one = O.feature_read(hq, z_all[:, :, 3:4], c_all[:, :, 3:4])
        want = torch.einsum("bqhd,bhde->bqhe", hq.double(), c_all[:, :, 3].double())
        assert torch.equal(one, want.to(BF16))
        pair_z = z_all[:, :, 3:4].expand(-1, -1, 2, -1)
        two = O.feature_read(hq, pair_z, c_all[:, :, 3:5])
        half = (O.rnd(hq.double() * 0.5, BF16).double())
        want = torch.einsum("bqhd,bhpde->bqhe", half, c_all[:, :, 3:5].double())
        assert torch.equal(two, want.to(BF16))
