"""Non-preset writers and the channel-given selected read on the GPU against
the CPU oracle (oracle/writers.py), through the package mirrors of the
reference modules (association_writer, structured_writer, indirect_fine),
which call the C ABI.

Bar: statistics within fp32 summation-order differences plus the rare bf16
flip of a feature value u (tolerances written per check); matrices and read
outputs within 2e-2 (bf16); the chronological sum bit-exact.
"""
import pytest
import torch

from oracle import writers as W
from tao_attention.association_writer import (association_matrix, association_statistics,
                                               chronological_sum, feature_read_coefficients)
from tao_attention.indirect_fine import selected_fine_numerator
from tao_attention.structured_writer import structured_matrix, structured_statistics

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def kv(n, t, h, d, seed):
    g = torch.Generator().manual_seed(seed)
    k = (torch.randn(n, t, h, d, generator=g) * 2).to(BF16)
    v = torch.randn(n, t, h, d, generator=g).to(BF16)
    return k, v


def close(got, want, rel):
    """|got - want| <= rel * max|want| elementwise."""
    got, want = got.double().cpu(), want.double().cpu()
    scale = want.abs().max().item() or 1.0
    err = (got - want).abs().max().item()
    assert err <= rel * scale, (err, scale)


@pytest.mark.parametrize("d,t", [(64, 256), (128, 256), (64, 100)])
def test_association_statistics(device, d, t):
    k, v = kv(3, t, 2, d, 11)
    gram, cross, mass = association_statistics(k.to(device), v.to(device), with_mass=True)
    wg, wc, wm = W.association_statistics(k, v, with_mass=True)
    assert gram.shape == (3, 2, d, d) and mass.shape == (3, 2, d)
    close(gram, wg, 2e-3)
    close(cross, wc, 2e-3)
    close(mass, wm, 2e-3)
    g2, c2 = association_statistics(k.to(device), v.to(device))
    assert torch.equal(g2, gram) and torch.equal(c2, cross)


def test_statistics_strided_inputs(device):
    """Token blocks cut from a longer [B, T, H, D] stream by a view (the
    reference's seal reshapes k[:, :S*256] into blocks)."""
    k, v = kv(1, 1024, 3, 64, 12)
    kd, vd = k.to(device), v.to(device)
    blocks_k = kd[:, :768].reshape(3, 256, 3, 64)
    blocks_v = vd[:, :768].reshape(3, 256, 3, 64)
    gram, cross = association_statistics(blocks_k[:, :, 1:], blocks_v[:, :, 1:])
    wg, wc = W.association_statistics(k[:, :768].reshape(3, 256, 3, 64)[:, :, 1:],
                                      v[:, :768].reshape(3, 256, 3, 64)[:, :, 1:])
    close(gram, wg, 2e-3)
    close(cross, wc, 2e-3)


@pytest.mark.parametrize("d", [64, 128])
def test_association_matrix(device, d):
    k, v = kv(4, 256, 2, d, 13)
    gram, cross = association_statistics(k.to(device), v.to(device))
    c = association_matrix(gram, cross)
    _, want = W.association_matrix(gram.cpu().double(), cross.cpu().double())
    assert c.dtype == BF16 and c.shape == gram.shape
    close(c, want, 2e-2)
    torch.testing.assert_close(c.double().cpu(), want.double(), atol=2e-2, rtol=2e-2)
    # the unchecked solve is the same arithmetic
    assert torch.equal(association_matrix(gram, cross, unchecked=True), c)


def test_association_matrix_checked_mode_raises(device):
    gram = -torch.eye(64, device=device).expand(2, 64, 64).contiguous()
    cross = torch.ones(2, 64, 64, device=device)
    with pytest.raises(torch.linalg.LinAlgError):
        association_matrix(gram, cross)


@pytest.mark.parametrize("d", [64, 128])
def test_structured_writer(device, d):
    k, v = kv(3, 256, 2, d, 14)
    square, cross, mass = structured_statistics(k.to(device), v.to(device))
    ws, wc, wm = W.structured_statistics(k, v)
    close(square, ws, 2e-3)
    close(cross, wc, 2e-3)
    close(mass, wm, 2e-3)
    c = structured_matrix(square, cross, mass, 256)
    _, want = W.structured_matrix(square.cpu(), cross.cpu(), mass.cpu(), 256)
    torch.testing.assert_close(c.double().cpu(), want.double(), atol=2e-2, rtol=2e-2)
    # page statistics: eight fines' statistics summed in order equal the
    # statistics of the 2048-token page (fp32 order), and give its matrix
    kp, vp = kv(8, 256, 2, d, 15)
    sq8, cr8, ms8 = structured_statistics(kp.to(device), vp.to(device))
    page_sq = chronological_sum(sq8)                          # [8, H, D]: fine axis -3
    page_ms = chronological_sum(ms8)
    page_cr = chronological_sum(cr8.transpose(0, 1))          # [H, 8, D, D]
    wsq, wcr, wms = W.structured_statistics(kp.reshape(1, 2048, 2, d), vp.reshape(1, 2048, 2, d))
    close(page_sq, wsq[0], 2e-3)
    close(page_cr, wcr[0], 2e-3)
    close(page_ms, wms[0], 2e-3)
    page = structured_matrix(page_sq, page_cr, page_ms, 2048)
    _, want_page = W.structured_matrix(page_sq.cpu(), page_cr.cpu(), page_ms.cpu(), 2048)
    torch.testing.assert_close(page.double().cpu(), want_page.double(), atol=2e-2, rtol=2e-2)


def test_chronological_sum_exact(device):
    g = torch.Generator().manual_seed(15)
    x = torch.randn(2, 3, 9, 64, 64, generator=g).to(device)
    got = chronological_sum(x)
    want = x[:, :, 0].clone()
    for i in range(1, 9):
        want = want + x[:, :, i]
    assert torch.equal(got, want)


@pytest.mark.parametrize("d", [64, 128])
def test_feature_read_coefficients(device, d):
    g = torch.Generator().manual_seed(16)
    h = torch.softmax(torch.randn(2, 7, 3, d, generator=g), -1).to(BF16)
    z = (torch.randn(2, 7, 3, 5, d, generator=g) - 5).to(BF16)
    got = feature_read_coefficients(h.to(device), z.to(device))
    want = W.feature_read_coefficients(h, z)
    torch.testing.assert_close(got.double().cpu(), want.double(), atol=1e-5, rtol=1.6e-2)
    zb = z[:, :1]                                        # broadcast over tokens
    got_b = feature_read_coefficients(h.to(device), zb.to(device))
    torch.testing.assert_close(got_b.double().cpu(),
                               W.feature_read_coefficients(h, zb).double(),
                               atol=1e-5, rtol=1.6e-2)


def selected_inputs(b, q, h, m, d, s, bank_b, seed, duplicates=False):
    g = torch.Generator().manual_seed(seed)
    channel = (torch.randn(b, q, h, m, d, generator=g) * 0.1).to(BF16)
    ids = torch.stack([torch.randperm(s, generator=g)[:m] for _ in range(b * q * h)])
    ids = ids.reshape(b, q, h, m)
    if duplicates:
        ids[:, ::3, :, 1] = ids[:, ::3, :, 0]
    bank = torch.randn(bank_b, h, s, d, d, generator=g).to(BF16)
    return channel, ids, bank


@pytest.mark.parametrize("d,q,bank_b,dup", [(64, 300, 1, False), (128, 70, 2, False),
                                            (64, 100, 2, True)])
def test_selected_numerator_forward(device, d, q, bank_b, dup):
    channel, ids, bank = selected_inputs(2, q, 2, 6, d, 37, bank_b, 17, dup)
    with torch.no_grad():
        got = selected_fine_numerator(channel.to(device), ids.to(device), bank.to(device))
    want = W.selected_fine_numerator(channel, ids, bank)
    torch.testing.assert_close(got.double().cpu(), want.double(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("d,bank_b", [(64, 1), (128, 2)])
def test_selected_numerator_backward(device, d, bank_b):
    channel, ids, bank = selected_inputs(2, 90, 2, 5, d, 21, bank_b, 18)
    g = torch.Generator().manual_seed(19)
    grad = torch.randn(2, 90, 2, d, generator=g).to(BF16)
    ch = channel.to(device).requires_grad_()
    bk = bank.to(device).requires_grad_()
    out = selected_fine_numerator(ch, ids.to(device), bk)
    out.backward(grad.to(device))
    want_ch, want_c = W.selected_fine_numerator_backward(channel, ids, bank, grad)
    torch.testing.assert_close(ch.grad.double().cpu(), want_ch.double(), atol=2e-2, rtol=2e-2)
    close(bk.grad, want_c, 2e-2)


def _bitmask_sets(qsel):
    words = qsel.cpu().to(torch.int64) & 0xFFFFFFFF
    bits = (words.unsqueeze(-1) >> torch.arange(32)) & 1
    return bits.reshape(*words.shape[:3], -1).bool()


@pytest.mark.parametrize("tokens,heads,width,index_only,seed,batch", [
    (2100, 2, 64, True, 51, 1), (2900, 2, 128, False, 52, 1), (2700, 2, 64, False, 53, 2)])
def test_full_sequence_regularized_writer(device, tokens, heads, width, index_only, seed, batch):
    """tao_attention with fine_writer="regularized_association": the softmax
    writer's z and routes (bit-exact), association value matrices for fines
    and completed pages, outputs within the bf16 tolerance of the oracle."""
    from oracle import tao_oracle as O
    from tao_attention import TaoConfig, tao_attention, training
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(batch, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    cfg = TaoConfig(fine_writer="regularized_association", coarse_index_only=index_only)
    q, k, v, rq, rk = (x.to(device) for x in xs)
    out, qsel = training.forward(q, k, v, rq, rk, fa.to(device), fb.to(device), 0.5, cfg,
                                 return_routes=True)
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True, writer="regularized_association")
    got = _bitmask_sets(qsel)
    for tile, sel in routes.items():
        s = tile * 256
        part = got[:, s:s + sel.shape[1]]
        want = torch.zeros_like(part)
        want.scatter_(-1, sel, True)
        assert torch.equal(part, want), f"selected sets of tile {tile}"
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    # the softmax writer's outputs differ once history is read
    soft = training.forward(q, k, v, rq, rk, fa.to(device), fb.to(device), 0.5,
                            TaoConfig(coarse_index_only=index_only))
    assert not torch.equal(soft[:, 768:], out[:, 768:])
    api = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.to(device),
                        fusion_b=fb.to(device), alpha=0.5, config=cfg)
    assert torch.equal(api, out)
    # gradients are checked against the oracle in test_gpu_parity.py


@pytest.mark.parametrize("index_only,width,batch", [(False, 64, 1), (True, 128, 1),
                                                   (False, 64, 2)])
def test_stream_regularized_writer(device, index_only, width, batch):
    """Streaming prefill and decode with fine_writer="regularized_association":
    seals inside a prefill call and in the decode driver (the step at 2559
    seals the 8th fine and completes page 0), the association fine and page
    matrices, the pending statistics, route ids bit-exact, outputs within the
    bf16 tolerance of the oracle; export -> import continues identically."""
    from oracle import tao_oracle as O
    from tao_attention import (StreamCache, TaoConfig, new_state, tao_attention_decode,
                               tao_attention_prefill)
    heads, tokens = 2, 2826
    g = torch.Generator().manual_seed(61 + width + batch)
    xs = [torch.randn(batch, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    cfg = TaoConfig(fine_writer="regularized_association", coarse_index_only=index_only)
    geo = O.Geometry.from_config(cfg)
    splits = [2540] + [1] * 30 + [250] + [1] * 5
    d = [x.to(device) for x in xs]
    state = new_state(0, cfg)
    ora = O.OracleStream(0, geo, writer="regularized_association")
    outs, refs, start = [], [], 0
    for w in splits:
        sl = slice(start, start + w)
        fn = tao_attention_decode if w == 1 else tao_attention_prefill
        out, state = fn(*(x[:, sl] for x in d[:3]), raw_q=d[3][:, sl], raw_k=d[4][:, sl],
                        fusion_a=fa.to(device), fusion_b=fb.to(device), alpha=0.5,
                        state=state, position=state.get_pos())
        outs.append(out.cpu())
        refs.append(ora.prefill(*(x[:, sl] for x in xs), fa, fb, 0.5))
        start += w
    torch.testing.assert_close(torch.cat(outs, 1).float(), torch.cat(refs, 1).float(),
                               atol=2e-2, rtol=2e-2)
    snap, osnap = state.export(), ora.export(config=cfg.export())
    assert len(snap["pending_z"]) == 1 and len(snap["pages"]) == 1
    assert torch.equal(snap["route_ids"][1].cpu(), osnap["route_ids"][1])
    torch.testing.assert_close(snap["packed_fine_c"].cpu().float(),
                               osnap["packed_fine_c"].float(), atol=2e-2, rtol=2e-2)
    pc, opc = snap["pages"][0][1], osnap["pages"][0][1]
    assert (pc is None) == index_only and (opc is None) == index_only
    if pc is not None:
        torch.testing.assert_close(pc.cpu().float(), opc.float(), atol=2e-2, rtol=2e-2)
    for key in ("pending_gram", "pending_cross"):
        got, want = snap[key], osnap[key]
        assert got is not None and got.dtype == torch.float32
        close(got, want, 1e-3)
    diag = state.bytes()
    assert diag["pending_writer_bytes"] == ora.pending_writer_bytes() == \
        2 * batch * heads * width * width * 4
    assert diag["pending_gram_cross_bytes"] == diag["pending_writer_bytes"]
    assert diag["pending_cross_bytes"] == diag["pending_writer_bytes"] // 2
    assert diag["logical_retained_bytes"] == (diag["history_bytes"] + diag["pending_writer_bytes"]
                                              + diag["logical_local_bf16_kv_bytes"])
    for key in ("peak_logical_cache_bytes", "peak_physical_cache_tensor_bytes"):
        assert diag[key] == ora.diag[key], key
    restored = StreamCache.from_export(snap)
    tok = [x[:, tokens - 1:tokens] for x in d]
    nxt = []
    for s in (state, restored):
        out, _ = tao_attention_decode(*tok[:3], raw_q=tok[3], raw_k=tok[4],
                                      fusion_a=fa.to(device), fusion_b=fb.to(device),
                                      alpha=0.5, state=s, position=s.get_pos())
        nxt.append(out)
    assert torch.equal(nxt[0], nxt[1])


@pytest.mark.parametrize("writer,width,index_only,long", [
    ("feature_mass_association", 64, True, True), ("feature_mass_association", 128, True, True),
    ("structured_gram_association", 128, True, True),
    ("structured_gram_association", 64, True, False),
    ("feature_mass_association", 128, False, False),
    ("structured_gram_association", 64, False, True)])
def test_stream_feature_writers(device, writer, width, index_only, long):
    """Streaming prefill and decode with the feature writers: z = r(log mass),
    page and pending descriptors r(log) of the run's summed mass (index-only
    the run never restarts, tao_stream.py:488-497; with page values it
    restarts at each page), decode through route refreshes (the step at 2559
    seals the 8th fine and completes page 0; the long cases go on to two
    completed pages and two pending fines at 5125 and decode through three
    more refreshes). Bit-exact against the oracle: every route after every
    call, the fine, page and pending descriptors, and the exported pending
    mass (the feature simplex and the fp32 mass sums follow the oracle's
    fixed orders). Within the bf16 tolerance: the fine and page matrices and
    the outputs. Export -> import (this build's snapshot and the oracle's,
    in the reference schema) continues identically."""
    from oracle import tao_oracle as O
    from tao_attention import (StreamCache, TaoConfig, new_state, tao_attention_decode,
                               tao_attention_prefill)
    heads, batch = 2, 1
    # without index_only the tokens after 2816 read page 0's matrix (the
    # mixture over completed pages)
    splits = [2540] + [1] * 30 + [250] + [1] * 5
    if long:
        splits += [2000, 300] + [1] * 75
    elif not index_only:
        splits += [300, 1, 1]
    tokens = sum(splits) + 4
    g = torch.Generator().manual_seed(83 + width)
    xs = [torch.randn(batch, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    cfg = TaoConfig(fine_writer=writer, coarse_index_only=index_only)
    geo = O.Geometry.from_config(cfg)
    d = [x.to(device) for x in xs]
    state = new_state(0, cfg)
    ora = O.OracleStream(0, geo, writer=writer)

    def step(st, sl):
        fn = tao_attention_decode if sl.stop - sl.start == 1 else tao_attention_prefill
        return fn(*(x[:, sl] for x in d[:3]), raw_q=d[3][:, sl], raw_k=d[4][:, sl],
                  fusion_a=fa.to(device), fusion_b=fb.to(device), alpha=0.5,
                  state=st, position=st.get_pos())

    outs, refs, start = [], [], 0
    for w in splits:
        sl = slice(start, start + w)
        print(f"{writer} D{width}: tokens [{start}, {start + w})", flush=True)
        out, state = step(state, sl)
        outs.append(out.cpu())
        refs.append(ora.prefill(*(x[:, sl] for x in xs), fa, fb, 0.5))
        start += w
        if ora.route_ids is not None:
            snap = state.export()
            assert torch.equal(snap["route_ids"][1].cpu(), ora.route_ids[1]), start
            assert torch.equal(snap["route_ids"][0].cpu(), ora.route_ids[0]), start
    torch.testing.assert_close(torch.cat(outs, 1).float(), torch.cat(refs, 1).float(),
                               atol=2e-2, rtol=2e-2)
    snap = state.export()
    fines = len(ora.fine_z)
    completed, pending = divmod(fines, 8)
    assert len(snap["pending_z"]) == pending and len(snap["pages"]) == completed
    assert completed == (2 if long else 1) and pending >= 1
    for i in range(completed):
        pz, pc, fz = snap["pages"][i]
        assert torch.equal(pz.cpu(), ora.page_z[i]), f"page {i} descriptor"
        assert torch.equal(fz.cpu(), torch.stack(ora.fine_z[8 * i:8 * i + 8], 2))
        assert (pc is None) == index_only
        if pc is not None:
            torch.testing.assert_close(pc.cpu().float(), ora.page_c[i].float(),
                                       atol=2e-2, rtol=2e-2)
    for j, z in enumerate(snap["pending_z"]):
        assert torch.equal(z.cpu(), ora.fine_z[8 * completed + j])
    assert torch.equal(state._dev.page_z[:, :, completed].cpu(),
                       ora.page_descriptors()[:, :, completed]), "pending descriptor"
    assert torch.equal(snap["pending_mass"].cpu(), ora.pending_mass)
    osnap = ora.export(config=cfg.export())
    for key in ("pending_gram", "pending_cross", "pending_square_mass"):
        got, want = snap[key], osnap[key]
        assert (got is None) == (want is None), key
        if got is not None:
            assert got.dtype == torch.float32
            close(got, want, 1e-3)
    packed = snap["packed_fine_c"].cpu().float()
    want = torch.stack(ora.fine_c, 2).float()
    torch.testing.assert_close(packed, want, atol=2e-2, rtol=2e-2)
    diag = state.bytes()
    assert diag["pending_writer_bytes"] == ora.pending_writer_bytes()
    assert diag["pending_feature_mass_bytes"] == batch * heads * width * 4
    assert diag["pending_square_mass_bytes"] == (
        batch * heads * width * 4 if writer == "structured_gram_association" else 0)
    # export -> import, of this build's snapshot and of the oracle's
    restored = StreamCache.from_export(snap)
    imported = StreamCache.from_export(osnap)
    tail = slice(start, start + 4)
    want = ora.prefill(*(x[:, tail] for x in xs), fa, fb, 0.5)
    got = []
    for st in (state, restored, imported):
        o, st = step(st, slice(start, start + 3))
        o2, st = step(st, slice(start + 3, start + 4))
        got.append(torch.cat((o, o2), 1))
        assert torch.equal(st.export()["route_ids"][1].cpu(), ora.route_ids[1])
    assert torch.equal(got[0], got[1])
    torch.testing.assert_close(got[2].cpu().float(), want.float(), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("writer,width,tokens,batch,index_only", [
    ("feature_mass_association", 64, 2900, 1, True),
    ("structured_gram_association", 128, 2900, 2, True),
    ("feature_mass_association", 128, 1300, 1, True),
    ("feature_mass_association", 128, 3100, 1, False),
    ("structured_gram_association", 64, 3100, 2, False)])
def test_full_sequence_feature_writers(device, writer, width, tokens, batch, index_only):
    """tao_attention with the feature writers (index-only, forward): every
    query's selected set bit-exact against the oracle's per-query routing
    over log-mass descriptors, outputs within the bf16 tolerance of its
    numerator-only mixture read (their gradients are checked in
    test_gpu_parity.py::test_full_sequence_backward_feature_writers)."""
    from oracle import tao_oracle as O
    from tao_attention import TaoConfig, tao_attention, training
    heads = 2
    g = torch.Generator().manual_seed(97 + width + batch)
    xs = [torch.randn(batch, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    cfg = TaoConfig(fine_writer=writer, coarse_index_only=index_only)
    q, k, v, rq, rk = (x.to(device) for x in xs)
    out, qsel = training.forward(q, k, v, rq, rk, fa.to(device), fb.to(device), 0.5, cfg,
                                 return_routes=True)
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True, writer=writer)
    assert routes, "the call must read history"
    got = _bitmask_sets(qsel)
    for tile, sel in routes.items():
        s = tile * 256
        part = got[:, s:s + sel.shape[1]]
        want = torch.zeros_like(part)
        want.scatter_(-1, sel, True)
        assert torch.equal(part, want), f"selected sets of tile {tile}"
    torch.testing.assert_close(out.cpu().float(), ref.float(), atol=2e-2, rtol=2e-2)
    api = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.to(device),
                        fusion_b=fb.to(device), alpha=0.5, config=cfg)
    assert torch.equal(api, out)
