"""HIP kernels vs the CPU oracle on the same seeded inputs (MI355X only).

Bar: routed ids and every bf16 descriptor feeding routing (fine z, page z)
bit-exact; head outputs and fine matrices within 2e-2 abs/rel (bf16).
Every test calls the product through its public API, which calls the C ABI.
"""
import pytest
import torch

from oracle import tao_oracle as O
from tao_attention import StreamCache, new_state, tao_attention_decode, tao_attention_prefill
from tao_attention.flash_attention import flash_attn_func
from tao_attention.presets import index_only_page_memo

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
TOL = dict(atol=2e-2, rtol=2e-2)


def inputs(tokens, heads, width, seed, unit_raw_k=False):
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(1, tokens, heads, width, generator=g) for _ in range(5)]
    if unit_raw_k:
        xs[4] = xs[4] / xs[4].norm(dim=-1, keepdim=True)
    xs = [x.to(BF16) for x in xs]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    return xs, fa, fb


def to_dev(xs, device):
    return [x.to(device) for x in xs]


def run_hip(state, xs, fa, fb, splits, alpha=0.5):
    q, k, v, rq, rk = xs
    outs, start = [], 0
    for width in splits:
        sl = slice(start, start + width)
        fn = tao_attention_decode if width == 1 else tao_attention_prefill
        out, state = fn(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl], raw_k=rk[:, sl],
                        fusion_a=fa, fusion_b=fb, alpha=alpha, state=state,
                        position=state.get_pos())
        outs.append(out.clone())
        start += width
    return torch.cat(outs, 1)


def run_oracle(layer, xs, fa, fb, splits, alpha=0.5, geometry=None):
    s = O.OracleStream(layer, geometry)
    q, k, v, rq, rk = xs
    outs, start = [], 0
    for width in splits:
        sl = slice(start, start + width)
        outs.append(s.prefill(q[:, sl], k[:, sl], v[:, sl], rq[:, sl], rk[:, sl], fa, fb, alpha))
        start += width
    return s, torch.cat(outs, 1)


def compare_snapshots(hip, ora):
    assert hip["position"] == ora["position"]
    assert hip["state_version"] == ora["state_version"]
    assert len(hip["pages"]) == len(ora["pages"])
    for (pz, pc, fz), (opz, opc, ofz) in zip(hip["pages"], ora["pages"]):
        assert torch.equal(pz.cpu(), opz), "page descriptor"
        assert torch.equal(fz.cpu(), ofz), "fine z"
        assert (pc is None) == (opc is None), "page value matrix presence"
        if opc is not None:
            torch.testing.assert_close(pc.cpu().float(), opc.float(), **TOL)
    for z, oz in zip(hip["pending_z"], ora["pending_z"]):
        assert torch.equal(z.cpu(), oz), "pending fine z"
    if ora["packed_fine_c"] is not None:
        torch.testing.assert_close(hip["packed_fine_c"].cpu().float(),
                                   ora["packed_fine_c"].float(), **TOL)
    if ora["route_ids"] is not None:
        assert torch.equal(hip["route_ids"][1].cpu(), ora["route_ids"][1]), "selected ids"
        assert torch.equal(hip["route_ids"][0].cpu(), ora["route_ids"][0]), "chosen pages"
    for a, b in zip(hip["local"], ora["local"]):
        assert torch.equal(a.cpu(), b)


def compare_diagnostics(state, ora):
    """StreamCache.bytes() counters == the oracle's restated accounting."""
    got = state.bytes()
    for key, value in ora.diag.items():
        assert got[key] == value, key
    assert got["fine_seal_events"] == ora.fine_seal_events
    assert got["route_refreshes_per_layer"] == [ora.route_refreshes]


@pytest.mark.parametrize("width", [64, 128])
@pytest.mark.parametrize("tq,tk", [(200, 200), (1, 700), (256, 768), (77, 333)])
def test_local_attention_plugin(device, width, tq, tk):
    g = torch.Generator().manual_seed(tq * 1000 + tk)
    q, k, v = (torch.randn(1, n, 4, width, generator=g).to(BF16) for n in (tq, tk, tk))
    print(f"local attention width={width} tq={tq} tk={tk}", flush=True)
    got = flash_attn_func(q.to(device), k.to(device), v.to(device)).cpu()
    ref = O.local_attention(q, k, v)
    torch.testing.assert_close(got.float(), ref.float(), **TOL)


@pytest.mark.parametrize("heads,width", [(4, 64), (2, 128)])
def test_prefill_matches_oracle(device, heads, width):
    xs, fa, fb = inputs(2100, heads, width, seed=11)
    print(f"prefill heads={heads} width={width}", flush=True)
    state = new_state(0, index_only_page_memo())
    out = run_hip(state, to_dev(xs, device), fa.to(device), fb.to(device), [2100])
    ora, ref = run_oracle(0, xs, fa, fb, [2100])
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())


def test_decode_matches_oracle_across_seal_and_refresh(device):
    heads, width = 4, 128
    xs, fa, fb = inputs(1330, heads, width, seed=12)
    splits = [1200] + [1] * 130          # seals at position 1279, refreshes every 24
    print("decode across seal", flush=True)
    state = new_state(3, index_only_page_memo())
    out = run_hip(state, to_dev(xs, device), fa.to(device), fb.to(device), splits)
    ora, ref = run_oracle(3, xs, fa, fb, splits,
                          geometry=O.Geometry.from_config(index_only_page_memo()))
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())
    compare_diagnostics(state, ora)


@pytest.mark.parametrize("heads,width", [(4, 128), (2, 64)])
def test_fused_refresh_fold_equals_two_launches(device, monkeypatch, heads, width):
    """The route refresh and its fold as one launch give the same route ids
    and the same outputs, bit for bit, as the route kernel followed by the
    fold kernel, through refreshes with completed pages (coarse selection)
    and a seal."""
    xs, fa, fb = inputs(4700, heads, width, seed=17, unit_raw_k=True)
    d = to_dev(xs, device)
    fa_d, fb_d = fa.to(device), fb.to(device)
    splits = [4600] + [1] * 100          # 4 refreshes and the seal at position 4607
    print(f"fused refresh+fold H{heads} D{width}", flush=True)
    runs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("TAO_REFRESH_FOLD", mode)
        state = new_state(2, index_only_page_memo(graph=False))
        out = run_hip(state, d, fa_d, fb_d, splits)
        runs[mode] = (out, state.export())
    assert torch.equal(runs["0"][0], runs["1"][0])
    for a, b in zip(runs["0"][1]["route_ids"], runs["1"][1]["route_ids"]):
        assert torch.equal(a, b)
    assert runs["1"][1]["route_ids"][0].numel() > 0, "coarse selection must be active"
    ora, ref = run_oracle(2, xs, fa, fb, splits,
                          geometry=O.Geometry.from_config(index_only_page_memo()))
    torch.testing.assert_close(runs["1"][0].cpu().float(), ref.float(), **TOL)
    compare_snapshots(runs["1"][1], ora.export())


def _assert_same_export(a, b):
    if isinstance(a, dict):
        assert a.keys() == b.keys()
        for key in a:
            _assert_same_export(a[key], b[key])
    elif isinstance(a, (list, tuple)):
        assert len(a) == len(b)
        for x, y in zip(a, b):
            _assert_same_export(x, y)
    elif isinstance(a, torch.Tensor):
        assert torch.equal(a, b)
    else:
        assert a == b


@pytest.mark.parametrize("heads,width,tokens", [(4, 128, 3000), (2, 64, 1300)])
def test_prompt_attention_before_the_state_equals_in_plan(device, monkeypatch, heads, width,
                                                          tokens):
    """A new state's first prefill starts its local attention before the
    state's buffers exist (tao_prompt_attention); its outputs, later decode
    steps and exported state equal, bit for bit, those of the local attention
    run inside tao_prefill."""
    xs, fa, fb = inputs(tokens, heads, width, seed=19)
    d = to_dev(xs, device)
    fa_d, fb_d = fa.to(device), fb.to(device)
    splits = [tokens - 24] + [1] * 24
    print(f"prompt attention H{heads} D{width} T{tokens}", flush=True)
    runs = {}
    for mode in ("0", "1"):
        monkeypatch.setenv("TAO_EARLY_LOCAL", mode)
        state = new_state(1, index_only_page_memo(graph=False))
        out = run_hip(state, d, fa_d, fb_d, splits)
        runs[mode] = (out, state.export())
    assert torch.equal(runs["0"][0], runs["1"][0])
    _assert_same_export(runs["0"][1], runs["1"][1])


def test_chunked_prefill_and_page_routing(device):
    """Arbitrary chunking plus completed pages (coarse selection active)."""
    heads, width = 2, 64
    xs, fa, fb = inputs(4700, heads, width, seed=13, unit_raw_k=True)
    splits = [1000, 256, 700, 2000, 1] + [1] * 30 + [713]
    print("chunked prefill with pages", flush=True)
    state = new_state(1, index_only_page_memo())
    out = run_hip(state, to_dev(xs, device), fa.to(device), fb.to(device), splits)
    ora, ref = run_oracle(1, xs, fa, fb, splits,
                          geometry=O.Geometry.from_config(index_only_page_memo()))
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())
    compare_diagnostics(state, ora)


def test_graph_equals_eager_bitwise(device):
    heads, width = 4, 128
    xs, fa, fb = inputs(1100, heads, width, seed=14)
    d = to_dev(xs, device)
    splits = [1000] + [1] * 100
    print("graph vs eager", flush=True)
    eager = run_hip(new_state(0, index_only_page_memo(graph=False)), d, fa.to(device),
                    fb.to(device), splits)
    graph_state = new_state(0, index_only_page_memo(graph=True))
    graph = run_hip(graph_state, d, fa.to(device), fb.to(device), splits)
    assert torch.equal(eager, graph)
    assert graph_state.history_region.counts["replays"] > 0
    graph_state.release_execution()


def test_export_import_reset_gpu_sanity(device):
    """tests/gpu_sanity.py invariants: cursor, export/import equality, reset."""
    heads, width = 6, 128
    xs, _, _ = inputs(1089, heads, width, seed=42)
    d = to_dev(xs, device)
    a = torch.zeros(heads, width, 3, device=device)
    b = torch.zeros_like(a)
    print("gpu sanity", flush=True)
    for graph in (False, True):
        state = new_state(0, index_only_page_memo(graph=graph))
        q, k, v, rq, rk = d
        for start in range(0, 1024, 256):
            sl = slice(start, start + 256)
            _, state = tao_attention_prefill(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                             raw_k=rk[:, sl], fusion_a=a, fusion_b=b, alpha=0.1,
                                             state=state, position=state.get_pos())
        for i in range(1024, 1088):
            sl = slice(i, i + 1)
            out, state = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                              raw_k=rk[:, sl], fusion_a=a, fusion_b=b, alpha=0.1,
                                              state=state, position=state.get_pos())
            assert torch.isfinite(out).all()
        assert state.get_pos() == 1088
        restored = StreamCache.from_export(state.export())
        sl = slice(1088, 1089)
        left, state = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                           raw_k=rk[:, sl], fusion_a=a, fusion_b=b, alpha=0.1,
                                           state=state, position=state.get_pos())
        right, restored = tao_attention_decode(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl],
                                               raw_k=rk[:, sl], fusion_a=a, fusion_b=b,
                                               alpha=0.1, state=restored,
                                               position=restored.get_pos())
        assert torch.equal(left, right)
        state.reset()
        assert state.get_pos() == 0 and restored.get_pos() == 1089
        state.release_execution()
        restored.release_execution()


def test_contract_errors(device):
    xs, fa, fb = inputs(4, 2, 64, seed=0)
    q, k, v, rq, rk = to_dev(xs, device)
    state = new_state(0, index_only_page_memo())
    with pytest.raises(ValueError):
        tao_attention_prefill(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.to(device),
                              fusion_b=fb.to(device), alpha=0.5, state=state, position=1)
    with pytest.raises(ValueError):
        tao_attention_decode(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.to(device),
                             fusion_b=fb.to(device), alpha=0.5, state=state, position=0)


@pytest.mark.parametrize("dtypes", [(torch.float16, torch.float16),
                                    (torch.float32, torch.bfloat16)])
def test_fusion_parameters_updated_in_place(device, dtypes):
    """fusion_a / fusion_b of fp16 or of mixed dtypes, updated in place between
    calls (an optimizer step): each call must use the values the tensors hold
    at that call, as the reference's per-call cast does (operator.py:23-24).
    Compared bitwise with fresh fp32 copies (fp16 and bf16 widen exactly)."""
    heads, width = 2, 64
    xs, fa, fb = inputs(1000, heads, width, seed=23)
    d = to_dev(xs, device)
    fa_live, fb_live = fa.to(device, dtypes[0]), fb.to(device, dtypes[1])
    print(f"fusion parameters in place {dtypes}", flush=True)
    live = new_state(0, index_only_page_memo())
    fresh = new_state(0, index_only_page_memo())
    for st in (live, fresh):
        run_hip(st, [x[:, :990] for x in d], fa_live.float(), fb_live.float(), [990])
    for step in range(990, 1000):
        tok = [x[:, step:step + 1] for x in d]
        want = run_hip(fresh, tok, fa_live.float(), fb_live.float(), [1])
        got = run_hip(live, tok, fa_live, fb_live, [1])
        assert torch.equal(got, want), step
        with torch.no_grad():
            fa_live.mul_(1.5)
            fb_live.add_(0.25)


def test_ingest_state_equals_prefill_state(device):
    """Writer-only state construction (bench state builder) == real prefill."""
    heads, width = 4, 128
    xs, fa, fb = inputs(3000, heads, width, seed=15)
    d = to_dev(xs, device)
    print("ingest vs prefill", flush=True)
    a = new_state(2, index_only_page_memo())
    run_hip(a, d, fa.to(device), fb.to(device), [1500, 1500])
    b = new_state(2, index_only_page_memo())
    b._ingest(*(x[:, :1500] for x in d))
    b._ingest(*(x[:, 1500:] for x in d))
    sa, sb = a.export(), b.export()
    assert sa["position"] == sb["position"] == 3000
    assert torch.equal(sa["packed_fine_c"], sb["packed_fine_c"])
    for (pz, _, fz), (qz, _, gz) in zip(sa["pages"], sb["pages"]):
        assert torch.equal(pz, qz) and torch.equal(fz, gz)
    for x, y in zip(sa["pending_z"], sb["pending_z"]):
        assert torch.equal(x, y)
    assert torch.equal(sa["route_ids"][1], sb["route_ids"][1])
    for x, y in zip(sa["local"], sb["local"]):
        assert torch.equal(x, y)
    # Both continue identically.
    tok = [x[:, 2999:3000].clone() for x in d]
    ya = run_hip(a, [torch.cat([x, x], 1)[:, :1] for x in tok], fa.to(device), fb.to(device), [1])
    yb = run_hip(b, [torch.cat([x, x], 1)[:, :1] for x in tok], fa.to(device), fb.to(device), [1])
    assert torch.equal(ya, yb)


COARSE_VALUES = O.Geometry(coarse_index_only=False)


def test_coarse_value_branch_prefill(device):
    """DEFAULT_CONFIG (coarse values on): page value matrices, the coarse
    pool of one prefill call spanning two page counts (pages complete at
    2560 and 4608) read in the MFMA epilogue, then decode on the folded
    coarse matrix."""
    heads, width = 2, 128
    xs, fa, fb = inputs(4720, heads, width, seed=16)
    splits = [4700] + [1] * 20
    print("coarse value branch prefill", flush=True)
    state = new_state(0)
    out = run_hip(state, to_dev(xs, device), fa.to(device), fb.to(device), splits)
    ora, ref = run_oracle(0, xs, fa, fb, splits, geometry=COARSE_VALUES)
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    snap = state.export()
    assert len(snap["pages"]) == 2
    compare_snapshots(snap, ora.export())
    compare_diagnostics(state, ora)


def test_coarse_value_branch_decode_across_page_completion(device):
    """The decode step at position 4607 seals the 16th fine: the driver builds
    page 1's value matrix and refolds the coarse read for the next steps.
    Export/import (with and without page values) continues identically."""
    heads, width = 2, 64
    xs, fa, fb = inputs(4641, heads, width, seed=17, unit_raw_k=True)
    splits = [4590] + [1] * 50
    print("coarse value branch decode", flush=True)
    d = to_dev(xs, device)
    state = new_state(1)
    out = run_hip(state, d, fa.to(device), fb.to(device), splits)
    ora, ref = run_oracle(1, xs, fa, fb, splits, geometry=COARSE_VALUES)
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    snap = state.export()
    compare_snapshots(snap, ora.export())
    bare = dict(snap, pages=[(pz, None, fz) for pz, _, fz in snap["pages"]])
    restored = StreamCache.from_export(snap)
    rebuilt = StreamCache.from_export(bare)
    tok = [x[:, 4640:4641] for x in d]
    outs = [run_hip(s, tok, fa.to(device), fb.to(device), [1]) for s in (state, restored, rebuilt)]
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])


@pytest.mark.parametrize("op", ["exp", "log"])
def test_exp_log_exhaustive_over_bf16(device, op):
    """The library's bf16(correctly rounded fp32 exp / log), evaluated on all
    65536 bf16 bit patterns (every kernel call site rounds its argument to
    bf16 first), against the oracle's fp64-evaluated functions."""
    import ctypes
    from tao_attention import _hip
    bits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    x = bits.view(BF16)
    xd = x.to(device)
    y = torch.empty_like(xd)
    print(f"numerics self-test {op}", flush=True)
    _hip.check(_hip.lib().tao_numerics_selftest(0 if op == "exp" else 1, xd.data_ptr(),
                                                y.data_ptr(), 65536, _hip.stream_ptr(xd.device)))
    got = y.cpu().float()
    ref = (O.exp32 if op == "exp" else O.log32)(x.float()).to(BF16).float()
    both_nan = torch.isnan(got) & torch.isnan(ref)
    same = (got == ref) | both_nan
    assert same.all(), x[~same][:8]


def test_fold_sums_equal_the_oracle_fold_order(device):
    """The routing kernels' 64-lane fp32 sums (DPP fold on the bit-reversed
    layout, and the shuffle butterfly) against the oracle's fold_sum, bit for
    bit, on groups whose magnitudes span many binades (so a different
    association would change low bits)."""
    from tao_attention import _hip
    g = torch.Generator().manual_seed(40)
    groups = 8192
    mant = torch.rand(groups, 64, generator=g) + 0.5
    sign = torch.where(torch.rand(groups, 64, generator=g) < 0.5, -1.0, 1.0)
    scale = torch.exp2(torch.randint(-30, 31, (groups, 64), generator=g).float())
    x = (sign * mant * scale).float()
    want = O.fold_sum(x, -1)
    assert not torch.equal(want, x.sum(-1)), "association should matter for these inputs"
    xd = x.to(device).contiguous()
    for op in (2, 3):
        y = torch.empty(groups, dtype=torch.float32, device=device)
        print(f"fold self-test op {op}", flush=True)
        _hip.check(_hip.lib().tao_numerics_selftest(op, xd.data_ptr(), y.data_ptr(),
                                                    groups * 64, _hip.stream_ptr(xd.device)))
        assert torch.equal(y.cpu(), want), op


@pytest.mark.parametrize("coarse,width", [(False, 64), (True, 64), (False, 128), (True, 128)])
def test_batched_decode_equals_per_request(device, coarse, width):
    """tao_attention_decode_batch == tao_attention_decode per request, bitwise:
    requests at different cursors (local-only, across a seal and refreshes,
    across the first page completion at 2560) and layers."""
    from tao_attention import TaoConfig, tao_attention_decode_batch
    heads, steps = 2, 40
    lengths, layers = [700, 1270, 2550], [0, 1, 3]
    cfg = TaoConfig() if coarse else index_only_page_memo()
    fa, fb = (torch.randn(heads, width, 3, generator=torch.Generator().manual_seed(9)) * 0.02
              for _ in range(2))
    fa, fb = fa.to(device), fb.to(device)
    xs = [to_dev(inputs(n + steps, heads, width, seed=20 + r)[0], device)
          for r, n in enumerate(lengths)]
    print(f"batched decode coarse={coarse} width={width}", flush=True)

    def prefilled():
        out = []
        for x, n, layer in zip(xs, lengths, layers):
            st = new_state(layer, cfg)
            q, k, v, rq, rk = (t[:, :n] for t in x)
            tao_attention_prefill(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb,
                                  alpha=0.5, state=st, position=0)
            out.append(st)
        return out

    batched, single = prefilled(), prefilled()
    for t in range(steps):
        rows = [[x[i][:, n + t:n + t + 1] for i in range(5)] for x, n in zip(xs, lengths)]
        q, k, v, rq, rk = (torch.cat([row[i] for row in rows], 0) for i in range(5))
        got, _ = tao_attention_decode_batch(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa,
                                            fusion_b=fb, alpha=0.5, states=batched)
        for r, st in enumerate(single):
            want, _ = tao_attention_decode(*rows[r][:3], raw_q=rows[r][3], raw_k=rows[r][4],
                                           fusion_a=fa, fusion_b=fb, alpha=0.5, state=st,
                                           position=st.get_pos())
            assert torch.equal(got[r:r + 1], want), (t, r)
    for a, b in zip(batched, single):
        sa, sb = a.export(), b.export()
        assert sa["position"] == sb["position"]
        for key in ("route_refreshes", "fine_seal_events", "state_version"):
            assert sa[key] == sb[key], key
        for x, y in zip(sa["local"], sb["local"]):
            assert torch.equal(x, y)
        if sb["packed_fine_c"] is not None:
            assert torch.equal(sa["packed_fine_c"], sb["packed_fine_c"])
            assert torch.equal(sa["route_ids"][1], sb["route_ids"][1])
        for (pz, pc, fz), (qz, qc, gz) in zip(sa["pages"], sb["pages"]):
            assert torch.equal(pz, qz) and torch.equal(fz, gz)
            assert (pc is None and qc is None) or torch.equal(pc, qc)


def test_batched_decode_after_member_reset(device):
    """A member of a running batch is reset and prefilled again (its buffers
    and native driver are recreated, possibly at recycled addresses): the
    batch must rebind to the new buffers and keep equalling per-request
    decode, bitwise, for every member."""
    from tao_attention import tao_attention_decode_batch
    heads, width = 2, 64
    lengths = [1300, 2000, 900]
    fa, fb = (torch.randn(heads, width, 3, generator=torch.Generator().manual_seed(19)) * 0.02
              for _ in range(2))
    fa, fb = fa.to(device), fb.to(device)
    xs = [to_dev(inputs(n + 60, heads, width, seed=120 + r)[0], device)
          for r, n in enumerate(lengths)]
    print("batched decode after a member reset", flush=True)

    def prefill(st, x, n):
        q, k, v, rq, rk = (t[:, :n] for t in x)
        tao_attention_prefill(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa, fusion_b=fb,
                              alpha=0.5, state=st, position=0)

    batched = [new_state(0, index_only_page_memo()) for _ in lengths]
    single = [new_state(0, index_only_page_memo()) for _ in lengths]
    for group in (batched, single):
        for st, x, n in zip(group, xs, lengths):
            prefill(st, x, n)
    cursor = list(lengths)

    def step():
        rows = [[x[i][:, c:c + 1] for i in range(5)] for x, c in zip(xs, cursor)]
        q, k, v, rq, rk = (torch.cat([row[i] for row in rows], 0) for i in range(5))
        got, _ = tao_attention_decode_batch(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa,
                                            fusion_b=fb, alpha=0.5, states=batched)
        for r, st in enumerate(single):
            want, _ = tao_attention_decode(*rows[r][:3], raw_q=rows[r][3], raw_k=rows[r][4],
                                           fusion_a=fa, fusion_b=fb, alpha=0.5, state=st,
                                           position=st.get_pos())
            assert torch.equal(got[r:r + 1], want), (cursor, r)
        for r in range(len(cursor)):
            cursor[r] += 1

    for _ in range(10):
        step()
    for group in (batched, single):
        group[1].reset()
        prefill(group[1], xs[1], lengths[1] - 700)
    cursor[1] = lengths[1] - 700
    for _ in range(30):
        step()


def _saved_and_loaded(snapshot):
    """torch.save, then torch.load(weights_only=True) (the trusted-file path)."""
    import io
    buf = io.BytesIO()
    torch.save(snapshot, buf)
    buf.seek(0)
    return torch.load(buf, weights_only=True)


def _to_cpu(snapshot):
    def cpu(x):
        if isinstance(x, torch.Tensor):
            return x.cpu()
        if isinstance(x, (list, tuple)):
            return type(x)(cpu(v) for v in x)
        return x
    return {k: cpu(v) for k, v in snapshot.items()}


@pytest.mark.parametrize("coarse", [False, True])
def test_snapshot_interop_with_oracle_through_torch_save(device, coarse):
    """Snapshot wire format: an oracle snapshot (the reference schema) written
    with torch.save and read with torch.load(weights_only=True) restores a
    HIP state that continues like the oracle; a HIP snapshot restores an
    oracle stream that continues like the HIP state."""
    from tao_attention import TaoConfig
    heads, width, n = 2, 64, 2700
    cfg = TaoConfig() if coarse else index_only_page_memo()
    geo = O.Geometry.from_config(cfg)
    xs, fa, fb = inputs(n + 330, heads, width, seed=21, unit_raw_k=True)
    head = [t[:, :n] for t in xs]
    rest = [t[:, n:] for t in xs]
    splits = [1] * 30 + [300]
    print(f"snapshot interop coarse={coarse}", flush=True)
    # oracle -> file -> HIP
    ora = O.OracleStream(1, geo)
    ora.prefill(*head, fa, fb, 0.5)
    hip = StreamCache.from_export(_saved_and_loaded(ora.export(config=cfg.export())))
    assert hip.get_pos() == n
    got = run_hip(hip, to_dev(rest, device), fa.to(device), fb.to(device), splits)
    want = []
    start = 0
    for w in splits:
        want.append(ora.prefill(*(t[:, start:start + w] for t in rest), fa, fb, 0.5))
        start += w
    torch.testing.assert_close(got.cpu().float(), torch.cat(want, 1).float(), **TOL)
    compare_snapshots(hip.export(), ora.export())
    # HIP -> file -> oracle
    hip2 = new_state(1, cfg)
    run_hip(hip2, to_dev(head, device), fa.to(device), fb.to(device), [n])
    ora2 = O.OracleStream.from_export(_saved_and_loaded(_to_cpu(hip2.export())), 1, geo)
    got2 = run_hip(hip2, to_dev(rest, device), fa.to(device), fb.to(device), splits)
    want2, start = [], 0
    for w in splits:
        want2.append(ora2.prefill(*(t[:, start:start + w] for t in rest), fa, fb, 0.5))
        start += w
    torch.testing.assert_close(got2.cpu().float(), torch.cat(want2, 1).float(), **TOL)
    compare_snapshots(hip2.export(), ora2.export())


# ------------------------------------------------------------- full sequence

def _bitmask_sets(qsel):
    """int32 bitmask words [B, T, H, W] -> bool [B, T, H, 32 W]."""
    words = qsel.cpu().to(torch.int64) & 0xFFFFFFFF
    bits = (words.unsqueeze(-1) >> torch.arange(32)) & 1
    return bits.reshape(*words.shape[:3], -1).bool()


@pytest.mark.parametrize("tokens,heads,width,index_only,seed", [
    (2100, 2, 64, True, 31), (2900, 2, 128, False, 32), (3000, 3, 64, False, 33)])
def test_full_sequence_read_matches_oracle(tokens, heads, width, index_only, seed):
    """tao_attention forward (per-query routes, per-query selected read, coarse
    read, fusion) against the oracle's read_training restatement: every
    query's selected set bit-exact, outputs within the bf16 tolerance."""
    from tao_attention import TaoConfig, tao_attention, training
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only)
    q, k, v, rq, rk = to_dev(xs, "cuda")
    fa_d, fb_d = fa.cuda(), fb.cuda()
    out, qsel = training.forward(q, k, v, rq, rk, fa_d, fb_d, 0.5, cfg, return_routes=True)
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True)
    got = _bitmask_sets(qsel)
    assert routes
    for tile, sel in routes.items():
        s = tile * 256
        part = got[:, s:s + sel.shape[1]]
        want = torch.zeros_like(part)
        want.scatter_(-1, sel, True)
        assert torch.equal(part, want), f"selected sets of tile {tile}"
    assert not got[:, :768].any()
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    api = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg)
    assert torch.equal(api, out)


def test_full_sequence_read_short_and_training_shape():
    """Below first_fine the output is the tiled local attention (oracle);
    at the training shape (B2, T8192, H12, D64) every history query selects
    exactly M of its tile's visible fines and the read is deterministic."""
    from tao_attention import TaoConfig, tao_attention, training
    cfg = TaoConfig()
    xs, fa, fb = inputs(700, 2, 128, 34)
    q, k, v, rq, rk = to_dev(xs, "cuda")
    out = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.cuda(), fusion_b=fb.cuda(),
                        alpha=0.5, config=cfg)
    ref = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg))
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    g = torch.Generator(device="cuda").manual_seed(35)
    b, t, h, d = 2, 8192, 12, 64
    xs = [torch.randn(b, t, h, d, generator=g, device="cuda").to(BF16) for _ in range(5)]
    fa = torch.randn(h, d, 3, generator=g, device="cuda") * 0.02
    fb = torch.randn(h, d, 3, generator=g, device="cuda") * 0.02
    out, qsel = training.forward(*xs, fa, fb, 0.5, cfg, return_routes=True)
    again = training.forward(*xs, fa, fb, 0.5, cfg)
    assert torch.equal(out, again)
    assert torch.isfinite(out.float()).all()
    counts = _bitmask_sets(qsel).sum(-1)                     # [B, T, H]
    geo = O.Geometry.from_config(cfg)
    for tile in range(t // 256):
        visible = max(0, tile - 2)
        m = geo.routed_counts(visible // 8, visible % 8)[2] if visible else 0
        assert bool((counts[:, tile * 256:(tile + 1) * 256] == m).all()), tile
    first = O.training_forward(*(x[:1, :768, :2].cpu() for x in xs), fa[:2].cpu(),
                               fb[:2].cpu(), 0.5, geo)
    torch.testing.assert_close(out[:1, :768, :2].cpu().float(), first.float(), **TOL)


def test_full_sequence_read_long_sequence_route_fallback():
    """T16484 at D128: the tile rows exceed the LDS rows of the lane-per-pair
    route, so the wave-per-query route runs. The read is causal, so the first
    2900 positions and the routes of tiles 3..11 must equal the oracle run on
    that prefix alone; every later query selects exactly M fines."""
    from tao_attention import TaoConfig, training
    cfg = TaoConfig()
    tokens, prefix = 16484, 2900
    xs, fa, fb = inputs(tokens, 2, 128, 37)
    dev = to_dev(xs, "cuda")
    out, qsel = training.forward(*dev, fa.cuda(), fb.cuda(), 0.5, cfg, return_routes=True)
    ref, routes = O.training_forward(*(x[:, :prefix] for x in xs), fa, fb, 0.5,
                                     O.Geometry.from_config(cfg), return_routes=True)
    got = _bitmask_sets(qsel)
    for tile, sel in routes.items():
        part = got[:, tile * 256:tile * 256 + sel.shape[1]]
        want = torch.zeros_like(part)
        want.scatter_(-1, sel, True)
        assert torch.equal(part, want), f"tile {tile}"
    torch.testing.assert_close(out[:, :prefix].cpu().float(), ref.float(), **TOL)
    geo = O.Geometry.from_config(cfg)
    counts = got.sum(-1)
    for tile in range(3, tokens // 256):
        visible = tile - 2
        m = geo.routed_counts(visible // 8, visible % 8)[2]
        assert bool((counts[:, tile * 256:(tile + 1) * 256] == m).all()), tile


GRAD_NAMES = ("q", "k", "v", "raw_q", "raw_k", "fusion_a", "fusion_b")


def _reference_gradients(xs, fa, fb, grad, cfg, routes):
    """fp64 autograd of the oracle's smooth full-sequence function at the
    bf16 forward's selections."""
    leaves = [x.double().requires_grad_(True) for x in xs]
    fa64, fb64 = fa.double().requires_grad_(True), fb.double().requires_grad_(True)
    out = O.training_forward_smooth(*leaves, fa64, fb64, 0.5, routes,
                                    O.Geometry.from_config(cfg), writer=cfg.fine_writer)
    every = leaves + [fa64, fb64]
    grads = torch.autograd.grad((out * grad.double()).sum(), every, allow_unused=True)
    return [torch.zeros_like(x) if g is None else g for g, x in zip(grads, every)]


def _compare_gradients(got, want, rel_tol):
    worst = {}
    for name, g, r in zip(GRAD_NAMES, got, want):
        g, r = g.detach().cpu().double(), r.double()
        scale = r.norm().item()
        err = (g - r).norm().item()
        worst[name] = err / scale if scale > 0 else err   # absolute when the reference is 0
    print("relative gradient errors:", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)
    for name, rel in worst.items():
        assert rel < rel_tol, (name, rel)


@pytest.mark.parametrize("tokens,heads,width,index_only,seed", [
    (700, 2, 64, True, 41), (700, 2, 128, False, 42),
    (2100, 2, 64, True, 43), (2900, 2, 128, False, 44), (3000, 3, 64, False, 45)])
def test_full_sequence_backward_matches_oracle(tokens, heads, width, index_only, seed):
    """tao_attention backward (fusion, local attention, selected read, coarse
    read, page / segment softmaxes, writer) against fp64 autograd of the
    oracle's smooth forward at the same selections."""
    from tao_attention import TaoConfig, tao_attention
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only)
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(seed + 100)).to(BF16)
    dev = [x.cuda().requires_grad_(True) for x in xs]
    fa_d = fa.cuda().requires_grad_(True)
    fb_d = fb.cuda().requires_grad_(True)
    print(f"full-sequence backward T{tokens} H{heads} D{width} index_only={index_only}",
          flush=True)
    out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg)
    got = torch.autograd.grad(out, dev + [fa_d, fb_d], grad.cuda())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True)
    want = _reference_gradients(xs, fa, fb, grad, cfg, routes)
    for g in got:
        assert torch.isfinite(g.float()).all()
    _compare_gradients(got, want, 5e-2)


@pytest.mark.parametrize("tokens,heads,width,seed,index_only", [
    (1300, 2, 64, 61, True), (2900, 2, 128, 62, True), (3100, 2, 64, 63, False)])
def test_full_sequence_backward_regularized_writer(tokens, heads, width, seed, index_only):
    """tao_attention backward with fine_writer="regularized_association"
    (index-only, and with page values past 2,560 tokens: each page matrix's
    adjoint adds to its fines'): the writer's share differentiates the association solve
    (dC -> W = A^{-1} dC, dG from W and the fp32 C, then U, V and the
    feature softmax), the z path stays the softmax writer's; all gradients
    against fp64 autograd of the oracle's smooth forward through
    torch.linalg.solve, at the bf16 forward's selections; the raw_k and v
    gradients differ from the softmax writer's."""
    from tao_attention import TaoConfig, tao_attention
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only, fine_writer="regularized_association")
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(seed + 100)).to(BF16)
    dev = [x.cuda().requires_grad_(True) for x in xs]
    fa_d = fa.cuda().requires_grad_(True)
    fb_d = fb.cuda().requires_grad_(True)
    print(f"regularized-writer backward T{tokens} H{heads} D{width}", flush=True)
    out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg)
    got = torch.autograd.grad(out, dev + [fa_d, fb_d], grad.cuda())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True, writer=cfg.fine_writer)
    want = _reference_gradients(xs, fa, fb, grad, cfg, routes)
    for g in got:
        assert torch.isfinite(g.float()).all()
    _compare_gradients(got, want, 5e-2)
    soft = _reference_gradients(xs, fa, fb, grad, TaoConfig(coarse_index_only=index_only),
                                routes)
    for i in (2, 4):                                    # v, raw_k
        assert (soft[i] - want[i]).norm() > 0.1 * want[i].norm()


@pytest.mark.parametrize("writer,tokens,width,index_only,seed", [
    ("feature_mass_association", 1300, 64, True, 71),
    ("feature_mass_association", 2900, 128, False, 72),
    ("structured_gram_association", 1300, 128, True, 73),
    ("structured_gram_association", 3100, 64, False, 74)])
def test_full_sequence_backward_feature_writers(writer, tokens, width, index_only, seed):
    """tao_attention backward through the feature writers (index-only, and
    with the page mixture past 2,560 tokens): the mixture reads' adjoints
    (coefficients r(w_m h), w_m from h . exp(z_m)), z = log mass, the
    association solve or the structured closed form of each block and page,
    the feature softmax; every gradient against fp64 autograd of the
    oracle's smooth forward at the bf16 forward's selections."""
    from tao_attention import TaoConfig, tao_attention
    heads = 2
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only, fine_writer=writer)
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(seed + 100)).to(BF16)
    dev = [x.cuda().requires_grad_(True) for x in xs]
    fa_d = fa.cuda().requires_grad_(True)
    fb_d = fb.cuda().requires_grad_(True)
    print(f"{writer} backward T{tokens} H{heads} D{width} index_only={index_only}", flush=True)
    out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg)
    got = torch.autograd.grad(out, dev + [fa_d, fb_d], grad.cuda())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True, writer=writer)
    want = _reference_gradients(xs, fa, fb, grad, cfg, routes)
    for g in got:
        assert torch.isfinite(g.float()).all()
    _compare_gradients(got, want, 5e-2)
    soft = _reference_gradients(xs, fa, fb, grad, TaoConfig(coarse_index_only=index_only),
                                routes)
    for i in (2, 3, 4):                                 # v, raw_q, raw_k
        assert (soft[i] - want[i]).norm() > 0.1 * want[i].norm()


@pytest.mark.parametrize("tokens,heads,width,index_only,seed", [
    (2100, 2, 64, True, 48), (2900, 2, 128, False, 49)])
def test_full_sequence_alpha_gradient(tokens, heads, width, index_only, seed):
    """d alpha (gain = 2 alpha; no reference counterpart) against fp64
    autograd of the oracle's smooth forward with alpha as a leaf; a float
    alpha gives the same output and no alpha gradient."""
    from tao_attention import TaoConfig, tao_attention
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only)
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(seed + 100)).to(BF16)
    dev = [x.cuda() for x in xs]
    alpha = torch.tensor(0.5, device="cuda", requires_grad=True)
    q = dev[0].clone().requires_grad_(True)
    out = tao_attention(q, *dev[1:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                        fusion_b=fb.cuda(), alpha=alpha, config=cfg)
    dq, dalpha = torch.autograd.grad(out, [q, alpha], grad.cuda())
    with torch.no_grad():
        plain = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                              fusion_b=fb.cuda(), alpha=0.5, config=cfg)
    assert torch.equal(plain, out.detach())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True)
    a64 = torch.tensor(0.5, dtype=torch.float64, requires_grad=True)
    ref = O.training_forward_smooth(*(x.double() for x in xs), fa.double(), fb.double(), a64,
                                    routes, O.Geometry.from_config(cfg))
    (want,) = torch.autograd.grad((ref * grad.double()).sum(), [a64])
    print(f"d alpha: {dalpha.item():.6e} (fp64 oracle {want.item():.6e})", flush=True)
    assert dalpha.shape == alpha.shape
    # a host alpha gets the same gradient on the host (asynchronous copy)
    alpha_h = torch.tensor(0.5, requires_grad=True)
    out_h = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                          fusion_b=fb.cuda(), alpha=alpha_h, config=cfg)
    (dh,) = torch.autograd.grad(out_h, [alpha_h], grad.cuda())
    torch.cuda.synchronize()
    assert dh.device.type == "cpu"
    assert abs(dh.item() - dalpha.item()) <= 1e-5 * abs(dalpha.item())
    assert abs(dalpha.item() - want.item()) <= 5e-2 * abs(want.item())
    # finite difference of the bf16 forward itself with a coherent upstream
    # gradient (ones): the fused output is linear in gain = bf16(2 alpha) up to
    # per-term bf16 roundings, which average out over the sum; gain moves
    # exactly from 0.5 to 1.5 for alpha = 0.25 and 0.75
    out1 = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                         fusion_b=fb.cuda(), alpha=alpha, config=cfg)
    (d1,) = torch.autograd.grad(out1, [alpha], torch.ones_like(out1))
    with torch.no_grad():
        f = [tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                           fusion_b=fb.cuda(), alpha=a, config=cfg).double().sum().item()
             for a in (0.25, 0.75)]
    fd = (f[1] - f[0]) / 0.5
    print(f"d alpha (ones): {d1.item():.6e} (finite difference {fd:.6e})", flush=True)
    assert abs(d1.item() - fd) <= 1e-2 * abs(fd)


@pytest.mark.parametrize("writer,tokens,heads,width,index_only,seed", [
    ("softmax", 2100, 2, 64, True, 46), ("softmax", 2900, 2, 128, False, 47),
    ("feature_mass_association", 2100, 2, 128, True, 75),
    ("structured_gram_association", 2900, 2, 64, False, 76)])
def test_full_sequence_memory_adjoints_match_oracle(writer, tokens, heads, width, index_only,
                                                    seed):
    """The memory branch's adjoints before the writer, d fine_z (segment
    weights, page weights, page / pending logsumexps, coarse weights and page
    value matrices; for the feature writers the mixture weights'
    h . exp(z) path) and d C (selected read and coarse read; the mixture
    read), against fp64 autograd at the oracle's fine_z and bank: each path
    that the end-to-end gradients cannot resolve (the page-weight softmax is
    ~0.2 % of d raw_k, the feature writers' descriptor path ~1 %) is a large
    part of these."""
    from tao_attention import TaoConfig, training
    xs, fa, fb = inputs(tokens, heads, width, seed)
    cfg = TaoConfig(coarse_index_only=index_only, fine_writer=writer)
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(seed + 100)).to(BF16)
    dev = to_dev(xs, "cuda")
    print(f"memory adjoints T{tokens} D{width} index_only={index_only}", flush=True)
    _, data = training._forward_for_backward(*dev, fa.cuda(), fb.cuda(), 0.5, cfg)
    mem = {}
    training.backward(data, grad.cuda(), fa.cuda(), fb.cuda(), 0.5, memory_adjoints=mem)
    geo = O.Geometry.from_config(cfg)
    _, routes = O.training_forward(*xs, fa, fb, 0.5, geo, return_routes=True, writer=writer)
    leaves = [x.double() for x in xs]
    inter = {}
    out = O.training_forward_smooth(*leaves[:4], leaves[4].requires_grad_(True), fa.double(),
                                    fb.double(), 0.5, routes, geo, intermediates=inter,
                                    writer=writer)
    dz, dc = torch.autograd.grad((out * grad.double()).sum(), [inter["fine_z"], inter["bank"]])
    for name, got, want in (("dz", mem["dz"], dz), ("dc", mem["dc"], dc)):
        rel = ((got.cpu().double() - want).norm() / want.norm()).item()
        print(f"{name} relative error {rel:.2e}", flush=True)
        assert rel < 2e-2, (name, rel)
