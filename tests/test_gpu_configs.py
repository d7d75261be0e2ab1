"""HIP path vs the CPU oracle at the routing regimes of the benchmark configs.

The configs route with coarse page selection active: a 16K prompt keeps 4 of
its 7 completed pages (E 38, M 14), a 32K state 5 of 15 (E 46, M 18) and a
131K state 9 of 63 (E 78, M 34). These tests run those states at reduced
heads (the per-head arithmetic is independent of H) so the oracle finishes
in seconds, and hold the bar of the parity suite: route ids, chosen pages,
fine and page descriptors bit-exact; outputs and fine matrices within 2e-2.
"""
import pytest
import torch

from oracle import tao_oracle as O
from tao_attention import StreamCache, TaoConfig, new_state
from tao_attention.presets import index_only_page_memo
from test_gpu_parity import (TOL, compare_diagnostics, compare_snapshots, inputs, run_hip,
                             run_oracle, to_dev, _bitmask_sets, _compare_gradients,
                             _reference_gradients)

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16
PRESET = index_only_page_memo()
PRESET_GEO = O.Geometry.from_config(PRESET)


def _route_shape(state):
    snap = state.export()
    return snap["route_ids"][0].shape[-1], snap["route_ids"][1].shape[-1], len(snap["pages"])


@pytest.mark.parametrize("width,splits", [
    (128, [16384]),
    (64, [9000] + [1] * 30 + [7354]),
])
def test_prefill_16k_page_selection_matches_oracle(device, width, splits):
    """configs[2] at H2: a 16,384-token prompt (unit-norm raw_k rows) whose
    last route keeps 4 of 7 completed pages; the chunked variant routes
    single tokens between the two long calls."""
    heads = 2
    xs, fa, fb = inputs(sum(splits), heads, width, seed=51 + width, unit_raw_k=True)
    print(f"16K prefill width={width} calls={len(splits)}", flush=True)
    state = new_state(0, PRESET)
    out = run_hip(state, to_dev(xs, device), fa.to(device), fb.to(device), splits)
    ora, ref = run_oracle(0, xs, fa, fb, splits, geometry=PRESET_GEO)
    coarse, selected, pages = _route_shape(state)
    assert (coarse, selected, pages) == (4, 14, 7)
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())
    compare_diagnostics(state, ora)


_LONG = {}


def _long_state(tokens, heads, width, layer, seed, decode):
    """Oracle prefill of `tokens` tokens plus `decode` single-token steps,
    cached per shape (the graph and eager variants share it)."""
    key = (tokens, heads, width, layer, seed, decode)
    if key not in _LONG:
        xs, fa, fb = inputs(tokens + decode, heads, width, seed)
        splits = [tokens] + [1] * decode
        ora, ref = run_oracle(layer, xs, fa, fb, splits, geometry=PRESET_GEO)
        _LONG.clear()
        _LONG[key] = (xs, fa, fb, splits, ora, ref)
    return _LONG[key]


@pytest.mark.parametrize("tokens,width,layer,graph,expect", [
    (32768, 64, 1, False, (5, 18, 15)),
    (32768, 64, 1, True, (5, 18, 15)),
    (131072, 128, 0, False, (9, 34, 63)),
    (131072, 128, 0, "hipgraph", (9, 34, 63)),
])
def test_decode_from_long_state_matches_oracle(device, monkeypatch, tokens, width, layer, graph,
                                               expect):
    """configs[3] regime at H2: prefill a 32K / 131K state, then 300 decode
    steps through at least 12 route refreshes and one seal (the local window
    holds 512 tokens at these cursors, so the seal is at +256). The graph
    preset replays the captured step across them, by recorded dispatch
    (True) or by hipGraph launches ("hipgraph", configs[3]'s mode)."""
    heads, decode = 2, 300
    xs, fa, fb, splits, ora, ref = _long_state(tokens, heads, width, layer, 60 + width, decode)
    print(f"decode from {tokens} width={width} graph={graph}", flush=True)
    if graph == "hipgraph":
        monkeypatch.setenv("TAO_GRAPH_REPLAY", "hipgraph")
    state = new_state(layer, index_only_page_memo(graph=bool(graph)))
    d = to_dev(xs, device)
    out = run_hip(state, d, fa.to(device), fb.to(device), splits)
    assert _route_shape(state) == expect
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())
    compare_diagnostics(state, ora)
    if graph:
        obs = state.history_region.observation()
        assert obs["replays"] > 0 and obs["captures"] > 0
    state.release_execution()


@pytest.mark.parametrize("tokens,width,index_only,seed", [
    (8960, 64, False, 71), (9300, 128, True, 72)])
def test_full_sequence_batch2_page_selection_matches_oracle(tokens, width, index_only, seed):
    """configs[1] regime at H2, batch 2: tiles past 8,704 tokens keep 3 of 4
    completed pages; every query's selected set bit-exact against the
    oracle's read_training restatement, outputs within the bf16 tolerance."""
    from tao_attention import training
    g = torch.Generator().manual_seed(seed)
    heads = 2
    xs = [torch.randn(2, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    cfg = TaoConfig(coarse_index_only=index_only)
    print(f"full sequence B2 T{tokens} D{width}", flush=True)
    out, qsel = training.forward(*to_dev(xs, "cuda"), fa.cuda(), fb.cuda(), 0.5, cfg,
                                 return_routes=True)
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True)
    got = _bitmask_sets(qsel)
    geo = O.Geometry.from_config(cfg)
    selecting = 0
    for tile, sel in routes.items():
        s = tile * 256
        part = got[:, s:s + sel.shape[1]]
        want = torch.zeros_like(part)
        want.scatter_(-1, sel, True)
        assert torch.equal(part, want), f"selected sets of tile {tile}"
        completed = (tile - 2) // 8
        if geo.routed_counts(completed, (tile - 2) % 8)[0] < completed:
            selecting += 1
    assert selecting > 0, "no tile selects among its completed pages"
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)


@pytest.mark.parametrize("tokens,width,index_only,seed", [
    (2900, 64, False, 73), (8960, 64, True, 74)])
def test_full_sequence_backward_batch2(tokens, width, index_only, seed):
    """configs[1] backward at batch 2: all seven gradients against fp64
    autograd of the oracle's smooth forward at the bf16 forward's selections
    (the 8,960-token case selects among completed pages)."""
    from tao_attention import tao_attention
    g = torch.Generator().manual_seed(seed)
    heads = 2
    xs = [torch.randn(2, tokens, heads, width, generator=g).to(BF16) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    grad = torch.randn(xs[0].shape, generator=g).to(BF16)
    cfg = TaoConfig(coarse_index_only=index_only)
    dev = [x.cuda().requires_grad_(True) for x in xs]
    fa_d = fa.cuda().requires_grad_(True)
    fb_d = fb.cuda().requires_grad_(True)
    print(f"full-sequence backward B2 T{tokens} D{width}", flush=True)
    out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg)
    got = torch.autograd.grad(out, dev + [fa_d, fb_d], grad.cuda())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True)
    want = _reference_gradients(xs, fa, fb, grad, cfg, routes)
    for t in got:
        assert torch.isfinite(t.float()).all()
    _compare_gradients(got, want, 5e-2)


@pytest.mark.parametrize("width", [64, 128])
def test_batched_decode_ragged_long_matches_oracle(device, width):
    """configs[4] regime at H2: four requests prefilled to ragged lengths in
    [16384, 32768] (seeded), 128 batched steps through their own route
    refreshes and seals; each request's outputs and final state against its
    own oracle stream. D128 is configs[4]'s width (the batch_units_kernel<128>
    and batch_combine_kernel<128> its bench line times)."""
    from tao_attention import tao_attention_decode_batch
    heads, steps = 2, 128
    g = torch.Generator().manual_seed(81)
    lengths = torch.randint(16384, 32769, (4,), generator=g).tolist()
    seals = [(n - 768) % 256 + steps >= 256 for n in lengths]
    assert any(seals) and not all(seals), lengths
    fa = (torch.randn(heads, width, 3, generator=g) * 0.02)
    fb = (torch.randn(heads, width, 3, generator=g) * 0.02)
    xs = [inputs(n + steps, heads, width, seed=90 + r)[0] for r, n in enumerate(lengths)]
    print(f"batched decode lengths={lengths} width={width}", flush=True)
    states, oracles = [], []
    for x, n in zip(xs, lengths):
        st = new_state(0, PRESET)
        run_hip(st, [t[:, :n].to(device) for t in x], fa.to(device), fb.to(device), [n])
        states.append(st)
        ora = O.OracleStream(0, PRESET_GEO)
        ora.prefill(*(t[:, :n] for t in x), fa, fb, 0.5)
        oracles.append(ora)
    got, want = [], []
    fa_d, fb_d = fa.to(device), fb.to(device)
    for t in range(steps):
        rows = [[x[i][:, n + t:n + t + 1] for i in range(5)] for x, n in zip(xs, lengths)]
        q, k, v, rq, rk = (torch.cat([row[i] for row in rows], 0).to(device) for i in range(5))
        out, _ = tao_attention_decode_batch(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa_d,
                                            fusion_b=fb_d, alpha=0.5, states=states)
        got.append(out.cpu())
        want.append(torch.cat([o.decode(*row, fa, fb, 0.5) for o, row in zip(oracles, rows)], 0))
    torch.testing.assert_close(torch.cat(got, 1).float(), torch.cat(want, 1).float(), **TOL)
    for st, ora in zip(states, oracles):
        compare_snapshots(st.export(), ora.export())
        assert st.export()["route_refreshes"] == ora.route_refreshes
