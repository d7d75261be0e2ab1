"""Decode-graph epochs of the graph preset (history_region_graph.py:10-113).

The native driver's epoch counters are checked against a step-by-step model
of the reference's HistoryRegionGraph state machine driven by the call
sequence (which positions refresh, which seal, which calls are region
calls), and the outputs of both replay mechanisms (recorded dispatch and
hipGraph) against the eager preset, bitwise.
"""
import pytest
import torch

from oracle import tao_oracle as O
from tao_attention import new_state, tao_attention_decode, tao_attention_prefill
from tao_attention.presets import index_only_page_memo
from test_gpu_parity import inputs, to_dev

pytestmark = pytest.mark.gpu

OBSERVATION_KEYS = {
    "epochs", "eager_warm", "captures", "replays", "id_copies", "invalidations",
    "active_graph", "active_staging", "epoch_state_version", "epoch_warm_count",
    "last_action", "invalidation_reasons", "last_retired_execution_tensors_alive",
    "python_owned_semantic_tensor_references", "capture_address_scope"}


class EpochModel:
    """HistoryRegionGraph's counters (history_region_graph.py:10-113) as its
    callers drive them (tao_stream.py:196-249, 358-359, 405-406, 444-445,
    838-844), stepped over absolute positions with the oracle's geometry."""

    def __init__(self, layer, geometry):
        self.g, self.layer = geometry, layer
        self.counts = dict(epochs=0, eager_warm=0, captures=0, replays=0, id_copies=0,
                           invalidations=0)
        self.reasons = {}
        self.key = None
        self.warm = 0
        self.graph = False
        self.route = None        # selected count of the current route

    def fines(self, p):
        return max(0, (p - self.g.local_keep) // self.g.fine_tokens)

    def invalidate(self, reason):
        if self.key is None:
            return
        self.key, self.warm, self.graph = None, 0, False
        self.counts["invalidations"] += 1
        self.reasons[reason] = self.reasons.get(reason, 0) + 1

    def refresh(self, fines):
        completed, pending = divmod(fines, self.g.coarse_group)
        self.route = self.g.routed_counts(completed, pending)[2]
        if self.key is not None:                       # update_routes
            if self.key[1] != self.route:
                self.invalidate("selected_shape")
            else:
                self.counts["id_copies"] += 1

    def run(self, fines):
        key = (fines, self.route)
        if key != self.key:
            self.invalidate("epoch_change")
            self.key, self.warm = key, 0
            self.counts["epochs"] += 1
            self.counts["id_copies"] += 1
        if self.warm < 3:
            self.warm += 1
            self.counts["eager_warm"] += 1
            return
        if not self.graph:
            self.graph = True
            self.counts["captures"] += 1
        self.counts["replays"] += 1

    def call(self, pos, width):
        """One prefill (width > 1) or decode (width 1) call at cursor pos."""
        for p in range(pos, pos + width):
            fines = self.fines(p)
            if fines and self.g.is_turn(p, self.layer):
                self.refresh(fines)
            elif fines and width == 1:
                self.run(fines)
            if self.fines(p + 1) != fines:
                self.invalidate("seal")


def _run(state, d, fa, fb, calls, model=None, busy_every=0):
    q, k, v, rq, rk = d
    outs, start = [], state.get_pos()
    for n, width in enumerate(calls):
        if width == "release":
            state.release_execution()
            if model is not None:
                model.invalidate("request_end")
            continue
        sl = slice(start, start + width)
        if busy_every and n % busy_every == 0:
            torch.cuda._sleep(8_000_000)       # queue the next calls behind the device (~3 ms)
        fn = tao_attention_decode if width == 1 else tao_attention_prefill
        out, state = fn(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl], raw_k=rk[:, sl],
                        fusion_a=fa, fusion_b=fb, alpha=0.5, state=state,
                        position=state.get_pos())
        outs.append(out.clone())
        if model is not None:
            model.call(start, width)
        start += width
    torch.cuda.synchronize()
    return torch.cat(outs, 1)


CALLS = [1000] + [1] * 300 + ["release"] + [1] * 40 + [130] + [1] * 300


@pytest.mark.parametrize("replay", ["dispatch", "hipgraph"])
def test_graph_epochs_follow_reference_state_machine(device, replay, monkeypatch):
    """Counters after every phase of a call sequence that crosses seals,
    route-size changes, a release and a prefill inside an epoch; outputs
    bitwise equal to the eager preset. The hipgraph run keeps the device
    busy before groups of calls so replays queue up behind each other (each
    replay's operands must be the ones it was launched with)."""
    heads, width, layer = 4, 128, 0
    tokens = sum(c for c in CALLS if c != "release")
    xs, fa, fb = inputs(tokens, heads, width, seed=91)
    d = to_dev(xs, device)
    fa, fb = fa.to(device), fb.to(device)
    print(f"graph epochs replay={replay}", flush=True)
    eager = _run(new_state(layer, index_only_page_memo(graph=False)), d, fa, fb, CALLS)
    monkeypatch.setenv("TAO_GRAPH_REPLAY", replay)
    state = new_state(layer, index_only_page_memo(graph=True))
    model = EpochModel(layer, O.Geometry.from_config(index_only_page_memo()))
    got = _run(state, d, fa, fb, CALLS, model, busy_every=25 if replay == "hipgraph" else 0)
    assert torch.equal(eager, got)
    obs = state.history_region.observation()
    assert set(obs) == OBSERVATION_KEYS
    assert {k: obs[k] for k in model.counts} == model.counts
    assert obs["invalidation_reasons"] == model.reasons
    assert model.counts["captures"] >= 3 and model.counts["replays"] > 300
    assert {"seal", "selected_shape", "request_end"} <= set(model.reasons)
    assert obs["active_staging"] == (model.key is not None)
    assert obs["epoch_warm_count"] == model.warm
    assert obs["epoch_state_version"] == (model.key[0] if model.key else None)
    state.release_execution()
    obs = state.history_region.observation()
    assert obs["last_action"] == "invalidate:request_end" and not obs["active_graph"]


def test_graph_epoch_ends_on_new_fusion_parameters(device):
    """A call with other fusion parameters ends the epoch as an epoch change
    (the reference's key covers every captured address) and restarts the
    three eager steps; outputs stay bitwise equal to eager."""
    heads, width, layer = 2, 64, 1
    xs, fa, fb = inputs(1100, heads, width, seed=92)
    d = to_dev(xs, device)
    fa, fb = fa.to(device), fb.to(device)
    fa2, fb2 = fa * 0.5, fb + 0.25
    print("graph epoch fusion change", flush=True)
    outs = {}
    for graph in (False, True):
        state = new_state(layer, index_only_page_memo(graph=graph))
        q, k, v, rq, rk = d
        out, state = tao_attention_prefill(q[:, :1000], k[:, :1000], v[:, :1000],
                                           raw_q=rq[:, :1000], raw_k=rk[:, :1000],
                                           fusion_a=fa, fusion_b=fb, alpha=0.5, state=state,
                                           position=0)
        res = []
        for p in range(1000, 1030):
            a, b = (fa, fb) if p < 1015 else (fa2, fb2)
            out, state = tao_attention_decode(q[:, p:p + 1], k[:, p:p + 1], v[:, p:p + 1],
                                              raw_q=rq[:, p:p + 1], raw_k=rk[:, p:p + 1],
                                              fusion_a=a, fusion_b=b, alpha=0.5, state=state,
                                              position=p)
            res.append(out.clone())
        outs[graph] = torch.cat(res, 1)
        if graph:
            obs = state.history_region.observation()
            assert obs["invalidation_reasons"].get("epoch_change", 0) >= 1
            assert obs["epoch_warm_count"] == 3 or obs["last_action"] in ("replay",
                                                                         "capture_replay")
    assert torch.equal(outs[False], outs[True])
