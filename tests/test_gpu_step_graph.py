"""Whole-step decode graph across layers (WholeStepGraph, step_graph.py).

A small model of the reference benchmark's block shape (RMSNorm, RoPE on the
normalised q / k, TaoMemory attention, residual output projection;
docs/benchmarks.md:15) with one state per layer decodes the same tokens two
ways: eagerly through every layer's driver, and through one captured graph
of the whole step whose decode launches read their cursors on the device.
Every token's hidden state must be bitwise equal between the two, across
route refreshes, a seal and the captures they force, and the states must
end equal (cursors, counters, device buffers). The eager decode itself is
checked against the oracle in test_gpu_parity.py.
"""
import pytest
import torch
import torch.nn.functional as F

from tao_attention import WholeStepGraph, new_state, schedule, tao_attention_decode
from tao_attention.presets import index_only_page_memo

pytestmark = pytest.mark.gpu

LAYERS, HEADS, DIM, VOCAB = 3, 2, 128, 512
WIDTH = HEADS * DIM


def _model(device, seed=5):
    g = torch.Generator(device=device).manual_seed(seed)

    def w(*shape):
        return (torch.randn(shape, generator=g, device=device) * 0.05).to(torch.bfloat16)

    return dict(embed=w(VOCAB, WIDTH), unembed=w(WIDTH, VOCAB),
                layers=[dict(qkv=w(WIDTH, 3 * WIDTH), o=w(WIDTH, WIDTH),
                             fa=w(HEADS, DIM, 3).float(), fb=w(HEADS, DIM, 3).float())
                        for _ in range(LAYERS)])


def _states(device, context, seed=9):
    """One state per layer, each with its layer index: layer l refreshes its
    route at first_fine + 2 l + 24 k (tao_stream.py:202-208), so the
    layers' refresh turns are staggered."""
    g = torch.Generator(device=device).manual_seed(seed)
    states = []
    for layer in range(LAYERS):
        st = new_state(layer, index_only_page_memo())
        xs = [torch.randn((1, context, HEADS, DIM), generator=g, device=device)
              .to(torch.bfloat16) for _ in range(5)]
        st._ingest(*xs)
        states.append(st)
    return states


def _step_fn(m, states):
    inv = 1.0 / (10000.0 ** (torch.arange(0, DIM, 2, device=m["embed"].device).float() / DIM))

    def rope(x, pos_t):
        ang = pos_t.float() * inv
        cos = torch.cat((ang.cos(), ang.cos())).to(torch.bfloat16)
        sin = torch.cat((-ang.sin(), ang.sin())).to(torch.bfloat16)
        return x * cos + x.roll(DIM // 2, -1) * sin

    def step(token):
        x = m["embed"].index_select(0, token.view(1)).view(1, 1, WIDTH)
        for lw, st in zip(m["layers"], states):
            pos_t = st.device_position()
            h = F.rms_norm(x, (WIDTH,))
            raw_q, raw_k, v = (h @ lw["qkv"]).view(1, 1, 3, HEADS, DIM).unbind(2)
            q = rope(F.rms_norm(raw_q, (DIM,)), pos_t)
            k = rope(F.rms_norm(raw_k, (DIM,)), pos_t)
            a, _ = tao_attention_decode(q, k, v, raw_q=raw_q, raw_k=raw_k, fusion_a=lw["fa"],
                                        fusion_b=lw["fb"], alpha=0.5, state=st,
                                        position=st.get_pos())
            x = x + a.reshape(1, 1, WIDTH) @ lw["o"]
        return (F.rms_norm(x, (WIDTH,)) @ m["unembed"]).view(-1).argmax(), x

    return step


# (context, tokens): 2200 crosses the three layers' staggered refreshes and
# the seal at 2303, after which the next refresh of each layer changes its
# route size; 700 crosses the first seal, which turns the fine branch on, and
# the first refreshes of every layer.
@pytest.mark.parametrize("context,steps", [(2200, 130), (700, 100)])
def test_whole_step_graph_equals_eager_loop(context, steps):
    device = torch.device("cuda:0")
    print(f"whole-step graph: {LAYERS} staggered layers H{HEADS} D{DIM}, context {context}, "
          f"{steps} tokens", flush=True)
    m = _model(device)
    eager_states, graph_states = _states(device, context), _states(device, context)
    for st in eager_states:
        assert int(st.device_position()) == st.position == context
    step_e, step_g = _step_fn(m, eager_states), _step_fn(m, graph_states)
    graph = WholeStepGraph(graph_states)
    tok_e = torch.zeros((), dtype=torch.long, device=device)
    tok_g = tok_e.clone()
    seals0 = eager_states[0].fine_seal_events
    cfg = graph_states[0].config
    replayed_turns = eager_turns = 0
    for i in range(steps):
        pos = context + i
        turns = [st.layer_index for st in graph_states
                 if schedule.fines_at(pos, cfg) > 0 and schedule.is_turn(pos, st.layer_index, cfg)]
        before = graph.replays
        tok_e, x_e = step_e(tok_e)
        out = graph.step(step_g, tok_g)
        tok_g, x_g = out[0].clone(), out[1].clone()
        assert torch.equal(x_e, x_g), f"token {i} (position {pos}) differs"
        assert torch.equal(tok_e, tok_g)
        if turns:
            if graph.replays > before:
                replayed_turns += 1
            else:
                eager_turns += 1
    torch.cuda.synchronize()
    print(f"replays {graph.replays}, eager {graph.eager_steps}, captures {graph.captures}, "
          f"refresh tokens replayed {replayed_turns}, eager {eager_turns}", flush=True)
    assert eager_states[0].fine_seal_events > seals0, "the run must cross a seal"
    assert graph.replays + graph.eager_steps == steps
    # Refresh tokens replay (their gated refreshes run on the device) unless a
    # route size changes; the eager tokens are the seal, the refreshes that
    # change a route size and the warm-up token before each capture.
    assert replayed_turns >= 3, (replayed_turns, eager_turns)
    assert graph.replays >= steps * 3 // 4, (graph.replays, graph.captures, graph.eager_steps)
    for a, b in zip(eager_states, graph_states):
        assert a.position == b.position == context + steps
        assert int(b.device_position()) == b.position
        for name in ("fusion_pointwise_calls", "fusion_no_history_local_returns",
                     "route_refreshes", "peak_selected_fine", "fine_seal_events", "route_size",
                     "route_coarse"):
            assert getattr(a, name) == getattr(b, name), name
        for name in ("ring_k", "ring_v", "ring_raw", "page_z", "sel", "fold_g", "fold_den"):
            assert torch.equal(getattr(a._dev, name), getattr(b._dev, name)), name
    graph.release()


def test_whole_step_graph_rejects_non_plain_capture():
    """A device-cursor step is refused for a token that refreshes or seals."""
    device = torch.device("cuda:0")
    m = _model(device)
    states = _states(device, 766)
    step = _step_fn(m, states)
    tok = torch.zeros((), dtype=torch.long, device=device)
    step(tok)                          # binds the drivers (eager)
    plan = states[0]._plan_next()
    assert plan[0] == 767 and plan[2] == 1      # the step at 767 fills the window: a seal
    assert not states[0]._replayable_next()
    states[0]._capturing = True
    try:
        with pytest.raises(RuntimeError, match="seals or changes its route"):
            step(tok)
    finally:
        states[0]._capturing = False
