"""The local_flash plugin slot (operator.py:42-47, 70-138; flash_attention.py:16-40).

A caller plugin computes the local attention with the reference's call
pattern: one call per next_chunk chunk over the retained window plus the
chunk (tao_stream.py:919-934) when streaming, and the tiling of
_local_training_corrected_4k (tao_stream.py:760-787) for tao_attention. The
read, fusion and state stay on the HIP path. Two plugins are used: a
recorder around this library's own kernel and a foreign fp32 torch SDPA (the
reference's adapter evaluated in fp32). Both must match the oracle.
"""
from types import SimpleNamespace

import pytest
import torch
import torch.nn.functional as F

from oracle import tao_oracle as O
from tao_attention import TaoConfig, new_state, tao_attention
from tao_attention import schedule
from tao_attention.flash_attention import flash_attn_func
from tao_attention.presets import index_only_page_memo
from test_gpu_parity import (TOL, compare_snapshots, inputs, run_oracle, to_dev,
                             _compare_gradients, _reference_gradients)

pytestmark = pytest.mark.gpu
BF16 = torch.bfloat16


def sdpa_fp32(q, k, v, causal=True, window_size=(-1, 0)):
    """The reference adapter's three SDPA modes (flash_attention.py:16-37) in fp32."""
    query, key, value = (t.float().transpose(1, 2).contiguous() for t in (q, k, v))
    tq, tk = q.shape[1], k.shape[1]
    if tq == tk:
        out = F.scaled_dot_product_attention(query, key, value, is_causal=True)
    elif tq == 1:
        out = F.scaled_dot_product_attention(query, key, value)
    else:
        rows = tk - tq + torch.arange(tq, device=q.device)
        allowed = torch.arange(tk, device=q.device)[None, :] <= rows[:, None]
        out = F.scaled_dot_product_attention(query, key, value, attn_mask=allowed)
    return out.transpose(1, 2).to(q.dtype)


class Recorder:
    """A plugin that records (Tq, Tk, batch) of every call."""

    def __init__(self, fn):
        self.fn = fn
        self.calls = []

    def flash_attn_func(self, q, k, v, causal=True, window_size=(-1, 0)):
        self.calls.append((q.shape[1], k.shape[1], q.shape[0]))
        return self.fn(q, k, v, causal=causal, window_size=window_size)


def stream_calls(splits, config):
    """(Tq, Tk, 1) of the reference's plugin calls for a sequence of calls."""
    calls, pos = [], 0
    for width in splits:
        for start, w in schedule.chunks(pos, width, config):      # absolute starts
            calls.append((w, schedule.local_len_at(start, config) + w, 1))
        pos += width
    return calls


@pytest.mark.parametrize("kind", ["own", "sdpa_fp32"])
def test_plugin_streaming_matches_oracle(device, kind):
    """Prefill in two calls, then decode across a seal and several refreshes,
    every local attention from the plugin."""
    heads, width = 2, 64
    xs, fa, fb = inputs(2400, heads, width, seed=61, unit_raw_k=True)
    splits = [1000, 1250] + [1] * 150
    plugin = Recorder(flash_attn_func if kind == "own" else sdpa_fp32)
    print(f"streaming plugin {kind}", flush=True)
    from tao_attention import tao_attention_decode, tao_attention_prefill
    state = new_state(1, index_only_page_memo())
    q, k, v, rq, rk = to_dev(xs, device)
    outs, start = [], 0
    for w in splits:
        sl = slice(start, start + w)
        fn = tao_attention_decode if w == 1 else tao_attention_prefill
        out, state = fn(q[:, sl], k[:, sl], v[:, sl], raw_q=rq[:, sl], raw_k=rk[:, sl],
                        fusion_a=fa.to(device), fusion_b=fb.to(device), alpha=0.5,
                        state=state, position=state.get_pos(), local_flash=plugin)
        outs.append(out.clone())
        start += w
    ora, ref = run_oracle(1, xs, fa, fb, splits,
                          geometry=O.Geometry.from_config(index_only_page_memo()))
    assert plugin.calls == stream_calls(splits, state.config)
    torch.testing.assert_close(torch.cat(outs, 1).cpu().float(), ref.float(), **TOL)
    compare_snapshots(state.export(), ora.export())


@pytest.mark.parametrize("tokens,index_only", [(2304, False), (2100, True)])
def test_plugin_full_sequence_forward_matches_oracle(tokens, index_only):
    """tao_attention with a plugin: 2304 tokens take the reference's three
    calls (first tile, second tile, the batched later tiles), 2100 tokens
    one call per tile; outputs within the bf16 tolerance of the oracle."""
    heads, width = 2, 64
    xs, fa, fb = inputs(tokens, heads, width, seed=62)
    cfg = TaoConfig(coarse_index_only=index_only)
    plugin = Recorder(flash_attn_func)
    print(f"full-sequence plugin T{tokens}", flush=True)
    q, k, v, rq, rk = to_dev(xs, "cuda")
    out = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.cuda(), fusion_b=fb.cuda(),
                        alpha=0.5, config=cfg, local_flash=plugin)
    if tokens % 256 == 0:
        assert plugin.calls == [(256, 256, 1), (256, 512, 1), (256, 768, tokens // 256 - 2)]
    else:
        assert plugin.calls == [(min(256, tokens - s), min(tokens, s + 256) - max(0, s - 512), 1)
                                for s in range(0, tokens, 256)]
    ref = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg))
    torch.testing.assert_close(out.cpu().float(), ref.float(), **TOL)
    own = tao_attention(q, k, v, raw_q=rq, raw_k=rk, fusion_a=fa.cuda(), fusion_b=fb.cuda(),
                        alpha=0.5, config=cfg)
    assert torch.equal(own, out)


def test_plugin_full_sequence_backward_matches_oracle():
    """Gradients through a differentiable foreign plugin (fp32 SDPA): autograd
    carries the HIP backward's d local through the plugin, and adds the
    writer's share of d v; all seven gradients against fp64 autograd."""
    heads, width, tokens = 2, 64, 2304
    xs, fa, fb = inputs(tokens, heads, width, seed=63)
    cfg = TaoConfig()
    grad = torch.randn(xs[0].shape, generator=torch.Generator().manual_seed(64)).to(BF16)
    dev = [x.cuda().requires_grad_(True) for x in xs]
    fa_d = fa.cuda().requires_grad_(True)
    fb_d = fb.cuda().requires_grad_(True)
    plugin = SimpleNamespace(flash_attn_func=sdpa_fp32)
    print("full-sequence plugin backward", flush=True)
    out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa_d, fusion_b=fb_d,
                        alpha=0.5, config=cfg, local_flash=plugin)
    got = torch.autograd.grad(out, dev + [fa_d, fb_d], grad.cuda())
    _, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                   return_routes=True)
    want = _reference_gradients(xs, fa, fb, grad, cfg, routes)
    _compare_gradients(got, want, 5e-2)
