"""Functional TaoMemory attention: the reference entry points on the HIP path.

Same signatures, argument meaning and errors as the reference operator.py
(:42-138). Inputs are [batch, tokens, heads, width]; raw_q / raw_k precede
the caller's Q/K transform, q / k are the local-attention operands after it.
The streaming path is bf16 on an MI355X device with width 64 or 128.
"""

import torch  # noqa: F401

from . import training
from .config import TaoConfig
from .flash_attention import caller_plugin
from .tao_stream import StreamCache

DEFAULT_CONFIG = TaoConfig()


def tao_attention(q, k, v, *, raw_q, raw_k, fusion_a, fusion_b, alpha,
                  config=DEFAULT_CONFIG, local_flash=None):
    """Full sequence read with fresh routing at every query (operator.py:40-52).

    Forward and backward on the HIP library (training.py) for bf16
    operands; fp32 operands take the forward-only fp32 read
    (training.forward_f32: every rounding point at fp32). A caller
    local_flash plugin computes the local attention with the reference's
    tiling (tao_stream.py:760-787), on the operands' dtype, and is
    differentiated by autograd (bf16); the rest stays on the HIP path.
    """
    return training.full_sequence_read(q, k, v, raw_q, raw_k, fusion_a, fusion_b,
                                       alpha, config, local_flash=caller_plugin(local_flash))


def new_state(layer_index, config=DEFAULT_CONFIG):
    """Independent mutable per-request, per-layer inference state."""
    return StreamCache(layer_index, route_interval=2, fusion_mode="pointwise",
                       fused_fine=True, config=config)


def tao_attention_prefill(q, k, v, *, raw_q, raw_k, fusion_a, fusion_b,
                          alpha, state, position, local_flash=None):
    """Advance only the supplied new tokens; the state is updated and returned."""
    if position != state.position:
        raise ValueError("position must match this request's causal cursor")
    plugin = caller_plugin(local_flash)
    if q.shape[1] == 0:
        return q.new_empty(q.shape), state
    out = state.prefill(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, local_flash=plugin)
    return out, state


def tao_attention_decode(q, k, v, *, raw_q, raw_k, fusion_a, fusion_b,
                         alpha, state, position, local_flash=None):
    """One-token prefill; no old token projection is recomputed."""
    if q.shape[1] != 1:
        raise ValueError("decode accepts exactly one new query/key/value")
    if position != state.position:
        raise ValueError("position must match this request's causal cursor")
    plugin = caller_plugin(local_flash)
    if plugin is None:
        out = state.decode(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha)
    else:
        out = state.decode(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, local_flash=plugin)
    return out, state


_BATCHES = {}


def tao_attention_decode_batch(q, k, v, *, raw_q, raw_k, fusion_a, fusion_b, alpha, states):
    """One new token for each of len(states) independent requests of one layer.

    No reference counterpart (the reference decodes one request per
    tao_attention_decode call, operator.py:130-138); the outputs and states
    equal that loop's. q / k / v / raw_q / raw_k: [R, 1, H, D] with request r
    in batch row r; every state is a one-request state at its own cursor.
    Returns ([R, 1, H, D], states).
    """
    from .tao_stream import DecodeBatch
    states = list(states)
    if not states:
        raise ValueError("states must hold at least one request state")
    key = tuple(id(s) for s in states)
    batch = _BATCHES.get(key)
    if batch is None or any(a is not b for a, b in zip(batch.states, states)):
        batch = DecodeBatch(states)
        _BATCHES.clear()
        _BATCHES[key] = batch
    return batch.decode(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha), states
