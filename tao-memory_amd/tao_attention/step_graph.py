"""Caller-side whole-step decode graph across layers.

The reference's published model benchmark decodes a 12-layer model with one
TaoMemory state per layer (docs/benchmarks.md:15) and captures only one
layer's history region (history_region_graph.py:95-113, "not whole-model
graph capture", docs/benchmarks.md:89-94). WholeStepGraph captures a caller's
whole model step -- every layer's projections, its TaoMemory decode and the
rest of the block -- as one graph and replays it for every token that no
layer seals after and whose route refreshes keep the layers' route sizes.
Those tokens launch each layer's work with the cursor read on the device
(the state header, which the step advances): the layer's route refresh and
fold kernels exit unless the cursor is a refresh turn of that layer (the
layers' turns are staggered, tao_stream.py:202-208), then its decode step
runs. One capture thus serves every such token of a state version; seal
tokens and refreshes that change a route size run eagerly through the
layers' drivers, as do the tokens before the first capture.

The step function must take its per-token positions from the device
(StreamCache.device_position()), not from host integers, since host values
are frozen into the graph at capture. Its tensor inputs are copied into the
graph's static inputs before each replay, and replays return the graph's
static outputs, which the next replay overwrites.
"""

import torch

__all__ = ["WholeStepGraph"]


class WholeStepGraph:
    """One captured model step over the per-layer states of one request.

    states: the layers' StreamCache states, all at one cursor. Calling
    `step(fn, *inputs)` runs `fn(*inputs)` for the next token, eagerly or by
    replaying the captured step; the states' cursors advance by one either
    way. The graph is captured again whenever what a captured decode bakes
    in changes (route size, fusion presence flags, state buffers).
    """

    def __init__(self, states):
        self.states = list(states)
        if not self.states:
            raise ValueError("WholeStepGraph needs at least one layer state")
        for st in self.states:
            if st._graph_mode:
                raise ValueError("a state with the regional graph preset cannot join a "
                                 "whole-step graph")
        self._graph = None
        self._key = None
        self._pending = None
        self._static_in = None
        self._static_out = None
        self.eager_steps = 0
        self.captures = 0
        self.replays = 0

    def _position(self):
        pos = {st.position for st in self.states}
        if len(pos) != 1:
            raise ValueError("the layer states are at different cursors")
        return pos.pop()

    def release(self):
        """Drop the captured step (its graph and static buffers)."""
        if self._graph is not None:
            torch.cuda.current_stream().synchronize()
        self._graph = self._key = self._static_in = self._static_out = None
        for st in self.states:
            st._capture_keep.clear()

    def _capture(self, fn, inputs, key):
        self.release()
        self._static_in = [x.clone() for x in inputs]
        graph = torch.cuda.CUDAGraph()
        for st in self.states:
            st._capturing = True
        try:
            with torch.cuda.graph(graph):
                out = fn(*self._static_in)
        finally:
            for st in self.states:
                st._capturing = False
        self._graph, self._static_out, self._key = graph, out, key
        self.captures += 1

    def step(self, fn, *inputs):
        """The next token through fn: replayed when every layer can run it as
        a device-cursor step and the captured key still holds, eager
        otherwise (the first such token under a new key runs eagerly, the
        next captures)."""
        self._position()
        if not all(st._replayable_next() for st in self.states):
            self.eager_steps += 1
            return fn(*inputs)
        key = tuple(st._graph_key() for st in self.states)
        if key != self._key:
            if key != self._pending:
                # The first plain token under a new key runs eagerly: it warms
                # the caller's kernels; the next one captures.
                self.release()
                self._pending = key
                self.eager_steps += 1
                return fn(*inputs)
            self._capture(fn, inputs, key)
            self._pending = None
        for dst, src in zip(self._static_in, inputs):
            dst.copy_(src)
        self._graph.replay()
        for st in self.states:
            st._advance_replayed(1)
        self.replays += 1
        return self._static_out
