"""Per-request, per-layer streaming state on the device (HIP path).

Mirrors the reference StreamCache (tao_stream.py:790-1094) and the LayerState
it owns (tao_stream.py:126-527): same constructor, cursor, next_chunk,
export/from_export schema, reset and release_execution. The storage is laid
out for MI355X instead of rebuilt per seal:

* the exact-local window is a token ring [B, serve_limit, H, D] (K, V, raw K)
  indexed by position % serve_limit, replacing three torch.cat per call
  (tao_stream.py:927-930) and the clone at each seal (:965-967);
* fine memories live in a capacity-backed bank [B, H, S_cap, D, D] written in
  place by the writer kernel, replacing the per-seal repack (:455-462); each
  slot holds C^T (d contiguous) so every reader contracts over contiguous
  memory; export/import transpose to and from the reference's C;
* page descriptors, segment weights r(exp(r(z - page_z))) and page weights
  r(softmax over pages) are updated once per seal by the epilogue kernel:
  this is the reference's page-normalisation memo (:399-416), kept valid
  across the whole seal epoch for every call shape;
* with the coarse value branch (coarse_index_only=False) each completed
  page's value matrix (:486-499) is kept in a page bank [B, H, P_cap, D, D]
  (C^T) and the coarse read of every completed page is folded into one
  fp32 D x D matrix per head at each page completion (:299-305).
Every count (local length, fines, pages, route turns) is a closed form of the
cursor (schedule.py), so no device-to-host synchronisation is needed.
"""

import contextlib
import ctypes
import itertools
import math
import os

import numpy as np
import torch

from . import _hip, diagnostics, schedule
from .config import TaoConfig

DEFAULT_CONFIG = TaoConfig()
_QTILE = 256
_STATS_CAP = 8          # blocks per statistics pass of the regularized writer
# Fine writers the stream implements: the softmax writer and the regularized
# association writer (same z and read, association value matrices).
_STREAM_WRITERS = ("softmax", "regularized_association", "feature_mass_association",
                   "structured_gram_association")
# Writers whose descriptors are log feature masses and whose read is the
# numerator-only mixture (tao_stream.py:56-65, 280-283, 362-367).
_FEATURE_WRITERS = {"feature_mass_association": 1, "structured_gram_association": 2}
# Process-wide serial numbers for buffer generations and native drivers: a
# reset state reallocates its buffers and reopens its driver, and neither the
# new handle's address nor a per-state counter is guaranteed to differ from
# the old one's, so a batch keys its binding on these instead.
_SERIAL = itertools.count(1)


def _zeroed_views(device, specs):
    """Zero-filled device buffers for specs [(shape, dtype) or None], carved
    at 256-byte offsets out of one allocation, so a new state issues one fill
    kernel instead of one per buffer (prefill latency). None stays None."""
    offsets, total = [], 0
    for spec in specs:
        if spec is None:
            offsets.append(None)
            continue
        shape, dtype = spec
        nbytes = math.prod(shape) * dtype.itemsize
        offsets.append((total, nbytes))
        total += (nbytes + 255) // 256 * 256
    arena = torch.zeros(max(total, 256), dtype=torch.uint8, device=device)
    views = []
    for spec, off in zip(specs, offsets):
        if spec is None:
            views.append(None)
        else:
            views.append(arena[off[0]:off[0] + off[1]].view(spec[1]).view(spec[0]))
    return views


class _DeviceState:
    """Device buffers of one state and the C-ABI view of them."""

    def __init__(self, config, batch, heads, head_dim, device, fine_cap, plan_words=4096):
        self.config = config
        self.B, self.H, self.D = batch, heads, head_dim
        self.device = device
        self.L = config.serve_limit
        bf16, f32 = torch.bfloat16, torch.float32
        shape = (batch, self.L, heads, head_dim)
        dd = (batch, heads, head_dim, head_dim)
        self.coarse_values = not config.coarse_index_only
        self.page_c = None
        # Regularized association writer: the pending page's fp32 statistic
        # sums (the reference's pending_gram / pending_cross) and scratch for
        # the statistics of up to _STATS_CAP blocks per pass; fixed size.
        self.association = config.fine_writer == "regularized_association"
        # Feature writers: per sealed fine, the fp32 feature-mass total of
        # its run through it (the reference's pending_mass after that seal;
        # r(log) of it at a page's last fine is the page descriptor),
        # statistics scratch with a mass region, and the run's statistic
        # sums (the reference's pending gram / square mass and cross). A run
        # restarts at each page with page values and never index-only
        # (tao_stream.py:463-499).
        self.feature = _FEATURE_WRITERS.get(config.fine_writer, 0)
        self.fine_mass = None
        pending = None
        if self.association:
            pending = (dd, dd)
        elif self.feature:
            pending = (dd if self.feature == 1 else (2, batch, heads, head_dim), dd)
        # The ring, header, fold (G^T and den weights), coarse fold and
        # pending sums: fixed size, they survive capacity growth.
        (self.ring_k, self.ring_v, self.ring_raw, self.header, self.starts, self.fold_g,
         self.fold_den, self.coarse_g, self.pending_gram, self.pending_cross) = _zeroed_views(
            device, [(shape, bf16), (shape, bf16), (shape, bf16), ((4,), torch.int64),
                     ((1,), torch.int64), (dd, f32), ((batch, heads, head_dim), f32),
                     (dd, f32) if self.coarse_values else None,
                     None if pending is None else (pending[0], f32),
                     None if pending is None else (pending[1], f32)])
        self.stats = None
        if self.association:
            self.stats = torch.empty((2, _STATS_CAP * batch, heads, head_dim, head_dim),
                                     dtype=f32, device=device)
        elif self.feature:
            words = _STATS_CAP * batch * heads * head_dim
            self.stats = torch.empty(words * (2 * head_dim + 1), dtype=f32, device=device)
        self.generation = next(_SERIAL)   # renewed whenever the buffers move
        self.fine_cap = 0
        self.plan_words = max(plan_words, 4096)
        self._allocate(fine_cap, copy_fines=0)

    def _allocate(self, fine_cap, copy_fines):
        cfg = self.config
        B, H, D, dev = self.B, self.H, self.D, self.device
        bf16 = torch.bfloat16
        page_cap = fine_cap // cfg.coarse_group + 2
        sel_cap = min(512, cfg.budget(fine_cap) + 1)
        chosen_cap = page_cap
        bank = torch.empty((B, H, fine_cap, D, D), dtype=bf16, device=dev)
        page_c = (torch.empty((B, H, page_cap, D, D), dtype=bf16, device=dev)
                  if self.coarse_values else None)
        fine_z, fine_sw, page_z, page_w, sel, chosen, fine_mass = _zeroed_views(
            dev, [((B, H, fine_cap, D), bf16), ((B, H, fine_cap, D), bf16),
                  ((B, H, page_cap, D), bf16), ((B, H, page_cap, D), bf16),
                  ((B, H, sel_cap), torch.int32), ((B, H, chosen_cap), torch.int32),
                  ((B, H, fine_cap, D), torch.float32) if self.feature else None])
        if copy_fines:
            n = copy_fines
            bank[:, :, :n].copy_(self.bank[:, :, :n])
            fine_z[:, :, :n].copy_(self.fine_z[:, :, :n])
            fine_sw[:, :, :n].copy_(self.fine_sw[:, :, :n])
            pages = min(self.page_z.shape[2], page_cap)
            page_z[:, :, :pages].copy_(self.page_z[:, :, :pages])
            page_w[:, :, :pages].copy_(self.page_w[:, :, :pages])
            m = min(self.sel.shape[2], sel_cap)
            sel[:, :, :m].copy_(self.sel[:, :, :m])
            c = min(self.chosen.shape[2], chosen_cap)
            chosen[:, :, :c].copy_(self.chosen[:, :, :c])
            if page_c is not None:
                done = n // cfg.coarse_group
                page_c[:, :, :done].copy_(self.page_c[:, :, :done])
            if fine_mass is not None:
                fine_mass[:, :, :n].copy_(self.fine_mass[:, :, :n])
        self.fine_mass = fine_mass
        self.bank, self.fine_z, self.fine_sw = bank, fine_z, fine_sw
        self.page_z, self.page_w, self.sel, self.chosen = page_z, page_w, sel, chosen
        self.page_c = page_c
        self.generation = next(_SERIAL)
        self.fine_cap, self.page_cap, self.sel_cap, self.chosen_cap = (
            fine_cap, page_cap, sel_cap, chosen_cap)
        self._workspace(self.plan_words)

    def _workspace(self, plan_words):
        ws_bytes = _hip.lib().tao_workspace_bytes(self.B, self.H, self.D, self.sel_cap,
                                                  plan_words)
        self.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=self.device)
        self.generation = next(_SERIAL)
        self.plan_words = plan_words
        self.struct = self._make_struct()
        _hip.check(_hip.lib().tao_workspace_init(ctypes.byref(self.struct), self.stream()))

    def ensure_plan(self, words):
        """Grow the workspace plan region; returns True if buffers moved."""
        if words <= self.plan_words:
            return False
        self._workspace(max(words, 2 * self.plan_words))
        return True

    def _make_struct(self):
        st = _hip.StateDev()
        st.batch, st.heads, st.head_dim = self.B, self.H, self.D
        st.local_keep = self.config.local_keep
        st.fine_tokens = self.config.fine_tokens
        st.coarse_group = self.config.coarse_group
        st.fine_cap, st.page_cap = self.fine_cap, self.page_cap
        st.sel_cap, st.chosen_cap = self.sel_cap, self.chosen_cap
        st.ring_k, st.ring_v = self.ring_k.data_ptr(), self.ring_v.data_ptr()
        st.ring_raw = self.ring_raw.data_ptr()
        st.bank_c, st.fine_z = self.bank.data_ptr(), self.fine_z.data_ptr()
        st.fine_sw, st.page_z = self.fine_sw.data_ptr(), self.page_z.data_ptr()
        st.page_w, st.sel = self.page_w.data_ptr(), self.sel.data_ptr()
        st.chosen, st.header = self.chosen.data_ptr(), self.header.data_ptr()
        st.fold_g, st.fold_den = self.fold_g.data_ptr(), self.fold_den.data_ptr()
        if self.coarse_values:
            st.page_c, st.coarse_g = self.page_c.data_ptr(), self.coarse_g.data_ptr()
        if self.association:
            st.pending_gram = self.pending_gram.data_ptr()
            st.pending_cross = self.pending_cross.data_ptr()
            st.stats, st.stats_cap = self.stats.data_ptr(), _STATS_CAP
        if self.feature:
            st.fine_writer, st.fine_mass = self.feature, self.fine_mass.data_ptr()
            st.stats, st.stats_cap = self.stats.data_ptr(), _STATS_CAP
            st.pending_gram = self.pending_gram.data_ptr()
            st.pending_cross = self.pending_cross.data_ptr()
        st.workspace = self.workspace.data_ptr()
        st.workspace_bytes = self.workspace.numel()
        return st

    def stream(self):
        return _hip.stream_ptr(self.device)

    def reserve(self, fines, current):
        """Grow the bank geometrically so ``fines`` sealed fines fit."""
        if fines <= self.fine_cap:
            return False
        cap = max(self.fine_cap, 16)
        while cap < fines:
            cap *= 2
        self._allocate(cap, copy_fines=current)
        return True

    def matches(self, batch, heads, head_dim, device):
        return (self.B, self.H, self.D) == (batch, heads, head_dim) and self.device == device


class HistoryRegionGraph:
    """The decode-graph epochs of one request x layer (history_region_graph.py:10-113).

    The epochs live in the native stream driver (stream.hip), which follows
    HistoryRegionGraph.run: the non-refresh steps of one state version,
    route size and fusion parameter set form an epoch; its first three steps
    run eagerly, the fourth captures the step and replays it, later steps
    replay; a refresh copies its route ids into the epoch (or ends it when
    the route size changed), a seal ends it, and so do release_execution,
    reset and buffer growth. This object reads the driver's counters and
    keeps the reference's counts and observation() keys.

    Replays dispatch the captured step: by default the recorded kernel
    arguments (the two step kernels, state and output addresses fixed for
    the epoch, the token's operands patched in per call); with
    TAO_GRAPH_REPLAY=hipgraph in the environment a one-node hipGraph of the
    step, instantiated twice and launched alternately, its operands set per
    call (hipGraphExecKernelNodeSetParams). Both write the heads into the
    epoch's fixed output buffer, which the next replay overwrites, as the
    reference's captured outputs.
    """

    capture_address_scope = ("State banks, route buffers and the driver's output "
                             "buffer of the current state version only; the captured step "
                             "is dropped at every seal, route-size change and release")

    def __init__(self, owner):
        self._owner = owner
        self._last = [0] * _hip.GRAPH_STATS
        self._last[8] = self._last[11] = -1

    def _stats(self):
        handle = self._owner._handle
        if handle is not None:
            buf = (ctypes.c_int64 * _hip.GRAPH_STATS)()
            _hip.check(_hip.lib().tao_stream_graph_stats(handle, buf, _hip.GRAPH_STATS))
            self._last = list(buf)
        return self._last

    @property
    def counts(self):
        st = self._stats()
        names = ("epochs", "eager_warm", "captures", "replays", "id_copies", "invalidations")
        return {n: int(st[i]) for i, n in enumerate(names)}

    @property
    def reasons(self):
        st = self._stats()
        base = _hip.GRAPH_STATS - len(_hip.GRAPH_REASONS)
        return {r: int(st[base + i]) for i, r in enumerate(_hip.GRAPH_REASONS)
                if st[base + i]}

    @property
    def last_action(self):
        st = self._stats()
        action = _hip.GRAPH_ACTIONS[int(st[10])]
        if action == "invalidate":
            return "invalidate:" + _hip.GRAPH_REASONS[int(st[11])]
        return action

    @property
    def warm_count(self):
        return int(self._stats()[9])

    def observation(self):
        st = self._stats()
        return {**self.counts, "active_graph": bool(st[6]), "active_staging": bool(st[7]),
                "epoch_state_version": None if st[8] < 0 else int(st[8]),
                "epoch_warm_count": int(st[9]), "last_action": self.last_action,
                "invalidation_reasons": self.reasons,
                # Staging and output buffers are bound to the state for its
                # life (fixed addresses across epochs); the captured step of a
                # closed epoch is destroyed, so no retired execution tensors
                # exist.
                "last_retired_execution_tensors_alive": 0,
                "python_owned_semantic_tensor_references": 0,
                "capture_address_scope": self.capture_address_scope}


_GRAPH_REPLAY = {"dispatch": 1, "hipgraph": 2}


class StreamCache:
    """One request's one-layer exact-local and hierarchical history state."""

    is_tao_stream = True

    def __init__(self, layer_index, route_interval=2, fusion_mode="pointwise",
                 pending_coarse_elision=False, pending_coarse_mask=False,
                 fused_fine=True, config=DEFAULT_CONFIG):
        self.config = config
        self.history_path_ablation = False
        self.history_value_ablation = False
        self.layer_index = layer_index
        self.route_interval = route_interval
        self.fusion_mode = fusion_mode
        self.fused_fine = fused_fine
        self.pending_coarse_elision = pending_coarse_elision
        self.pending_coarse_mask = pending_coarse_mask
        self.position = 0
        self.fine_seal_events = 0
        self.fusion_pointwise_calls = 0
        self.fusion_no_history_local_returns = 0
        self.route_refreshes = 0
        self.peak_selected_fine = 0
        self.route_size = 0          # M of the current route (0: no route)
        self.route_coarse = 0
        self.history_region = None
        self._dev = None
        # Optional launch probe: probe(name) -> context manager wrapped around
        # each kernel launch (used by bench.py for live kernel timing).
        self._probe = None
        self._tok = None
        self._handle = None          # native stream driver (stream.hip)
        self._handle_serial = 0      # process-unique id of the open driver
        self._handle_dirty = True
        self._fast = None            # decode fast-path key (see decode)
        self._native = None          # native decode entry (tao_fast.cpp)
        self._fast_limit = -1
        # The regional graph serves the memo-backed index-only read only
        # (tao_stream.py:238-248). Replay mechanism: see HistoryRegionGraph.
        self._graph_mode = 0
        if (config.q1_history_region_graph and config.q1_page_normalization_memo
                and config.coarse_index_only):
            replay = os.environ.get("TAO_GRAPH_REPLAY", "dispatch")
            if replay not in _GRAPH_REPLAY:
                raise ValueError(f"TAO_GRAPH_REPLAY must be one of {sorted(_GRAPH_REPLAY)}")
            self._graph_mode = _GRAPH_REPLAY[replay]
        self._first_fine = self.config.first_fine
        self._graph_buffers = None
        self._capturing = False      # inside a WholeStepGraph capture (step_graph.py)
        self._capture_keep = []      # operands of the captured step, kept for its graph
        self._log = []               # call log of the diagnostics counters
        self._run_open = False       # the last log entry is an open one-token run
        self._info = (ctypes.c_int64 * 7)()

    # ------------------------------------------------------------------ cursor
    def get_pos(self):
        return self.position

    @property
    def state_version(self):
        return schedule.fines_at(self.position, self.config)

    def next_chunk(self, desired):
        return schedule.next_chunk(self.position, desired, self.config)

    # -------------------------------------------------------------- lifecycle
    def release_execution(self, reason="request_end"):
        """Drop the captured graph and the page memo; the semantic state stays."""
        self._log_event("release", 0)
        self._release_graph(reason)

    def _log_event(self, kind, tokens):
        """Append a call (tokens > 1) or release to the diagnostics log,
        closing an open one-token run."""
        if self._run_open:
            self._log[-1][2] = self.position - self._log[-1][1]
            self._run_open = False
        self._log.append([kind, self.position, tokens, self.route_size])

    def _open_run(self):
        self._log.append(["run", self.position, None, self.route_size])
        self._run_open = True

    def _release_graph(self, reason):
        """End the open graph epoch (HistoryRegionGraph.invalidate): the
        caller's stream is drained first, as the reference does before it
        drops captured addresses (history_region_graph.py:42-45)."""
        if self._handle is not None:
            if self._dev is not None:
                torch.cuda.current_stream(self._dev.device).synchronize()
            _hip.check(_hip.lib().tao_stream_invalidate(
                self._handle, _hip.GRAPH_REASONS.index(reason)))

    def _close_driver(self):
        if self._handle is not None:
            if self._dev is not None:
                torch.cuda.current_stream(self._dev.device).synchronize()
            if self.history_region is not None:
                self.history_region._stats()         # keep the final counters
            _hip.lib().tao_stream_close(self._handle)
            self._handle = None
            self._handle_dirty = True
            self._fast = None
            self._native = None

    def __del__(self):
        try:
            self._close_driver()
        except Exception:
            pass

    def reset(self):
        """Discard this request's state; position returns to zero."""
        self._release_graph("reset")
        self._close_driver()
        self.__init__(self.layer_index, self.route_interval, self.fusion_mode,
                      self.pending_coarse_elision, self.pending_coarse_mask,
                      self.fused_fine, self.config)

    def _check_supported(self, q):
        cfg = self.config
        if cfg.fine_writer not in _STREAM_WRITERS:
            raise NotImplementedError(
                f"the HIP streaming path implements the fine writers {_STREAM_WRITERS}")
        if cfg.fine_tokens != 256 or cfg.local_keep != 512:
            raise NotImplementedError("the HIP path implements fine_tokens=256, local_keep=512")
        if q.dtype != torch.bfloat16:
            raise TypeError("the HIP path computes on bf16 operands")
        if q.shape[-1] not in (64, 128):
            raise ValueError("head width must be 64 or 128")
        _hip.require_device(q)

    def _device_for(self, q, total_positions, plan_words=4096):
        b, _, h, d = q.shape
        fines = schedule.fines_at(total_positions, self.config)
        if self._dev is None:
            cap = 16
            while cap < fines:
                cap *= 2
            self._dev = _DeviceState(self.config, b, h, d, q.device, cap, plan_words)
        elif not self._dev.matches(b, h, d, q.device):
            raise ValueError("batch/heads/width/device must stay fixed for a state")
        elif self._dev.reserve(fines, schedule.fines_at(self.position, self.config)):
            self._release_graph("capacity")
            self._handle_dirty = True
        return self._dev

    # ----------------------------------------------------------------- kernels
    def _timed(self, name):
        return self._probe(name) if self._probe is not None else contextlib.nullcontext()

    def _route(self, dev, raw_q_row, fines):
        completed, pending = divmod(fines, self.config.coarse_group)
        coarse, _, selected = schedule.routed_counts(completed, pending, self.config)
        strides = (ctypes.c_int64 * 2)(raw_q_row.stride(0), raw_q_row.stride(1))
        with self._timed("route"):
            _hip.check(_hip.lib().tao_route(
                ctypes.byref(dev.struct), raw_q_row.data_ptr(), strides,
                completed, pending, coarse, selected, dev.stream()))
        self.route_size, self.route_coarse = selected, coarse
        self.route_refreshes += 1
        self.peak_selected_fine = max(self.peak_selected_fine, selected)

    def _seal(self, dev, tok, new_base, block_start, slot):
        dev.starts.fill_(block_start)
        with self._timed("writer"):
            _hip.check(_hip.lib().tao_write_fine(
                ctypes.byref(dev.struct), ctypes.byref(tok), new_base,
                dev.starts.data_ptr(), slot, 1, dev.stream()))
        self._epilogue(dev, slot)
        self.fine_seal_events += 1

    def _epilogue(self, dev, slot):
        with self._timed("epilogue"):
            _hip.check(_hip.lib().tao_seal_epilogue(
                ctypes.byref(dev.struct), slot, slot // self.config.coarse_group + 1, 1,
                dev.stream()))

    # ---------------------------------------------------------------- streaming
    def _stream_cfg(self):
        cfg = self.config
        return _hip.StreamCfg(self.layer_index, cfg.local_keep, cfg.fine_tokens,
                              cfg.coarse_group, cfg.route_period, cfg.layer_stagger,
                              cfg.budget_root_scale, cfg.budget_offset,
                              int(self._graph_mode))

    def _plan(self, pos0, tokens, outputs):
        """int64 plan of tao_prefill for tokens [pos0, pos0 + tokens), built by
        the library (tao_prefill_plan).

        outputs=False plans a state-only advance (no attention or reads; only
        the last refresh turn is routed, in its own epoch).
        """
        lib = _hip.lib()
        scfg = self._stream_cfg()
        info = (ctypes.c_int64 * 10)()
        args = (ctypes.byref(scfg), pos0, tokens, self.route_coarse, self.route_size,
                int(outputs))
        # One planner call when the plan fits a 64K-word guess (every prompt up
        # to about 1M tokens); a second, sized one otherwise.
        plan = np.empty(1 << 16, dtype=np.int64)
        rc = lib.tao_prefill_plan(*args, plan.ctypes.data, plan.size, info)
        if rc != 0 and not info[0] > plan.size:
            _hip.check(rc)
        if info[0] > plan.size:
            plan = np.empty(info[0], dtype=np.int64)
            _hip.check(lib.tao_prefill_plan(*args, plan.ctypes.data, info[0], info))
        plan = plan[:info[0]]
        return plan, dict(epochs=info[1], turns=info[2], route=(info[3], info[4]),
                          pool_pcap=info[5], history_chunks=info[6], chunks=info[7],
                          coarse_first=info[8], coarse_count=info[9])

    def _run_plan(self, dev, tok, fu, plan, info, local, out):
        plan_np = np.asarray(plan, dtype=np.int64)
        plan_arr = plan_np.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
        if dev.ensure_plan(len(plan)):
            self._release_graph("capacity")
            self._handle_dirty = True
        pools = _hip.PrefillPools()
        keep = []
        if info["epochs"] or info["turns"]:
            B, H, D = dev.B, dev.H, dev.D
            pcap = info["pool_pcap"]
            pw_pool = torch.empty((info["epochs"], B, H, pcap, D), dtype=torch.bfloat16,
                                  device=dev.device)
            psw_pool = torch.empty((info["epochs"], B, H, self.config.coarse_group, D),
                                   dtype=torch.bfloat16, device=dev.device)
            sel_pool = torch.empty((info["turns"] + 1, B, H, dev.sel_cap), dtype=torch.int32,
                                   device=dev.device)
            pools.pw_pool, pools.psw_pool = pw_pool.data_ptr(), psw_pool.data_ptr()
            pools.sel_pool = sel_pool.data_ptr()
            pools.pool_pcap, pools.epochs, pools.sel_slots = pcap, info["epochs"], info["turns"] + 1
            keep = [pw_pool, psw_pool, sel_pool]
            if dev.coarse_values and info["coarse_count"]:
                coarse_pool = torch.empty((info["coarse_count"], B, H, D, D),
                                          dtype=torch.bfloat16, device=dev.device)
                pools.coarse_pool = coarse_pool.data_ptr()
                pools.coarse_first = info["coarse_first"]
                pools.coarse_count = info["coarse_count"]
                keep.append(coarse_pool)
        out_s = (ctypes.c_int64 * 3)(*(_hip.strides_bth(out) if out is not None else (0, 0, 0)))
        dummy = dev.workspace.data_ptr()
        with self._timed("prefill"):
            _hip.check(_hip.lib().tao_prefill(
                ctypes.byref(dev.struct), ctypes.byref(tok), ctypes.byref(fu), plan_arr,
                len(plan), ctypes.byref(pools),
                local.data_ptr() if local is not None else dummy,
                out.data_ptr() if out is not None else dummy, out_s, dev.stream()))
        del keep      # the caching allocator keeps them stream-ordered

    def prefill(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, local_flash=None):
        """Advance by q.shape[1] tokens; returns the fused heads [B, T, H, D].

        local_flash: a caller plugin (flash_attention.caller_plugin) that
        computes the local attention of each chunk, as the reference calls it
        (tao_stream.py:919-934); the read, the fusion and the state update
        stay on the HIP path."""
        self._check_supported(q)
        if q.shape[1] == 1:
            if not self._run_open:
                self._open_run()
        else:
            self._log_event("call", q.shape[1])
        cfg = self.config
        pos0 = self.position
        tokens = q.shape[1]
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        tok = _hip.tokens(q, k, v, raw_q, raw_k)
        local = None
        if (local_flash is None and self._dev is None and pos0 == 0 and
                os.environ.get("TAO_EARLY_LOCAL", "1") != "0"):
            # A new state's first call: its window holds only the call's own
            # keys, so its local attention starts now, on the stream, and the
            # plan and the state's buffers are made while it runs.
            local = self._prompt_attention(q, tok)
        plan, info = self._plan(pos0, tokens, outputs=True)
        if local is not None:
            plan = _hip.without_attention(plan)
        dev = self._device_for(q, pos0 + tokens, plan_words=len(plan))
        if local is None and local_flash is not None:
            from .flash_attention import plugin_stream_local
            window = self._local_window()
            empty = q[:, :0]
            local = plugin_stream_local(local_flash, q, k, v,
                                        empty if window is None else window[0],
                                        empty if window is None else window[1], pos0, cfg)
            if local.shape != q.shape:
                raise ValueError("local_flash returned a local output of the wrong shape")
            plan = _hip.without_attention(plan)
        elif local is None:
            local = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
        self._run_plan(dev, tok, fu, plan, info, local, out)
        self._advance(pos0, tokens, info)
        self.fusion_pointwise_calls += info["history_chunks"]
        self.fusion_no_history_local_returns += info["chunks"] - info["history_chunks"]
        return out

    def _prompt_attention(self, q, tok):
        """Local attention of a call at position 0 without a state
        (tao_prompt_attention): every tile's keys are the call's own, and the
        tiles are those of the call's plan."""
        b, t, h, d = q.shape
        words = 3 * (2 * (t // 256) + 4)     # chunks of at most 256, two per 256 tokens
        local = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        tiles_dev = torch.empty(words, dtype=torch.int64, device=q.device)
        scfg = self._stream_cfg()
        _hip.check(_hip.lib().tao_prompt_attention(
            ctypes.byref(scfg), b, h, d, ctypes.byref(tok), 0, tiles_dev.data_ptr(), words,
            local.data_ptr(), _hip.stream_ptr(q.device)))
        return local   # tiles_dev: the caching allocator keeps it stream-ordered

    def _advance(self, pos0, tokens, info):
        cfg = self.config
        end = pos0 + tokens
        self.fine_seal_events += schedule.fines_at(end, cfg) - schedule.fines_at(pos0, cfg)
        self.route_refreshes += schedule.count_turns(pos0, end, self.layer_index, cfg)
        self.route_coarse, self.route_size = info["route"]
        self.peak_selected_fine = max(self.peak_selected_fine, self.route_size)
        self.position = end
        self._dev.header[0:1].fill_(end)
        self._handle_dirty = True
        if self._handle is not None:
            # The driver's graph epoch sees this advance now (its refreshes
            # and seal), before any later release.
            self._driver(self._dev)
        self._fold()

    def _fold(self):
        """Fold the current route under the current page weights (tao_fold_route)
        and, with the coarse value branch, the coarse read of the completed
        pages (tao_fold_coarse)."""
        fines = schedule.fines_at(self.position, self.config)
        dev = self._dev
        if dev is not None and fines > 0:
            _hip.check(_hip.lib().tao_fold_route(ctypes.byref(dev.struct), self.route_size,
                                                 dev.stream()))
            completed = fines // self.config.coarse_group
            if dev.coarse_values and completed:
                _hip.check(_hip.lib().tao_fold_coarse(ctypes.byref(dev.struct), completed,
                                                      dev.stream()))

    def _driver(self, dev):
        """Native per-token driver bound to the current buffers and cursor."""
        cfg = self.config
        if self._handle is None:
            scfg = self._stream_cfg()
            out_stage = None
            if self._graph_mode:
                out_stage = torch.empty((dev.B, 1, dev.H, dev.D), dtype=torch.bfloat16,
                                        device=dev.device)
                self._graph_buffers = (None, out_stage)
            handle = ctypes.c_void_p()
            _hip.check(_hip.lib().tao_stream_open(
                ctypes.byref(dev.struct), ctypes.byref(scfg), self.position, self.route_coarse,
                self.route_size, None,
                out_stage.data_ptr() if out_stage is not None else None, ctypes.byref(handle)))
            self._handle = handle
            self._handle_serial = next(_SERIAL)
        elif self._handle_dirty:
            _hip.check(_hip.lib().tao_stream_sync(
                self._handle, ctypes.byref(dev.struct), self.position, self.route_coarse,
                self.route_size))
        self._handle_dirty = False
        return self._handle

    def decode(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, local_flash=None):
        """One new token; returns the fused heads [B, 1, H, D].

        With a caller local_flash plugin the token runs as a one-token
        prefill whose local attention is the plugin's (the fused decode step
        computes its own local attention, so neither it nor its graph can
        take a plugin's output).

        With the graph preset a replayed step returns the epoch's output
        buffer, overwritten by the next replay (as the reference's regional
        graph returns its captured outputs); eager steps return new tensors.

        Fast path: the operand shapes, dtypes, devices and strides, the fusion
        parameter tensors and the driver binding are compared with the
        previous call's; anything different goes through the full checks.
        """
        if local_flash is not None:
            return self.prefill(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, local_flash)
        if self.config.fine_writer in _FEATURE_WRITERS:
            # The feature writers' read depends on each query (its mixture
            # over the selected fines), so there is no folded route: a token
            # runs as a one-token prefill.
            if self._capturing:
                raise NotImplementedError("device-cursor steps serve the folded-route read only")
            return self.prefill(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha)
        if self._capturing:
            return self._decode_captured(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha)
        nat = self._native
        if nat is not None and self.position < self._fast_limit and not self._handle_dirty:
            pos = self.position
            try:
                r = nat(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, pos,
                        _hip.raw_stream(self._stream_index))
            except TypeError:
                r = None
            if r is not None:
                return self._book(pos, r is True, r)
        fp = self._fast
        if (fp is not None and self.position < fp[8]
                and (q.shape, k.shape, v.shape, raw_q.shape, raw_k.shape) == fp[0]
                and (q.dtype, k.dtype, v.dtype, raw_q.dtype, raw_k.dtype,
                     q.device, k.device, v.device, raw_q.device, raw_k.device) == fp[1]
                and (q.stride(), k.stride(), v.stride(), raw_q.stride(), raw_k.stride()) == fp[2]
                and fusion_a is fp[3] and fusion_b is fp[4] and alpha == fp[5]
                and not self._handle_dirty):
            ptrs = (q.data_ptr(), k.data_ptr(), v.data_ptr(), raw_q.data_ptr(), raw_k.data_ptr())
            if not (ptrs[0] | ptrs[1] | ptrs[2] | ptrs[3] | ptrs[4]) & 15 and \
                    fusion_a.data_ptr() == fp[6] and fusion_b.data_ptr() == fp[7]:
                tok = self._tok
                tok.q, tok.k, tok.v, tok.raw_q, tok.raw_k = ptrs
                return self._decode_launch(q)
        return self._decode_slow(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha)

    def _decode_slow(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha):
        """Full argument checks, buffer growth and struct setup; then launch."""
        pos = self.position
        shape = q.shape
        if (k.shape, v.shape, raw_q.shape, raw_k.shape) != (shape, shape, shape, shape):
            raise ValueError("q, k, v, raw_q and raw_k must share one [B, 1, H, D] shape")
        for x in (k, v, raw_q, raw_k):
            if x.dtype != q.dtype or x.device != q.device:
                raise TypeError("q, k, v, raw_q and raw_k must share dtype and device")
        self._check_supported(q)
        dev = self._device_for(q, pos + 1)
        # Last cursor whose decode still fits the bank without growing.
        limit = self.config.serve_limit - 1 + dev.fine_cap * self.config.fine_tokens
        strides = (q.stride(), k.stride(), v.stride(), raw_q.stride(), raw_k.stride())
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        self._tok = _hip.tokens(q, k, v, raw_q, raw_k)
        self._tok_ref = ctypes.byref(self._tok)
        fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
        self._fu_ref = ctypes.byref(fu)
        self._fu_keep = fu
        self._driver(dev)
        # Outputs are allocated like q (empty_like keeps q's dense layout, the
        # same one for every call with q's strides).
        self._out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(torch.empty_like(q)))
        self._stream_index = q.device.index if q.device.index is not None else \
            torch.cuda.current_device()
        self._call = _hip.lib().tao_stream_decode
        # Operands used in place, and fusion parameters the kernels read in
        # place (a converted copy would freeze the parameters' values).
        fast_ok = self._tok._strides == strides and not fu.converted
        self._fast = ((shape,) * 5, (q.dtype,) * 5 + (q.device,) * 5, strides,
                      fusion_a, fusion_b, alpha, fusion_a.data_ptr(), fusion_b.data_ptr(),
                      limit) if fast_ok else None
        self._fast_limit = limit
        self._native = None
        native = _hip.fast_module()
        if fast_ok and native is not None and self._probe is None:
            try:
                self._native = native.DecodeCall(
                    q, k, v, raw_q, raw_k, fusion_a, fusion_b, float(alpha),
                    _hip.function_address("tao_stream_decode"),
                    _hip.function_address("tao_last_error"), self._handle.value,
                    ctypes.addressof(self._tok), ctypes.addressof(fu),
                    ctypes.addressof(self._info), ctypes.addressof(self._out_s))
            except TypeError:
                self._native = None
        return self._decode_launch(q)

    def _decode_launch(self, q):
        """Issue one token through the native driver and book-keep counters."""
        pos = self.position
        out = torch.empty_like(q)
        out_ptr, out_s = out.data_ptr(), self._out_s
        info = self._info
        stream = _hip.raw_stream(self._stream_index)
        if self._probe is None:
            rc = self._call(self._handle, self._tok_ref, self._fu_ref, out_ptr, out_s, stream,
                            info)
        else:
            with self._probe("decode_step"):
                rc = self._call(self._handle, self._tok_ref, self._fu_ref, out_ptr, out_s,
                                stream, info)
        if rc:
            _hip.check(rc)
        return self._book(pos, bool(info[5]), out)

    # ------------------------------------------------- caller whole-step graphs
    def device_position(self):
        """This request's cursor on the device: a 0-dim int64 view of the
        state header that every decode step advances, so code captured in
        a graph can derive per-token positions (RoPE) from it."""
        if self._dev is None:
            raise RuntimeError("the state has no device buffers yet")
        return self._dev.header[0]

    def _plan_next(self):
        """The driver's view of the next token (tao_stream_plan_step), or
        None while the driver is not bound to the current buffers."""
        if self._handle is None or self._handle_dirty:
            return None
        info = (ctypes.c_int64 * 7)()
        _hip.check(_hip.lib().tao_stream_plan_step(self._handle, info))
        return tuple(info)

    def _replayable_next(self):
        """The next token can run as a device-cursor step
        (tao_stream_graph_step): no seal after it, and either no route
        refresh before it or one that keeps the route (tao_stream_plan_step)."""
        info = self._plan_next()
        return (info is not None and info[0] == self.position and not info[2]
                and (not info[1] or info[6]))

    def _graph_key(self):
        """What a captured device-cursor step bakes in: route size, fusion
        presence flags, whether it carries the version's gated refresh (and
        then the state version, whose counts the refresh kernels take), and
        the state's device buffers."""
        info = self._plan_next()
        if not info:
            return None
        version = self.state_version if info[6] else None
        return (info[3], info[4], info[5], info[6], version, bytes(self._dev.struct))

    def _decode_captured(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha):
        """The next token's decode step with the cursor read on the device
        (tao_stream_graph_step), for a caller's stream capture; the host
        cursor moves when the caller reports the replays (_advance_replayed)."""
        shape = q.shape
        if (k.shape, v.shape, raw_q.shape, raw_k.shape) != (shape, shape, shape, shape):
            raise ValueError("q, k, v, raw_q and raw_k must share one [B, 1, H, D] shape")
        self._check_supported(q)
        if not self._replayable_next():
            raise RuntimeError("the next token seals or changes its route; decode it eagerly")
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        tok = _hip.tokens(q, k, v, raw_q, raw_k)
        fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
        out = torch.empty_like(q)
        out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
        index = q.device.index if q.device.index is not None else torch.cuda.current_device()
        _hip.check(_hip.lib().tao_stream_graph_step(
            self._handle, ctypes.byref(tok), ctypes.byref(fu), out.data_ptr(), out_s,
            _hip.raw_stream(index)))
        self._capture_keep.append((q, k, v, raw_q, raw_k, tok, fu, out_s))
        return out

    def _advance_replayed(self, count):
        """Book `count` tokens that ran as replays of a captured
        device-cursor step: driver cursor (tao_stream_advance), host cursor
        and the counters a driver call would have moved (a refresh turn
        among them ran its gated refresh on the device, keeping the route)."""
        _hip.check(_hip.lib().tao_stream_advance(self._handle, count))
        if not self._run_open:
            self._open_run()
        cfg = self.config
        for _ in range(count):
            if self.position >= self._first_fine:
                self.fusion_pointwise_calls += 1
                if schedule.is_turn(self.position, self.layer_index, cfg):
                    self.route_refreshes += 1
                    self.peak_selected_fine = max(self.peak_selected_fine, self.route_size)
            else:
                self.fusion_no_history_local_returns += 1
            self.position += 1

    def _book(self, pos, staged, out):
        """Cursor and counters after one driver call (info from the driver)."""
        if not self._run_open:
            self._open_run()
        info = self._info
        self.position = pos + 1
        if pos >= self._first_fine:
            self.fusion_pointwise_calls += 1
            if info[3] or info[4]:
                self.route_coarse, self.route_size = info[1], info[2]
                if info[3]:
                    self.route_refreshes += 1
                    if info[2] > self.peak_selected_fine:
                        self.peak_selected_fine = info[2]
                if info[4]:
                    self.fine_seal_events += 1
        else:
            self.fusion_no_history_local_returns += 1
            if info[4]:
                self.fine_seal_events += 1
        if self._graph_mode and pos >= self._first_fine and self.history_region is None:
            self.history_region = HistoryRegionGraph(self)
        if staged:
            return self._graph_buffers[1]
        return out

    def _launch_prompt_kernels(self, q, k, v, raw_q, raw_k):
        """Launch only the prompt's local attention and writer kernels.

        Measurement helper (bench.py): the launches are wrapped in the probe
        as "local_attention" and "writer"; the cursor does not move.
        """
        self._check_supported(q)
        pos0 = self.position
        tokens = q.shape[1]
        dev = self._device_for(q, pos0 + tokens)
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        tok = _hip.tokens(q, k, v, raw_q, raw_k)
        plan, _ = self._plan(pos0, tokens, outputs=True)
        n_attn, n_write = int(plan[1]), int(plan[2])
        base = _hip.PLAN_HEADER
        tiles = torch.from_numpy(plan[base:base + 3 * n_attn].copy()).to(q.device)
        starts = torch.from_numpy(plan[base + 3 * n_attn:base + 3 * n_attn + max(n_write, 1)]
                                  .copy()).to(q.device)
        local = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
        lib = _hip.lib()
        with self._timed("local_attention"):
            _hip.check(lib.tao_local_attention(
                ctypes.byref(dev.struct), ctypes.byref(tok), pos0, pos0, tiles.data_ptr(),
                n_attn, local.data_ptr(), dev.stream()))
        with self._timed("writer"):
            _hip.check(lib.tao_write_fine(
                ctypes.byref(dev.struct), ctypes.byref(tok), pos0, starts.data_ptr(),
                int(plan[3]), n_write, dev.stream()))
        return local

    def _ingest(self, q, k, v, raw_q, raw_k):
        """Advance the state by q.shape[1] tokens without computing outputs.

        The resulting state equals prefill()'s: the banks depend only on raw_k
        and v (every seal goes to the writer in one launch), page and epoch
        bookkeeping is batched, and the route of the last refresh turn is
        recomputed in its own seal epoch from that turn's anchor query.
        """
        self._check_supported(q)
        pos0 = self.position
        tokens = q.shape[1]
        self._log_event("call", tokens)
        dev = self._device_for(q, pos0 + tokens)
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        tok = _hip.tokens(q, k, v, raw_q, raw_k)
        plan, info = self._plan(pos0, tokens, outputs=False)
        fu = _hip.fusion(torch.zeros(1, device=q.device), torch.zeros(1, device=q.device),
                         0.0, False, False)
        self._run_plan(dev, tok, fu, plan, info, None, None)
        self._advance(pos0, tokens, info)

    # ---------------------------------------------------------------- snapshot
    def _local_window(self):
        dev = self._dev
        n = schedule.local_len_at(self.position, self.config)
        if dev is None or n == 0:
            return None
        slots = torch.arange(self.position - n, self.position, device=dev.device) % dev.L
        return tuple(buf.index_select(1, slots) for buf in (dev.ring_k, dev.ring_v, dev.ring_raw))

    def export(self):
        """Owned tensors in the reference snapshot schema (tao_stream.py:853-877)."""
        cfg = self.config
        dev = self._dev
        fines = schedule.fines_at(self.position, cfg)
        group = cfg.coarse_group
        completed, pending = divmod(fines, group)
        route_ids = None
        if dev is not None and self.route_size:
            chosen = dev.chosen[:, :, :self.route_coarse].to(torch.int64).unsqueeze(1).clone()
            selected = dev.sel[:, :, :self.route_size].to(torch.int64).unsqueeze(1).clone()
            route_ids = (chosen, selected)
        pages, pending_z = [], []
        packed = None
        if fines:
            # The bank stores C^T[e][d]; the snapshot keeps the reference's C[d][e].
            packed = dev.bank[:, :, :fines].transpose(-1, -2).contiguous()
            for i in range(completed):
                pc = (dev.page_c[:, :, i].transpose(-1, -2).contiguous()
                      if dev.coarse_values else None)
                pages.append((dev.page_z[:, :, i].clone(), pc,
                              dev.fine_z[:, :, i * group:(i + 1) * group].clone()))
            for j in range(pending):
                pending_z.append(dev.fine_z[:, :, completed * group + j].clone())
        local = self._local_window()
        # The regularized writer's pending statistics (fp32 [B, H, D, D]):
        # None until the first seal and, with page values, after each page
        # completion, as the reference keeps them (tao_stream.py:463-499).
        pending_gram = pending_cross = pending_mass = pending_square = None
        held = (dev is not None and fines and (pending or not dev.coarse_values))
        if held and (dev.association or dev.feature == 1):
            pending_gram = dev.pending_gram.clone()
        if held and (dev.association or dev.feature):
            pending_cross = dev.pending_cross.clone()
        # Feature writers: the run's summed mass, in seal order (the
        # reference's pending_mass), and the structured writer's square mass.
        if held and dev.feature:
            pending_mass = dev.fine_mass[:, :, fines - 1].clone()
        if held and dev.feature == 2:
            pending_square = dev.pending_gram[0].clone()
        return {
            "layer_index": self.layer_index,
            "config": cfg.export(),
            "route_interval": self.route_interval,
            "fusion_mode": self.fusion_mode,
            "fused_fine": self.fused_fine,
            "position": self.position,
            "local": None if local is None else tuple(t.clone() for t in local),
            "packed_fine_c": packed,
            "pages": pages,
            "pending_z": pending_z,
            "pending_square_mass": pending_square,
            "pending_mass": pending_mass,
            "pending_gram": pending_gram,
            "pending_cross": pending_cross,
            "route_ids": route_ids,
            "route_key": None,
            "state_version": fines,
            "route_refreshes": self.route_refreshes,
            "fine_seal_events": self.fine_seal_events,
        }

    @classmethod
    def from_export(cls, saved):
        """Restore an independent state (tao_stream.py:879-912).

        Accepts this build's snapshots and the reference's (the same schema),
        also after torch.save / torch.load(weights_only=True). A snapshot
        whose tensors are on the host is restored onto the current device.
        """
        config = TaoConfig(**saved["config"])
        state = cls(saved["layer_index"], saved["route_interval"], saved["fusion_mode"],
                    fused_fine=saved["fused_fine"], config=config)
        position = saved["position"]
        local = saved["local"]
        packed = saved["packed_fine_c"]
        pages, pending_z = saved["pages"], saved["pending_z"]
        if local is not None and local[0].device.type == "cpu":
            device = torch.device("cuda", torch.cuda.current_device())
            move = lambda t: None if t is None else t.to(device)
            local = tuple(move(t) for t in local)
            packed = move(packed)
            pages = [(move(pz), move(pc), move(fz)) for pz, pc, fz in pages]
            pending_z = [move(z) for z in pending_z]
        pending_stats = (saved.get("pending_gram"), saved.get("pending_cross"),
                         saved.get("pending_mass"), saved.get("pending_square_mass"))
        fines = len(pages) * config.coarse_group + len(pending_z)
        if fines != schedule.fines_at(position, config):
            raise ValueError("snapshot fine count does not match its position")
        sample = local[0] if local is not None else None
        if sample is None:
            state.position = position
            state.route_refreshes = saved["route_refreshes"]
            state.fine_seal_events = saved["fine_seal_events"]
            return state
        state._check_supported(sample)
        dev = state._device_for(sample, position)
        group = config.coarse_group
        n = sample.shape[1]
        if n != schedule.local_len_at(position, config):
            raise ValueError("snapshot local window does not match its position")
        slots = torch.arange(position - n, position, device=dev.device) % dev.L
        for buf, src in zip((dev.ring_k, dev.ring_v, dev.ring_raw), local):
            buf.index_copy_(1, slots, src.to(torch.bfloat16))
        if dev.feature:
            # The run's sums (tao_stream.py:463-499): present from the first
            # seal and, with page values, while the pending page has fines.
            gram, cross, mass, square = pending_stats
            first = square if dev.feature == 2 else gram
            held = fines and (not dev.coarse_values or fines % group)
            if held and (first is None or cross is None or mass is None):
                raise ValueError("feature-writer snapshot lacks its pending sums")
            if held:
                # fine_mass holds the run's total at its last fine: the page
                # (and pending) descriptors of later seals continue from it.
                f32 = lambda t: t.to(dev.device, torch.float32)
                dev.fine_mass[:, :, fines - 1].copy_(f32(mass))
                if dev.feature == 2:
                    dev.pending_gram[0].copy_(f32(square))
                    dev.pending_gram[1].copy_(f32(mass))
                else:
                    dev.pending_gram.copy_(f32(gram))
                dev.pending_cross.copy_(f32(cross))
            if dev.coarse_values and any(pc is None for _, pc, _ in pages):
                raise NotImplementedError(
                    "page value matrices of a feature writer cannot be rebuilt from a "
                    "snapshot without them (its page statistics are not part of the schema)")
        if dev.association:
            gram, cross = pending_stats[:2]
            if (gram is None) != (cross is None):
                raise ValueError("snapshot has only one of pending_gram / pending_cross")
            if gram is None and fines and (not dev.coarse_values or fines % group):
                raise ValueError("regularized-writer snapshot lacks its pending statistics")
            if gram is not None:
                dev.pending_gram.copy_(gram.to(dev.device, torch.float32))
                dev.pending_cross.copy_(cross.to(dev.device, torch.float32))
            if dev.coarse_values and any(pc is None for _, pc, _ in pages):
                raise NotImplementedError(
                    "page value matrices of the regularized writer cannot be rebuilt from a "
                    "snapshot without them (its page statistics are not part of the schema)")
        if fines:
            dev.bank[:, :, :fines].copy_(packed.transpose(-1, -2))
            rebuild = []
            for i, (pz, pc, fz) in enumerate(pages):
                dev.page_z[:, :, i].copy_(pz)
                dev.fine_z[:, :, i * group:(i + 1) * group].copy_(fz)
                if dev.coarse_values:
                    if pc is None:
                        rebuild.append(i)
                    else:
                        dev.page_c[:, :, i].copy_(pc.transpose(-1, -2))
            for j, z in enumerate(pending_z):
                dev.fine_z[:, :, len(pages) * group + j].copy_(z)
            # Completed pages keep their snapshot descriptors; the pending
            # summary is recomputed (it is not part of the snapshot schema).
            lib = _hip.lib()
            for i in range(len(pages)):
                _hip.check(lib.tao_seal_epilogue(
                    ctypes.byref(dev.struct), i * group + group - 1, i + 1, 0,
                    dev.stream()))
            # A snapshot without page values (written by an index-only state)
            # gets them rebuilt from its fines and descriptors.
            for i in rebuild:
                _hip.check(lib.tao_page_coarse(ctypes.byref(dev.struct), i, 1, dev.stream()))
            if pending_z:
                _hip.check(lib.tao_seal_epilogue(
                    ctypes.byref(dev.struct), fines - 1, len(pages) + 1, 1, dev.stream()))
        if saved["route_ids"] is not None:
            chosen, selected = saved["route_ids"]
            state.route_coarse = chosen.shape[-1]
            state.route_size = selected.shape[-1]
            dev.sel[:, :, :state.route_size].copy_(selected[:, 0].to(torch.int32))
            dev.chosen[:, :, :state.route_coarse].copy_(chosen[:, 0].to(torch.int32))
            dev.header[1:2].fill_(state.route_size)
        state.position = position
        dev.header[0:1].fill_(position)
        state.route_refreshes = saved["route_refreshes"]
        state.fine_seal_events = saved["fine_seal_events"]
        state._fold()
        return state

    # ------------------------------------------------------------- diagnostics
    def bytes(self):
        """The reference diagnostics (tao_stream.py:988-1094), same keys.

        Logical sizes and counters follow the reference's definitions (the
        counters from the call log, diagnostics.py). Physical sizes describe
        this build's buffers: the local window is a token ring of
        serve_limit slots, and "unique_allocated_cache_storage_bytes" sums
        the device buffers the state holds (capacity included).
        """
        cfg = self.config
        fines = schedule.fines_at(self.position, cfg)
        completed, pending = divmod(fines, cfg.coarse_group)
        dev = self._dev
        if dev is None:
            heads = width = batch = 0
        else:
            batch, heads, width = dev.B, dev.H, dev.D
        count = completed * (cfg.coarse_group + 1) + pending
        history = count * (width * width + width) * batch * heads * 2
        if cfg.coarse_index_only:
            history -= completed * width * width * batch * heads * 2
        local_tokens = schedule.local_len_at(self.position, cfg)
        log = [tuple(e) for e in self._log]
        c = diagnostics.counters(cfg, self.layer_index, batch, heads, width, log, self.position)
        memo = diagnostics.memo_bytes(c.memo, completed, pending, batch, heads, width)
        route_bytes = (8 * batch * heads * (self.route_coarse + self.route_size)
                       if self.route_size else 0)
        logical_local = local_tokens * 2 * heads * width * 2 * batch
        # The writer's pending sums (fp32 gram, cross, feature mass and
        # square mass), counted while the reference holds them
        # (tao_stream.py:463-499, 514-516; the rule export follows).
        parts = diagnostics.pending_writer_parts(batch, heads, width, cfg)
        held = bool(diagnostics.pending_present(fines, cfg))
        pending_writer = sum(parts.values()) if held else 0
        pending_cross = parts["cross"] if held else 0
        pending_square = parts["square"] if held else 0
        pending_mass = parts["mass"] if held else 0
        physical_local = 0
        unique = 0
        if dev is not None:
            physical_local = sum(t.numel() * t.element_size()
                                 for t in (dev.ring_k, dev.ring_v, dev.ring_raw))
            unique = sum(t.numel() * t.element_size() for t in (
                dev.ring_k, dev.ring_v, dev.ring_raw, dev.bank, dev.fine_z, dev.fine_sw,
                dev.page_z, dev.page_w, dev.sel, dev.chosen, dev.header, dev.fold_g,
                dev.fold_den, dev.workspace) if t is not None)
            unique += sum(t.numel() * t.element_size()
                          for t in (dev.page_c, dev.coarse_g, dev.pending_gram,
                                    dev.pending_cross, dev.stats) if t is not None)
        return {"history_bytes": history,
                "page_normalization_memo_bytes": memo,
                "pending_writer_bytes": pending_writer,
                "pending_gram_cross_bytes": pending_writer - pending_mass - pending_square,
                "pending_cross_bytes": pending_cross,
                "pending_square_mass_bytes": pending_square,
                "pending_feature_mass_bytes": pending_mass,
                "fused_fine": self.fused_fine,
                "fused_fine_calls": c.fused_fine_calls if self.fused_fine else 0,
                "fusion_mode": self.fusion_mode,
                "fusion_pointwise_calls": self.fusion_pointwise_calls,
                "fusion_no_history_local_returns": self.fusion_no_history_local_returns,
                "fusion_eager_calls": 0,
                "pending_coarse_elision": self.pending_coarse_elision,
                "pending_coarse_mask": self.pending_coarse_mask,
                "pending_only_masked_coarse_calls": 0,
                "pending_only_coarse_present_query_heads": 0,
                "pending_only_fine_present_query_heads": c.pending_only_fine_present_query_heads,
                "pending_coarse_elided_query_heads": 0,
                "pending_coarse_matrix_constructions": 0,
                "pending_coarse_elision_reads": 0,
                "fine_seal_events": self.fine_seal_events,
                "route_integer_bytes": route_bytes,
                "logical_local_bf16_kv_bytes": logical_local,
                "logical_retained_bytes": history + pending_writer + logical_local,
                "physical_local_including_raw_key_bytes": physical_local,
                "allocated_cache_tensor_bytes": (history + pending_writer + physical_local
                                                 + route_bytes + memo),
                "unique_allocated_cache_storage_bytes": unique,
                "local_length_tokens": local_tokens,
                "completed_coarse_pages": completed,
                "pending_fine_states": pending,
                "selected_fine_per_layer": [self.route_size],
                "peak_selected_fine_per_layer": [self.peak_selected_fine],
                "route_refreshes_per_layer": [self.route_refreshes],
                "peak_local_length_tokens": c.peak_local_length_tokens,
                "peak_logical_cache_bytes": c.peak_logical_cache_bytes,
                "peak_physical_cache_tensor_bytes": c.peak_physical_cache_tensor_bytes,
                "coarse_matrix_contractions": c.coarse_matrix_contractions,
                "fine_matrix_contractions": c.fine_matrix_contractions,
                "fine_candidate_scores": c.fine_candidate_scores,
                "route_query_heads": c.route_query_heads,
                "route_selection_calls": c.route_selection_calls,
                "fine_matrix_repack_bytes": 0}


class DecodeBatch:
    """Native batched decode over independent one-request states of one
    layer (tao_batch_*): one new token per state per call, the per-request
    route refreshes and seals as each cursor requires, and one decode step
    launch pair for all. No reference counterpart: the reference decodes one
    request per call (tao_attention_decode); the results are the same.
    """

    def __init__(self, states):
        self.states = list(states)
        self._handle = None
        self._table = None
        self._key = None
        self._gens = None
        self._info = (ctypes.c_int64 * (4 * len(self.states)))()

    def close(self):
        if self._handle is not None:
            _hip.lib().tao_batch_close(self._handle)
            self._handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _bind(self, q):
        """Device state and driver of every request; (re)open or sync the
        native batch when a driver was recreated or buffers moved."""
        first = self.states[0]
        for r, st in enumerate(self.states):
            row = q[r:r + 1]
            st._check_supported(row)
            if (st.config.coarse_index_only != first.config.coarse_index_only
                    or st.config.local_keep != first.config.local_keep
                    or st.config.fine_tokens != first.config.fine_tokens
                    or st.config.coarse_group != first.config.coarse_group):
                raise ValueError("batched states must share the coarse branch and geometry")
            dev = st._device_for(row, st.position + 1)
            if dev.B != 1:
                raise ValueError("batched decode takes one-request states (batch 1)")
            st._driver(dev)
        key = tuple((id(st), st._handle_serial) for st in self.states)
        gens = tuple(st._dev.generation for st in self.states)
        lib = _hip.lib()
        stream = self.states[0]._dev.stream()
        if self._handle is None or key != self._key:
            self.close()
            nbytes = lib.tao_batch_table_bytes(len(self.states))
            self._table = torch.empty(nbytes, dtype=torch.uint8, device=q.device)
            handles = (ctypes.c_void_p * len(self.states))(
                *[st._handle.value for st in self.states])
            handle = ctypes.c_void_p()
            _hip.check(lib.tao_batch_open(handles, len(self.states), self._table.data_ptr(),
                                          nbytes, stream, ctypes.byref(handle)))
            self._handle, self._key, self._gens = handle, key, gens
        elif gens != self._gens:
            _hip.check(lib.tao_batch_sync(self._handle, stream))
            self._gens = gens
        # What the next steps may skip re-checking (_bound): the operands'
        # geometry, each state's driver and buffers, and the last position
        # whose token its bank holds without growing.
        cfg = first.config
        self._sig = (q.dtype, q.shape[2], q.shape[3], q.device)
        self._serials = tuple(st._handle_serial for st in self.states)
        self._limits = tuple(cfg.serve_limit + st._dev.fine_cap * cfg.fine_tokens - 1
                             for st in self.states)

    def _bound(self, q):
        """True when the last _bind holds for this step: the same operand
        geometry, no state re-opened, resized or advanced outside the batch
        since, and every bank large enough for this token."""
        if self._handle is None or self._sig != (q.dtype, q.shape[2], q.shape[3], q.device):
            return False
        for st, gen, serial, limit in zip(self.states, self._gens, self._serials, self._limits):
            dev = st._dev
            if (dev is None or dev.generation != gen or st._handle_serial != serial
                    or st._handle_dirty or st._handle is None or st.position + 1 > limit):
                return False
        return True

    def decode(self, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha):
        """One token for each request: operands [R, 1, H, D]; returns [R, 1, H, D]."""
        R = len(self.states)
        shape = q.shape
        if len(shape) != 4 or shape[0] != R or shape[1] != 1:
            raise ValueError("batched decode takes [len(states), 1, H, D] operands")
        if (k.shape, v.shape, raw_q.shape, raw_k.shape) != (shape, shape, shape, shape):
            raise ValueError("q, k, v, raw_q and raw_k must share one [R, 1, H, D] shape")
        for x in (k, v, raw_q, raw_k):
            if x.dtype != q.dtype or x.device != q.device:
                raise TypeError("q, k, v, raw_q and raw_k must share dtype and device")
        if len({id(st) for st in self.states}) != R:
            raise ValueError("a state appears twice in the batch")
        q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
        if not self._bound(q):
            self._bind(q)
        tok = _hip.tokens(q, k, v, raw_q, raw_k)
        fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
        out = torch.empty_like(q)
        out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
        info = self._info
        _hip.check(_hip.lib().tao_batch_decode(
            self._handle, ctypes.byref(tok), ctypes.byref(fu), out.data_ptr(), out_s,
            self.states[0]._dev.stream(), info))
        for r, st in enumerate(self.states):
            if not st._run_open:
                st._open_run()
            pos = st.position
            st.position = pos + 1
            refreshed, sealed = info[4 * r], info[4 * r + 1]
            if pos >= st._first_fine:
                st.fusion_pointwise_calls += 1
            else:
                st.fusion_no_history_local_returns += 1
            if refreshed:
                st.route_refreshes += 1
                st.peak_selected_fine = max(st.peak_selected_fine, info[4 * r + 3])
            if refreshed or sealed:
                st.route_coarse, st.route_size = info[4 * r + 2], info[4 * r + 3]
            if sealed:
                st.fine_seal_events += 1
        return out
