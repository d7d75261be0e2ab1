"""Full-sequence read: the forward of ``tao_attention`` on the HIP library.

Reference: ``tao_attention`` (operator.py:40-52) = ``read_training``
(tao_stream.py:668-757) with ``route_interval=1`` followed by
``_fuse_training`` (operator.py:21-38).

The full-sequence read is the streaming prefill of the same tokens with a
route refresh at every query: tile t (256 tokens) attends to the keys the
stream's local ring holds at that point, reads the t - 2 fines the stream
has sealed, and the fusion presence flags are the stream's. So the whole
sequence runs as ONE ``tao_prefill`` on a fresh, call-private device state,
under a plan from ``tao_train_plan``: local attention for every tile, the
writer for every visible block, page and epoch summaries, a route for every
history query (bitmask selections), then the per-query selected read with
the coarse read and the fusion in its epilogue.

Gradients (``backward``): the HIP adjoints of every step, at the forward's
values and selections; in grad mode the forward runs on a call-private
workspace and saves what the backward reads.
"""

import collections
import ctypes

import numpy as np
import torch

from . import _hip
from .config import TaoConfig


# Writers whose read is the softmax writer's (fine z and the selected read are
# unchanged; only the value matrices differ, tao_stream.py:72-74, 530-575).
_VALUE_WRITERS = ("softmax", "regularized_association")


# Writers with log-mass descriptors and the numerator-only mixture read
# (tao_stream.py:80-123, 600-662).
_FEATURE_WRITERS = ("feature_mass_association", "structured_gram_association")


def _check(q, k, v, raw_q, raw_k, config, dtype=torch.bfloat16):
    if config.fine_writer in _FEATURE_WRITERS:
        pass
    elif config.fine_writer not in _VALUE_WRITERS:
        raise NotImplementedError(
            f"the HIP full-sequence read implements the fine writers {_VALUE_WRITERS}")
    if config.fine_tokens != 256 or config.local_keep != 512 or config.coarse_group != 8:
        raise NotImplementedError(
            "the HIP path implements fine_tokens=256, local_keep=512, coarse_group=8")
    shape = q.shape
    if q.dim() != 4 or any(t.shape != shape for t in (k, v, raw_q, raw_k)):
        raise ValueError("q, k, v, raw_q and raw_k must share one [B, T, H, D] shape")
    if any(t.dtype != dtype for t in (q, k, v, raw_q, raw_k)):
        raise TypeError("the HIP full-sequence read takes five bf16 or five fp32 operands")
    if shape[-1] not in (64, 128):
        raise ValueError("head width must be 64 or 128")
    for t in (q, k, v, raw_q, raw_k):
        _hip.require_device(t)


def plan(config, tokens):
    """(int64 plan, info) of the full-sequence read of `tokens` tokens."""
    lib = _hip.lib()
    scfg = _hip.StreamCfg(0, config.local_keep, config.fine_tokens, config.coarse_group,
                          config.route_period, config.layer_stagger,
                          config.budget_root_scale, config.budget_offset, 0)
    info = (ctypes.c_int64 * 12)()
    _hip.check(lib.tao_train_plan(ctypes.byref(scfg), tokens, None, 0, info))
    words = np.empty(info[0], dtype=np.int64)
    _hip.check(lib.tao_train_plan(ctypes.byref(scfg), tokens, words.ctypes.data, info[0], info))
    keys = ("length", "epochs", "turns", "route_coarse", "route_size", "pool_pcap",
            "history_tiles", "tiles", "coarse_first", "coarse_count", "fines", "qsel_words")
    return words, dict(zip(keys, info))


class _Workspace:
    """Plan, call-private device state, pools and scratch of one shape.

    Every buffer is fully written before it is read within a call (the bank
    and page state by the writer and page kernels, the pools by the epoch and
    route kernels, qsel words of history queries by the route), so calls of
    the same shape on the same stream reuse them.
    """

    def __init__(self, config, b, tokens, heads, d, device):
        from .tao_stream import _DeviceState

        self.plan, self.info = plan(config, tokens)
        info = self.info
        self.plan_arr = self.plan.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
        # The same plan without its local attention (local from a plugin).
        self.plan_ext = _hip.without_attention(self.plan)
        self.plan_ext_arr = self.plan_ext.ctypes.data_as(ctypes.POINTER(ctypes.c_int64))
        self.dev = _DeviceState(config, b, heads, d, device, max(info["fines"], 8))
        self.dev.ensure_plan(len(self.plan))
        self.local = torch.empty((b, tokens, heads, d), dtype=torch.bfloat16, device=device)
        self.pools = _hip.PrefillPools()
        self.keep = []
        self.qsel = None
        if info["epochs"]:
            pcap = info["pool_pcap"]
            pw_pool = torch.empty((info["epochs"], b, heads, pcap, d), dtype=torch.bfloat16,
                                  device=device)
            psw_pool = torch.empty((info["epochs"], b, heads, config.coarse_group, d),
                                   dtype=torch.bfloat16, device=device)
            self.qsel = torch.zeros((b, tokens, heads, info["qsel_words"]), dtype=torch.int32,
                                    device=device)
            pools = self.pools
            pools.pw_pool, pools.psw_pool = pw_pool.data_ptr(), psw_pool.data_ptr()
            pools.pool_pcap, pools.epochs = pcap, info["epochs"]
            pools.qsel, pools.qsel_words = self.qsel.data_ptr(), info["qsel_words"]
            self.keep = [pw_pool, psw_pool]
            if self.dev.coarse_values and info["coarse_count"]:
                coarse_pool = torch.empty((info["coarse_count"], b, heads, d, d),
                                          dtype=torch.bfloat16, device=device)
                pools.coarse_pool = coarse_pool.data_ptr()
                pools.coarse_first = info["coarse_first"]
                pools.coarse_count = info["coarse_count"]
                self.keep.append(coarse_pool)


_WORKSPACES = collections.OrderedDict()
_MAX_WORKSPACES = 4


def _workspace(config, b, tokens, heads, d, device):
    key = (config, b, tokens, heads, d, device, _hip.stream_ptr(device))
    ws = _WORKSPACES.get(key)
    if ws is None:
        ws = _WORKSPACES[key] = _Workspace(config, b, tokens, heads, d, device)
        while len(_WORKSPACES) > _MAX_WORKSPACES:
            _WORKSPACES.popitem(last=False)
    else:
        _WORKSPACES.move_to_end(key)
    return ws


def _association_values(ws, raw_k, v, config):
    """The regularized association writer's value matrices of the visible
    blocks and of the completed pages (tao_stream.py:80-123, 530-575):
    C_f = association_matrix(u_f^T u_f, u_f^T v_f) per 256-token block and,
    with the coarse value branch, page C = association_matrix of the
    chronological sums of its eight fines' statistics. Written into the
    call's state in its C^T layout; the prefill then keeps them
    (pools.external_values)."""
    from .association_writer import association_matrix, association_statistics, chronological_sum

    fines = ws.info["fines"]
    dev = ws.dev
    ws.pools.external_values = 1
    if not fines:
        return
    group = config.coarse_group
    pages = fines // group if dev.coarse_values else 0
    span = fines * config.fine_tokens
    with torch.no_grad():
        for bi in range(raw_k.shape[0]):
            kb = raw_k[bi, :span].unflatten(0, (fines, config.fine_tokens))
            vb = v[bi, :span].unflatten(0, (fines, config.fine_tokens))
            gram, cross = association_statistics(kb, vb)                # [S, H, D, D]
            dev.bank[bi, :, :fines] = association_matrix(gram, cross).permute(1, 0, 3, 2)
            if pages:
                def page_sum(t):
                    t = t[:pages * group].unflatten(0, (pages, group))   # [P, 8, H, D, D]
                    return chronological_sum(t.transpose(1, 2))          # [P, H, D, D]
                page_c = association_matrix(page_sum(gram), page_sum(cross))
                dev.page_c[bi, :, :pages] = page_c.permute(1, 0, 3, 2)


def _run(ws, tok, fu, local, out):
    """tao_prefill of the full-sequence plan; `local` given: the caller's
    local attention output (the plan without its attention section)."""
    out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
    if local is None:
        plan_arr, plan_len, local_ptr = ws.plan_arr, len(ws.plan), ws.local.data_ptr()
    else:
        plan_arr, plan_len, local_ptr = ws.plan_ext_arr, len(ws.plan_ext), local.data_ptr()
    _hip.check(_hip.lib().tao_prefill(
        ctypes.byref(ws.dev.struct), ctypes.byref(tok), ctypes.byref(fu), plan_arr, plan_len,
        ctypes.byref(ws.pools), local_ptr, out.data_ptr(), out_s, ws.dev.stream()))


def _plugin_local(local, q):
    """A plugin's local output as the bf16 [B, T, H, D] contiguous operand."""
    if tuple(local.shape) != tuple(q.shape):
        raise ValueError("local_flash returned a local output of the wrong shape")
    return local.to(torch.bfloat16).contiguous()


def forward(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config, return_routes=False,
            local=None):
    """Fused heads [B, T, H, D] of the full-sequence read (no autograd).

    With return_routes, also the per-query selections: int32 [B, T, H, W]
    bitmask words over fine ids (bit f of word f // 32) for queries with
    history, zero before first_fine. `local`: the local attention output
    of a caller plugin, used instead of the library's.
    """
    _check(q, k, v, raw_q, raw_k, config)
    b, tokens, heads, d = q.shape
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    if tokens == 0:
        return (out, None) if return_routes else out
    ws = _workspace(config, b, tokens, heads, d, q.device)
    q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
    if config.fine_writer == "regularized_association":
        _association_values(ws, raw_k, v, config)
    tok = _hip.tokens(q, k, v, raw_q, raw_k)
    fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
    _run(ws, tok, fu, None if local is None else _plugin_local(local, q), out)
    if return_routes:
        return out, None if ws.qsel is None else ws.qsel.clone()
    return out


def forward_f32(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config, return_routes=False,
                local=None):
    """tao_attention on fp32 operands (tao_full_sequence_f32), forward only.

    The reference's torch operations follow the operand dtype
    (operator.py:21-39, tao_stream.py:668-757); here every rounding point of
    the bf16 contract rounds to fp32, with the routing sums in the bf16
    path's orders, so routes are reproducible bit for bit and the output is
    within 1e-4 of exact arithmetic. Returns fp32 [B, T, H, D] and, with
    return_routes, each query's selected fine ids in score order (int32
    [B, T, H, M_max], -1 padded). local: a caller plugin's local attention
    output (fp32 [B, T, H, D]), taken in place of the library's
    (tao_full_sequence_f32_local)."""
    if config.fine_writer != "softmax":
        raise NotImplementedError("the fp32 full-sequence read implements the softmax writer")
    _check(q, k, v, raw_q, raw_k, config, dtype=torch.float32)
    b, tokens, heads, d = q.shape
    if local is not None:
        if local.shape != q.shape or local.dtype != torch.float32 or local.device != q.device:
            raise ValueError(f"the local attention output must be fp32 {tuple(q.shape)} on "
                             f"{q.device}, got {local.dtype} {tuple(local.shape)}")
        local = local.contiguous()
    out = torch.empty(q.shape, dtype=torch.float32, device=q.device)
    sel = None
    if return_routes:
        # The last tile's route is the largest (routed counts grow with the
        # visible fines).
        from . import schedule
        tiles = -(-tokens // config.fine_tokens)
        vmax = max(0, tiles - 1 - config.visibility_tiles)
        group = config.coarse_group
        m = schedule.routed_counts(vmax // group, vmax % group, config)[2] if vmax else 1
        sel = torch.empty((b, tokens, heads, max(1, m)), dtype=torch.int32, device=q.device)
    if tokens == 0:
        return (out, sel) if return_routes else out
    ops = tuple(t if t.stride(-1) == 1 else t.contiguous() for t in (q, k, v, raw_q, raw_k))
    coarse = int(not config.coarse_index_only)
    lib = _hip.lib()
    nbytes = lib.tao_full_sequence_f32_workspace_bytes(b, heads, d, tokens, coarse)
    scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    tok = _hip.tokens(*ops)
    fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
    fu32 = _hip.Fusion.from_buffer_copy(fu)
    # gain = torch.full((), 2 * alpha, dtype=float32) (operator.py:34)
    fu32.gain = float(torch.full((), 2 * float(alpha), dtype=torch.float32))
    scfg = _hip.StreamCfg(0, config.local_keep, config.fine_tokens, config.coarse_group,
                          config.route_period, config.layer_stagger,
                          config.budget_root_scale, config.budget_offset, 0)
    out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
    tail = (out.data_ptr(), out_s, None if sel is None else sel.data_ptr(),
            0 if sel is None else sel.shape[-1], scratch.data_ptr(), nbytes,
            _hip.stream_ptr(q.device))
    head = (ctypes.byref(scfg), ctypes.byref(tok), ctypes.byref(fu32), b, heads, d, coarse)
    if local is None:
        _hip.check(lib.tao_full_sequence_f32(*head, *tail))
    else:
        _hip.check(lib.tao_full_sequence_f32_local(*head, local.data_ptr(), *tail))
    return (out, sel) if return_routes else out


def _forward_for_backward(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config,
                          local=None):
    """The forward on a call-private workspace, with the saves the backward
    reads: local-attention log2-sum-exp (not with a plugin's `local`),
    pre-fusion coarse / fine heads and denominators. Returns (out, context
    for backward)."""
    _check(q, k, v, raw_q, raw_k, config)
    b, tokens, heads, d = q.shape
    ws = _Workspace(config, b, tokens, heads, d, q.device)
    q, k, v, raw_q, raw_k = _hip.vector_operands(q, k, v, raw_q, raw_k)
    if config.fine_writer == "regularized_association":
        _association_values(ws, raw_k, v, config)
    saves = dict(
        lse=torch.empty((b, tokens, heads), dtype=torch.float32, device=q.device),
        coarse=torch.zeros(q.shape, dtype=torch.bfloat16, device=q.device),
        fine=torch.zeros(q.shape, dtype=torch.bfloat16, device=q.device),
        den=torch.zeros((b, tokens, heads), dtype=torch.float32, device=q.device))
    if local is not None:
        local = _plugin_local(local, q)
        del saves["lse"]
    else:
        ws.pools.local_lse = saves["lse"].data_ptr()
    ws.pools.coarse_out = saves["coarse"].data_ptr()
    ws.pools.fine_out = saves["fine"].data_ptr()
    ws.pools.den_out = saves["den"].data_ptr()
    tok = _hip.tokens(q, k, v, raw_q, raw_k)
    fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    _run(ws, tok, fu, local, out)
    return out, dict(ws=ws, saves=saves, operands=(q, k, v, raw_q, raw_k), local=local)


def backward(ctx_data, grad, fusion_a, fusion_b, alpha, memory_adjoints=None):
    """Gradients (dq, dk, dv, draw_q, draw_k, dfusion_a, dfusion_b) of the
    full-sequence read at the forward recorded in ctx_data. With a dict
    `memory_adjoints`, it also receives "dz" (d fine_z, fp32 [B, H, S, D]),
    "dc" (d C, fp32 [B, H, S, D, D]) of the S written fines and "dalpha"
    (fp32 [1], through gain = 2 alpha). When the forward's local attention
    came from a plugin, dq and dk are None, dk's place is taken by nothing
    and the first output is d local (bf16 [B, T, H, D]) instead of dq; dv
    is the writer's share only."""
    ws = ctx_data["ws"]
    saves = ctx_data["saves"]
    q, k, v, raw_q, raw_k = ctx_data["operands"]
    grad = grad.to(torch.bfloat16)
    if not _hip.vector_ready(grad):
        grad = grad.contiguous()
    b, tokens, heads, d = q.shape
    dev = q.device
    outs = [torch.empty((b, tokens, heads, d), dtype=torch.bfloat16, device=dev)
            for _ in range(5)]
    dfa = torch.zeros((heads, d, 3), dtype=torch.float32, device=dev)
    dfb = torch.zeros((heads, d, 3), dtype=torch.float32, device=dev)
    lib = _hip.lib()
    nbytes = lib.tao_train_bwd_workspace_bytes(ctypes.byref(ws.dev.struct), tokens,
                                               ws.info["fines"], ctypes.byref(ws.pools))
    scratch = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)
    args = _hip.TrainBwd()
    args.grad = grad.data_ptr()
    args.grad_s = _hip.i64x3(_hip.strides_bth(grad))
    plugin = ctx_data.get("local") is not None
    if plugin:
        args.local = ctx_data["local"].data_ptr()
        args.dlocal_out = outs[0].data_ptr()
    else:
        args.local = ws.local.data_ptr()
        args.local_lse = saves["lse"].data_ptr()
    args.coarse_out = saves["coarse"].data_ptr()
    args.fine_out = saves["fine"].data_ptr()
    args.den_out = saves["den"].data_ptr()
    args.dv, args.draw_q, args.draw_k = (t.data_ptr() for t in outs[2:])
    if not plugin:
        args.dq, args.dk = outs[0].data_ptr(), outs[1].data_ptr()
    args.dfusion_a, args.dfusion_b = dfa.data_ptr(), dfb.data_ptr()
    args.workspace, args.workspace_bytes = scratch.data_ptr(), nbytes
    fines = ws.info["fines"]
    if memory_adjoints is not None:
        memory_adjoints["dalpha"] = torch.zeros(1, dtype=torch.float32, device=dev)
        args.dalpha_out = memory_adjoints["dalpha"].data_ptr()
    if memory_adjoints is not None and fines:
        memory_adjoints["dz"] = torch.empty((b, heads, fines, d), dtype=torch.float32, device=dev)
        memory_adjoints["dc_t"] = torch.empty((b, heads, fines, d, d), dtype=torch.float32,
                                              device=dev)
        args.dz_out = memory_adjoints["dz"].data_ptr()
        args.dc_out = memory_adjoints["dc_t"].data_ptr()
    tok = _hip.tokens(q, k, v, raw_q, raw_k)
    fu = _hip.fusion(fusion_a, fusion_b, alpha, False, True, like=q)
    _hip.check(lib.tao_train_backward(ctypes.byref(ws.dev.struct), ctypes.byref(tok),
                                      ctypes.byref(fu), ctypes.byref(ws.pools),
                                      ctypes.byref(args), ws.dev.stream()))
    if memory_adjoints is not None and fines:
        memory_adjoints["dc"] = memory_adjoints.pop("dc_t").transpose(-1, -2)
    if plugin:
        outs[1] = None
    return (*outs, dfa, dfb)


class _FullSequenceRead(torch.autograd.Function):
    """Autograd node of the full-sequence read: HIP forward and backward."""

    @staticmethod
    def forward(ctx, q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config):
        alpha_f = float(alpha)
        out, data = _forward_for_backward(q, k, v, raw_q, raw_k, fusion_a, fusion_b,
                                          alpha_f, config)
        ctx.data = data
        ctx.alpha = alpha_f
        ctx.alpha_like = alpha if torch.is_tensor(alpha) else None
        ctx.save_for_backward(fusion_a, fusion_b)
        return out

    @staticmethod
    def backward(ctx, grad):
        fusion_a, fusion_b = ctx.saved_tensors
        need = ctx.needs_input_grad
        extra = {} if need[7] else None
        dq, dk, dv, drq, drk, dfa, dfb = backward(ctx.data, grad, fusion_a, fusion_b,
                                                  ctx.alpha, memory_adjoints=extra)
        ctx.data = None
        dalpha = None
        if need[7]:
            like = ctx.alpha_like
            # a host alpha receives its gradient without a device sync
            dalpha = extra["dalpha"].reshape(like.shape).to(like.dtype).to(
                like.device, non_blocking=True)
        return (dq if need[0] else None, dk if need[1] else None, dv if need[2] else None,
                drq if need[3] else None, drk if need[4] else None,
                dfa.to(fusion_a.dtype) if need[5] else None,
                dfb.to(fusion_b.dtype) if need[6] else None, dalpha, None)


class _FullSequenceReadLocal(torch.autograd.Function):
    """Autograd node of the full-sequence read whose local attention a caller
    plugin computed: inputs (local, v, raw_q, raw_k, fusion_a, fusion_b,
    alpha); q and k ride along for the operand layout only. The backward
    returns d local (autograd carries it through the plugin) and the
    writer's share of d v."""

    @staticmethod
    def forward(ctx, local, v, raw_q, raw_k, fusion_a, fusion_b, alpha, q, k, config):
        alpha_f = float(alpha)
        out, data = _forward_for_backward(q, k, v, raw_q, raw_k, fusion_a, fusion_b,
                                          alpha_f, config, local=local)
        ctx.data = data
        ctx.alpha_like = alpha if torch.is_tensor(alpha) else None
        ctx.alpha = alpha_f
        ctx.save_for_backward(fusion_a, fusion_b)
        return out

    @staticmethod
    def backward(ctx, grad):
        fusion_a, fusion_b = ctx.saved_tensors
        need = ctx.needs_input_grad
        extra = {} if need[6] else None
        dlocal, _, dv, drq, drk, dfa, dfb = backward(ctx.data, grad, fusion_a, fusion_b,
                                                     ctx.alpha, memory_adjoints=extra)
        ctx.data = None
        dalpha = None
        if need[6]:
            like = ctx.alpha_like
            dalpha = extra["dalpha"].reshape(like.shape).to(like.dtype).to(
                like.device, non_blocking=True)
        return (dlocal if need[0] else None, dv if need[1] else None,
                drq if need[2] else None, drk if need[3] else None,
                dfa.to(fusion_a.dtype) if need[4] else None,
                dfb.to(fusion_b.dtype) if need[5] else None, dalpha, None, None, None)


def full_sequence_read(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha,
                       config=None, local_flash=None):
    """tao_attention's read and fusion. alpha is a Python float, as in the
    reference, or a 0-dim tensor; a tensor that requires grad receives
    d alpha through gain = 2 alpha (the reference has no such gradient). The
    kernels take alpha as a host scalar, so a device tensor costs one
    synchronisation per call; a host tensor costs none. local_flash: a
    caller plugin (flash_attention.caller_plugin) for the local attention."""
    config = config or TaoConfig()
    tensors = (q, k, v, raw_q, raw_k, fusion_a, fusion_b)
    alpha_grad = torch.is_tensor(alpha) and alpha.requires_grad
    grad = torch.is_grad_enabled() and (alpha_grad or any(t.requires_grad for t in tensors))
    if q.dtype == torch.float32:
        if grad:
            raise NotImplementedError(
                "the fp32 full-sequence read is forward-only: run it under torch.no_grad() "
                "or on bf16 operands for gradients")
        local = None
        if local_flash is not None:
            from .flash_attention import plugin_training_local
            _check(q, k, v, raw_q, raw_k, config, dtype=torch.float32)
            local = plugin_training_local(local_flash, q, k, v, config)
        return forward_f32(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config, local=local)
    if local_flash is not None:
        from .flash_attention import plugin_training_local
        _check(q, k, v, raw_q, raw_k, config)
        local = plugin_training_local(local_flash, q, k, v, config)
        if grad or local.requires_grad:
            return _FullSequenceReadLocal.apply(local, v, raw_q, raw_k, fusion_a, fusion_b,
                                                alpha, q.detach(), k.detach(), config)
        return forward(q, k, v, raw_q, raw_k, fusion_a, fusion_b, float(alpha), config,
                       local=local)
    if grad:
        return _FullSequenceRead.apply(q, k, v, raw_q, raw_k, fusion_a, fusion_b, alpha, config)
    return forward(q, k, v, raw_q, raw_k, fusion_a, fusion_b, float(alpha), config)
