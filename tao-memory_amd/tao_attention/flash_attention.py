"""Causal local attention plugin slot (reference flash_attention.py:16-40).

``flash_attn.flash_attn_func(q, k, v, causal=True, window_size=(-1, 0))``
keeps the reference contract: [B, T, H, D] operands, scale 1/sqrt(D), query
rows aligned to the suffix of the keys (square -> causal, one query -> all
keys). It runs the MFMA local-attention kernel of libtao_hip.so.
"""

import ctypes
from types import SimpleNamespace

import torch

from . import _hip

USE_FA3 = False
_QTILE = 256


def _bare_state(q):
    """A state view with no ring: every key comes from the operands."""
    st = _hip.StateDev()
    b, _, h, d = q.shape
    st.batch, st.heads, st.head_dim = b, h, d
    st.local_keep, st.fine_tokens, st.coarse_group = 512, 256, 8
    dummy = q.data_ptr()
    for name in ("ring_k", "ring_v", "ring_raw", "bank_c", "fine_z", "fine_sw",
                 "page_z", "page_w", "sel", "chosen", "header", "fold_g", "fold_den",
                 "workspace"):
        setattr(st, name, dummy)
    st.workspace_bytes = _hip.lib().tao_workspace_bytes(b, h, d, 0, 0)
    return st


def flash_attn_func(q, k, v, causal=True, window_size=(-1, 0)):
    if not causal or window_size != (-1, 0):
        raise ValueError("standalone Tao supports causal full-local attention only")
    _hip.require_device(q)
    if q.dtype != torch.bfloat16 or k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise TypeError("the HIP local attention computes on bf16 operands")
    if q.shape[-1] not in (64, 128):
        raise ValueError("head width must be 64 or 128")
    tq, tk = q.shape[1], k.shape[1]
    if tq > tk:
        raise ValueError("queries must be a suffix of the keys")
    q, k, v = _hip.vector_operands(q, k, v)
    out = torch.empty(q.shape, dtype=torch.bfloat16, device=q.device)
    if tq == 0:
        return out
    st = _bare_state(q)
    tok = _hip.tokens(q, k, v, q, k)
    shift = tk - tq
    tiles = [(r, min(_QTILE, tq - r), 0) for r in range(0, tq, _QTILE)]
    tiles_dev = torch.tensor(tiles, dtype=torch.int64).to(q.device)
    _hip.check(_hip.lib().tao_local_attention(
        ctypes.byref(st), ctypes.byref(tok), shift, 0, tiles_dev.data_ptr(), len(tiles),
        out.data_ptr(), _hip.stream_ptr(q.device)))
    return out


flash_attn = SimpleNamespace(flash_attn_func=flash_attn_func)


def caller_plugin(local_flash):
    """The caller's local_flash plugin, or None for this module's own kernel
    (the default, operator.py:42-47): only a foreign plugin changes how the
    local attention is computed."""
    if local_flash is None or local_flash is flash_attn:
        return None
    if not callable(getattr(local_flash, "flash_attn_func", None)):
        raise TypeError("local_flash must provide flash_attn_func(q, k, v, causal, window_size)")
    return local_flash


def _bf16(x):
    return x if x.dtype == torch.bfloat16 and x.is_contiguous() else x.to(torch.bfloat16).contiguous()


def plugin_training_local(plugin, q, k, v, config):
    """The full-sequence local attention on a caller plugin, with the
    reference's call pattern (_local_training_corrected_4k,
    tao_stream.py:760-787): a sequence of whole 256-token tiles of at least
    three tiles is one causal call on the first tile, one suffix call of the
    second tile over 512 keys, and one batched call of every later tile over
    its 768-key window; any other length is one call per tile over its
    window [max(0, start - local_keep), end). Differentiable when the plugin
    is."""
    call = plugin.flash_attn_func
    b, total, heads, d = q.shape
    ft, keep = config.fine_tokens, config.local_keep
    window = keep + ft
    if ft != 256 or keep != 512 or total < 3 * ft or total % ft:
        parts = [call(q[:, s:min(total, s + ft)], k[:, max(0, s - keep):min(total, s + ft)],
                      v[:, max(0, s - keep):min(total, s + ft)], causal=True,
                      window_size=(-1, 0)) for s in range(0, total, ft)]
        return torch.cat(parts, 1)
    tiles = total // ft - 2
    head = [call(q[:, :ft], k[:, :ft], v[:, :ft], causal=True, window_size=(-1, 0)),
            call(q[:, ft:2 * ft], k[:, :2 * ft], v[:, :2 * ft], causal=True,
                 window_size=(-1, 0))]

    def windows(x):       # [B, T, H, D] -> [B * tiles, 768, H, D], tile t = rows [256 t, 256 t + 768)
        return x.unfold(1, window, ft).permute(0, 1, 4, 2, 3).reshape(b * tiles, window, heads, d)

    rest = call(q[:, 2 * ft:].reshape(b * tiles, ft, heads, d), windows(k), windows(v),
                causal=True, window_size=(-1, 0))
    return torch.cat(head + [rest.reshape(b, total - 2 * ft, heads, d)], 1)


def plugin_stream_local(plugin, q, k, v, window_k, window_v, pos0, config):
    """A streaming call's local attention on a caller plugin, with the
    reference's call pattern (StreamCache.process, tao_stream.py:919-934):
    the call's tokens split at next_chunk (min(rest, fine_tokens,
    serve_limit - local length)), and each chunk's queries attend to the
    retained local window plus the chunk's keys. window_k / window_v hold
    the retained window before pos0 ([B, n, H, D], n = local length at pos0).
    Returns bf16 [B, T, H, D] contiguous."""
    from . import schedule
    total = q.shape[1]
    base = pos0 - window_k.shape[1]
    keys = torch.cat((window_k, k), 1) if window_k.shape[1] else k
    vals = torch.cat((window_v, v), 1) if window_v.shape[1] else v
    parts, start = [], 0
    while start < total:
        p = pos0 + start
        width = schedule.next_chunk(p, total - start, config)
        first = p - schedule.local_len_at(p, config) - base
        end = p + width - base
        parts.append(_bf16(plugin.flash_attn_func(q[:, start:start + width], keys[:, first:end],
                                                  vals[:, first:end], causal=True,
                                                  window_size=(-1, 0))))
        start += width
    return torch.cat(parts, 1).contiguous()
