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
