"""tao_decode_step_noalloc (no reference counterpart; for callers that cannot
allocate) against tao_decode_step, through the C ABI: the same state twice
(snapshot restored twice), one token each, outputs and the advanced state
bitwise equal; two calls in a row, the second on a smaller state (fewer
heads, narrower head), so the shared static scratch holds the first call's
records when the second runs. The no-allocation call gets a state with no
workspace."""
import ctypes

import pytest
import torch

from tao_attention import StreamCache, _hip, new_state, tao_attention_prefill
from tao_attention.presets import index_only_page_memo
from test_gpu_parity import inputs, to_dev

pytestmark = pytest.mark.gpu


def _pair(device, heads, width, tokens, seed):
    """Two identical prefilled states and the next token's operands."""
    xs, fa, fb = inputs(tokens + 1, heads, width, seed)
    q, k, v, rq, rk = to_dev(xs, device)
    st = new_state(0, index_only_page_memo())
    tao_attention_prefill(q[:, :tokens], k[:, :tokens], v[:, :tokens], raw_q=rq[:, :tokens],
                          raw_k=rk[:, :tokens], fusion_a=fa.to(device), fusion_b=fb.to(device),
                          alpha=0.5, state=st, position=0)
    snap = st.export()
    a, b = StreamCache.from_export(snap), StreamCache.from_export(snap)
    tok = [x[:, tokens:tokens + 1].contiguous() for x in (q, k, v, rq, rk)]
    return a, b, tok, fa.to(device), fb.to(device)


def _step(fn, state, tok, fa, fb, no_workspace):
    dev = state._dev
    st = _hip.StateDev.from_buffer_copy(dev.struct)
    if no_workspace:
        st.workspace, st.workspace_bytes = None, 0
    t = _hip.tokens(*tok)
    fu = _hip.fusion(fa, fb, 0.5, False, True, like=tok[0])
    out = torch.empty_like(tok[0])
    out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
    _hip.check(fn(ctypes.byref(st), ctypes.byref(t), ctypes.byref(fu), state.route_size,
                  out.data_ptr(), out_s, dev.stream()))
    return out


def test_decode_step_noalloc_matches_decode_step(device):
    lib = _hip.lib()
    print("no-alloc decode step", flush=True)
    for heads, width, tokens, seed in ((8, 128, 1500, 131), (2, 64, 1300, 132)):
        a, b, tok, fa, fb = _pair(device, heads, width, tokens, seed)
        assert a.route_size > 0
        want = _step(lib.tao_decode_step, a, tok, fa, fb, False)
        got = _step(lib.tao_decode_step_noalloc, b, tok, fa, fb, True)
        assert torch.equal(got, want), (heads, width)
        for x, y in zip((a._dev.ring_k, a._dev.ring_v, a._dev.ring_raw, a._dev.header),
                        (b._dev.ring_k, b._dev.ring_v, b._dev.ring_raw, b._dev.header)):
            assert torch.equal(x, y)
        assert int(b._dev.header[0]) == tokens + 1


def test_decode_step_noalloc_rejects_oversized_state(device):
    a, _, tok, fa, fb = _pair(device, 2, 64, 800, 133)
    st = _hip.StateDev.from_buffer_copy(a._dev.struct)
    st.heads = 600          # 600 heads at D64 exceed the 4 MiB scratch; no launch happens
    t = _hip.tokens(*tok)
    fu = _hip.fusion(fa, fb, 0.5, False, True, like=tok[0])
    out = torch.empty_like(tok[0])
    out_s = (ctypes.c_int64 * 3)(*_hip.strides_bth(out))
    rc = _hip.lib().tao_decode_step_noalloc(ctypes.byref(st), ctypes.byref(t), ctypes.byref(fu),
                                            a.route_size, out.data_ptr(), out_s, a._dev.stream())
    assert rc == -2
    with pytest.raises(ValueError, match="static scratch"):
        _hip.check(rc)
