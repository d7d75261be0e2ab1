"""ctypes binding of libtao_hip.so (C ABI: include/tao_memory.h).

The library must be built (``python tao-memory_amd/build.py``) and torch must
be imported first so the library binds to torch's HIP runtime and can use
torch's streams and allocations. There is no fallback: a missing library or
device raises immediately.
"""

import ctypes
import os

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libtao_hip.so")
_lib = None

TAO_BF16 = 0
TAO_FP32 = 1
TAO_FP16 = 2
_PARAM_DTYPES = {torch.bfloat16: TAO_BF16, torch.float32: TAO_FP32, torch.float16: TAO_FP16}

_i32, _i64, _sz, _vp = ctypes.c_int32, ctypes.c_int64, ctypes.c_size_t, ctypes.c_void_p
_I64x3 = ctypes.c_int64 * 3


class StateDev(ctypes.Structure):
    _fields_ = [
        ("batch", _i32), ("heads", _i32), ("head_dim", _i32),
        ("local_keep", _i32), ("fine_tokens", _i32), ("coarse_group", _i32),
        ("fine_cap", _i32), ("page_cap", _i32), ("sel_cap", _i32), ("chosen_cap", _i32),
        ("ring_k", _vp), ("ring_v", _vp), ("ring_raw", _vp),
        ("bank_c", _vp), ("fine_z", _vp), ("fine_sw", _vp),
        ("page_z", _vp), ("page_w", _vp),
        ("sel", _vp), ("chosen", _vp), ("header", _vp),
        ("fold_g", _vp), ("fold_den", _vp),
        ("page_c", _vp), ("coarse_g", _vp),
        ("workspace", _vp), ("workspace_bytes", _sz),
        ("pending_gram", _vp), ("pending_cross", _vp), ("stats", _vp), ("stats_cap", _i32),
        ("fine_writer", _i32), ("fine_mass", _vp),
    ]


class Tokens(ctypes.Structure):
    _fields_ = [
        ("q", _vp), ("k", _vp), ("v", _vp), ("raw_q", _vp), ("raw_k", _vp),
        ("q_s", _I64x3), ("k_s", _I64x3), ("v_s", _I64x3), ("rq_s", _I64x3), ("rk_s", _I64x3),
        ("tokens", _i32),
    ]


class PrefillPools(ctypes.Structure):
    _fields_ = [("pw_pool", _vp), ("psw_pool", _vp), ("sel_pool", _vp),
                ("pool_pcap", _i32), ("epochs", _i32), ("sel_slots", _i32),
                ("coarse_pool", _vp), ("coarse_first", _i32), ("coarse_count", _i32),
                ("qsel", _vp), ("qsel_words", _i32),
                ("local_lse", _vp), ("coarse_out", _vp), ("fine_out", _vp), ("den_out", _vp),
                ("external_values", _i32)]


class TrainBwd(ctypes.Structure):
    _fields_ = [("grad", _vp), ("grad_s", _I64x3),
                ("local", _vp), ("local_lse", _vp), ("coarse_out", _vp), ("fine_out", _vp),
                ("den_out", _vp),
                ("dq", _vp), ("dk", _vp), ("dv", _vp), ("draw_q", _vp), ("draw_k", _vp),
                ("dfusion_a", _vp), ("dfusion_b", _vp),
                ("workspace", _vp), ("workspace_bytes", _sz),
                ("dz_out", _vp), ("dc_out", _vp), ("dalpha_out", _vp), ("dlocal_out", _vp)]


class StreamCfg(ctypes.Structure):
    _fields_ = [("layer", _i32), ("local_keep", _i32), ("fine_tokens", _i32),
                ("coarse_group", _i32), ("route_period", _i32), ("layer_stagger", _i32),
                ("budget_root_scale", _i32), ("budget_offset", _i32), ("use_graph", _i32)]


PLAN_HEADER = 16
PLAN_ATTN_TILES = 1


def without_attention(plan):
    """A prefill plan with its local-attention section removed: the call's
    local output then comes from the caller (a local_flash plugin) through
    tao_prefill's `local` buffer."""
    import numpy as np
    n = int(plan[PLAN_ATTN_TILES])
    out = np.concatenate((plan[:PLAN_HEADER], plan[PLAN_HEADER + 3 * n:]))
    out[PLAN_ATTN_TILES] = 0
    return out


class Fusion(ctypes.Structure):
    _fields_ = [
        ("fusion_a", _vp), ("fusion_b", _vp), ("dtype", _i32),
        ("a_s", _I64x3), ("b_s", _I64x3),
        ("gain", ctypes.c_float), ("coarse_on", _i32), ("fine_on", _i32),
    ]


_SIGNATURES = {
    "tao_abi_version": ([], _i32),
    "tao_last_error": ([], ctypes.c_char_p),
    "tao_workspace_bytes": ([_i32, _i32, _i32, _i32, _i32], _sz),
    "tao_workspace_init": ([ctypes.POINTER(StateDev), _vp], _i32),
    "tao_decode_step": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens),
                         ctypes.POINTER(Fusion), _i32, _vp, ctypes.POINTER(_i64), _vp], _i32),
    "tao_decode_step_noalloc": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens),
                                 ctypes.POINTER(Fusion), _i32, _vp, ctypes.POINTER(_i64), _vp],
                                _i32),
    "tao_fold_route": ([ctypes.POINTER(StateDev), _i32, _vp], _i32),
    "tao_page_coarse": ([ctypes.POINTER(StateDev), _i32, _i32, _vp], _i32),
    "tao_fold_coarse": ([ctypes.POINTER(StateDev), _i32, _vp], _i32),
    "tao_route": ([ctypes.POINTER(StateDev), _vp, ctypes.POINTER(_i64),
                   _i32, _i32, _i32, _i32, _vp], _i32),
    "tao_write_fine": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens), _i64, _vp,
                        _i32, _i32, _vp], _i32),
    "tao_seal_epilogue": ([ctypes.POINTER(StateDev), _i32, _i32, _i32, _vp], _i32),
    "tao_prompt_attention": ([ctypes.POINTER(StreamCfg), _i32, _i32, _i32, ctypes.POINTER(Tokens),
                              _i64, _vp, _i64, _vp, _vp], _i32),
    "tao_local_attention": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens), _i64, _i64,
                             _vp, _i32, _vp, _vp], _i32),
    "tao_prefill": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens), ctypes.POINTER(Fusion),
                     ctypes.POINTER(_i64), _i64, ctypes.POINTER(PrefillPools), _vp, _vp,
                     ctypes.POINTER(_i64), _vp], _i32),
    "tao_ring_append": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens), _i32, _i32,
                         _i64, _vp], _i32),
    "tao_prefill_plan": ([ctypes.POINTER(StreamCfg), _i64, _i64, _i32, _i32, _i32,
                          _vp, _i64, ctypes.POINTER(_i64)], _i32),
    "tao_train_plan": ([ctypes.POINTER(StreamCfg), _i64, _vp, _i64, ctypes.POINTER(_i64)], _i32),
    "tao_train_bwd_workspace_bytes": ([ctypes.POINTER(StateDev), _i64, _i32,
                                       ctypes.POINTER(PrefillPools)], _sz),
    "tao_train_backward": ([ctypes.POINTER(StateDev), ctypes.POINTER(Tokens),
                            ctypes.POINTER(Fusion), ctypes.POINTER(PrefillPools),
                            ctypes.POINTER(TrainBwd), _vp], _i32),
    "tao_stream_open": ([ctypes.POINTER(StateDev), ctypes.POINTER(StreamCfg), _i64, _i32, _i32,
                         _vp, _vp, ctypes.POINTER(_vp)], _i32),
    "tao_stream_sync": ([_vp, ctypes.POINTER(StateDev), _i64, _i32, _i32], _i32),
    "tao_stream_decode": ([_vp, ctypes.POINTER(Tokens), ctypes.POINTER(Fusion), _vp,
                           ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64)], _i32),
    "tao_stream_plan_step": ([_vp, ctypes.POINTER(_i64)], _i32),
    "tao_stream_graph_step": ([_vp, ctypes.POINTER(Tokens), ctypes.POINTER(Fusion), _vp,
                               ctypes.POINTER(_i64), _vp], _i32),
    "tao_stream_advance": ([_vp, _i64], _i32),
    "tao_stream_release": ([_vp], _i32),
    "tao_stream_invalidate": ([_vp, _i32], _i32),
    "tao_stream_graph_stats": ([_vp, ctypes.POINTER(_i64), _i32], _i32),
    "tao_stream_close": ([_vp], _i32),
    "tao_graph_create": ([ctypes.POINTER(StateDev), ctypes.POINTER(Fusion), _i32, _vp, _vp,
                          _vp, ctypes.POINTER(_vp)], _i32),
    "tao_graph_launch": ([_vp, ctypes.POINTER(Tokens), _vp], _i32),
    "tao_graph_destroy": ([_vp], _i32),
    "tao_step_stamps": ([_vp, _i64, _i64], _i32),
    "tao_step_stamps_count": ([], _i64),
    "tao_numerics_selftest": ([_i32, _vp, _vp, _i64, _vp], _i32),
    "tao_full_sequence_f32_workspace_bytes": ([_i32, _i32, _i32, _i64, _i32], _sz),
    "tao_full_sequence_f32": ([ctypes.POINTER(StreamCfg), ctypes.POINTER(Tokens),
                               ctypes.POINTER(Fusion), _i32, _i32, _i32, _i32, _vp,
                               ctypes.POINTER(_i64), _vp, _i32, _vp, _sz, _vp], _i32),
    "tao_full_sequence_f32_local": ([ctypes.POINTER(StreamCfg), ctypes.POINTER(Tokens),
                                     ctypes.POINTER(Fusion), _i32, _i32, _i32, _i32, _vp, _vp,
                                     ctypes.POINTER(_i64), _vp, _i32, _vp, _sz, _vp], _i32),
    "tao_batch_table_bytes": ([_i32], _sz),
    "tao_batch_open": ([ctypes.POINTER(_vp), _i32, _vp, _sz, _vp, ctypes.POINTER(_vp)], _i32),
    "tao_batch_sync": ([_vp, _vp], _i32),
    "tao_batch_decode": ([_vp, ctypes.POINTER(Tokens), ctypes.POINTER(Fusion), _vp,
                          ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64)], _i32),
    "tao_batch_close": ([_vp], _i32),
    "tao_writer_statistics": ([_vp, ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64), _i32, _i32,
                               _i32, _i32, _i32, _vp, _vp, _vp, _vp], _i32),
    "tao_association_matrix": ([_vp, _vp, _i32, _i32, _vp, _vp, _vp], _i32),
    "tao_structured_matrix": ([_vp, _vp, _vp, _i32, _i32, ctypes.c_float, _vp, _vp], _i32),
    "tao_chronological_sum": ([_vp, _i64, _i32, _i64, _vp, _vp], _i32),
    "tao_feature_read_coefficients": ([_vp, ctypes.POINTER(_i64), _vp, ctypes.POINTER(_i64),
                                       _i32, _i32, _i32, _i32, _i32, _vp, _vp], _i32),
    "tao_selected_numerator": ([_vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp,
                                _vp], _i32),
    "tao_selected_numerator_backward": ([_vp, _vp, _vp, _vp, _i32, _i32, _i32, _i32, _i32, _i32,
                                         _i32, _vp, _vp, _vp], _i32),
}

EXPORTED = tuple(_SIGNATURES)

ABI_VERSION = 13               # TAO_ABI_VERSION of include/tao_memory.h

# Decode-graph epoch counters (enum tao_graph_stat / tao_graph_reason).
GRAPH_STATS = 19
GRAPH_REASONS = ("seal", "selected_shape", "epoch_change", "memo_replace", "request_end",
                 "reset", "capacity")
GRAPH_ACTIONS = ("uninitialized", "eager_warm", "capture_replay", "replay", "route_copy",
                 "invalidate")


_fast = None


def fast_module():
    """The native per-token decode entry (torch extension built beside the
    library), or None when it is not built: the host then issues the same
    C-ABI call through ctypes."""
    global _fast
    if _fast is None:
        import importlib.util
        import sysconfig
        path = os.path.join(os.path.dirname(_LIB_PATH),
                            "_tao_fast" + sysconfig.get_config_var("EXT_SUFFIX"))
        _fast = False
        if os.path.exists(path):
            spec = importlib.util.spec_from_file_location("_tao_fast", path)
            mod = importlib.util.module_from_spec(spec)
            spec.loader.exec_module(mod)
            _fast = mod
    return _fast or None


def function_address(name):
    return ctypes.cast(getattr(lib(), name), ctypes.c_void_p).value


def library_path():
    return _LIB_PATH


def lib():
    """Load (once) and return the HIP library; raise if it is not built."""
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(
                f"TaoMemory HIP library not built ({_LIB_PATH}); run "
                "`python tao-memory_amd/build.py` (no CPU fallback exists)")
        handle = ctypes.CDLL(_LIB_PATH)
        for name, (args, res) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        if handle.tao_abi_version() != ABI_VERSION:
            raise ImportError(f"{_LIB_PATH} has ABI {handle.tao_abi_version()}, these "
                              f"bindings ABI {ABI_VERSION}: rebuild the library")
        _lib = handle
    return _lib


def check(rc):
    """Map the library's return convention onto Python exceptions."""
    if rc == 0:
        return
    msg = lib().tao_last_error().decode(errors="replace")
    if rc < 0:
        raise ValueError(msg)
    raise RuntimeError(f"HIP error {rc}: {msg}")


def require_device(tensor):
    if not tensor.is_cuda:
        raise RuntimeError("TaoMemory HIP path needs device tensors (no CPU fallback)")


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def raw_stream(index):
    """The current HIP stream handle of device `index`."""
    if _raw_stream is not None:
        return _raw_stream(index)
    return torch.cuda.current_stream(index).cuda_stream


def stream_ptr(device):
    """The caller's current HIP stream on `device` (raw handle)."""
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def i64x3(values):
    return _I64x3(*[int(x) for x in values])


def vector_ready(t):
    """Rows load as 16-byte vectors: unit last stride, 8-element strides, aligned base."""
    st = t.stride()
    return st[-1] == 1 and all(x % 8 == 0 for x in st[:-1]) and t.data_ptr() % 16 == 0


def vector_operands(*tensors):
    """The operands, copied to contiguous storage where a row is not 16-byte aligned."""
    return tuple(t if vector_ready(t) else t.contiguous() for t in tensors)


def strides_bth(t):
    """Element strides (batch, token, head) of a [B, T, H, D] tensor."""
    s = t.stride()
    return (s[0], s[1], s[2])


def tokens(q, k, v, raw_q, raw_k, reuse=None):
    """Fill a Tokens struct; `reuse` (a previous struct) skips unchanged strides."""
    strides = (q.stride(), k.stride(), v.stride(), raw_q.stride(), raw_k.stride())
    if reuse is not None and reuse._strides == strides and reuse.tokens == q.shape[1]:
        tok = reuse
    else:
        tok = Tokens()
        tok.q_s = i64x3(strides[0][:3])
        tok.k_s = i64x3(strides[1][:3])
        tok.v_s = i64x3(strides[2][:3])
        tok.rq_s = i64x3(strides[3][:3])
        tok.rk_s = i64x3(strides[4][:3])
        tok.tokens = q.shape[1]
        tok._strides = strides
    tok.q, tok.k, tok.v = q.data_ptr(), k.data_ptr(), v.data_ptr()
    tok.raw_q, tok.raw_k = raw_q.data_ptr(), raw_k.data_ptr()
    return tok


_FUSION_CACHE = {}


def fusion(fusion_a, fusion_b, alpha, coarse_on, fine_on, like=None):
    """Fusion struct, cached per (parameter tensors, alpha, presence).

    Parameters of one dtype among bf16, fp32 and fp16 are read in place by
    the kernels, so in-place updates are seen by later calls; a tensor whose
    storage or layout changed gets a new struct. Other dtypes and mixed pairs
    are converted to fp32 on every call and never cached (the reference casts
    them on every call too, operator.py:23-24, fusion_pointwise.py:103-108).
    """
    key = (id(fusion_a), id(fusion_b), alpha, coarse_on, fine_on,
           None if like is None else (like.shape[2], like.shape[3], like.device))
    hit = _FUSION_CACHE.get(key)
    if (hit is not None and hit._keep[2] is fusion_a and hit._keep[3] is fusion_b
            and hit._check == (fusion_a.data_ptr(), fusion_b.data_ptr(),
                               fusion_a.stride(), fusion_b.stride(),
                               fusion_a.dtype, fusion_b.dtype)):
        return hit
    if like is not None:
        # The kernels read fusion_*[h, d, i] for every head and channel of the
        # operands (operator.py:83-89 takes [H, D, 3] parameters).
        _, _, heads, width = like.shape
        for t in (fusion_a, fusion_b):
            if tuple(t.shape) != (heads, width, 3):
                raise ValueError(f"fusion parameters must be [{heads}, {width}, 3], "
                                 f"got {tuple(t.shape)}")
            if t.device != like.device:
                raise ValueError("fusion parameters must live on the operands' device")
    fu = _make_fusion(fusion_a, fusion_b, alpha, coarse_on, fine_on)
    if fu.converted:
        return fu
    fu._check = (fusion_a.data_ptr(), fusion_b.data_ptr(), fusion_a.stride(),
                 fusion_b.stride(), fusion_a.dtype, fusion_b.dtype)
    if len(_FUSION_CACHE) > 64:
        _FUSION_CACHE.clear()
    _FUSION_CACHE[key] = fu
    return fu


def _make_fusion(fusion_a, fusion_b, alpha, coarse_on, fine_on):
    originals = (fusion_a, fusion_b)
    fu = Fusion()
    code = _PARAM_DTYPES.get(fusion_a.dtype)
    fu.converted = code is None or fusion_b.dtype != fusion_a.dtype
    if fu.converted:
        # A per-call copy: the caller's later in-place updates reach the
        # next call's copy, never a cached one.
        fusion_a = fusion_a.float()
        fusion_b = fusion_b.float()
        code = TAO_FP32
    fu.dtype = code
    fu.fusion_a, fu.fusion_b = fusion_a.data_ptr(), fusion_b.data_ptr()
    fu.a_s = i64x3(fusion_a.stride())
    fu.b_s = i64x3(fusion_b.stride())
    # gain = torch.full((), 2 * alpha, dtype=bf16) as in operator.py:89.
    fu.gain = float(torch.full((), 2 * alpha, dtype=torch.bfloat16))
    fu.coarse_on, fu.fine_on = int(bool(coarse_on)), int(bool(fine_on))
    # Keep the (possibly converted) parameter tensors alive with the struct.
    fu._keep = (fusion_a, fusion_b) + originals
    return fu
