"""Simplex-feature statistics and regularised solves on the HIP library.

Mirrors the reference module tao_attention/association_writer.py (same
function names, arguments, shapes and dtypes): bf16 features
u = bf16(softmax_D(fp32 k)), fp32 statistics, the trace-regularised Cholesky
solve and the bf16 matrix, the chronological statistic sum and the
feature-mass read coefficients. Every function runs the library's kernels on
device tensors (no CPU path) and is forward-only: with autograd recording and
an input that requires grad it raises, rather than silently detaching.
"""
import ctypes

import torch

from . import _hip

__all__ = ["association_statistics", "association_matrix", "chronological_sum",
           "feature_read_coefficients"]


def _forward_only(name, *tensors):
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise RuntimeError(f"{name}: the HIP writer path has no autograd; "
                           "call it under torch.no_grad() or on detached inputs")


def _blocks(k, v, name):
    """[N, T, H, D] bf16 device operands with a contiguous channel axis."""
    for t in (k, v):
        _hip.require_device(t)
    if k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"{name} expects k and v of one shape [N, T, H, D]")
    if k.dtype != torch.bfloat16 or v.dtype != torch.bfloat16:
        raise ValueError(f"{name} expects bf16 k and v")
    k, v = _hip.vector_operands(k, v)
    return k, v


def _statistics(k, v, mode, with_mass, name):
    _forward_only(name, k, v)
    k, v = _blocks(k, v, name)
    n, t, h, d = k.shape
    dev = k.device
    cross = torch.empty(n, h, d, d, device=dev, dtype=torch.float32)
    mass = torch.empty(n, h, d, device=dev, dtype=torch.float32) if with_mass else None
    if mode == 1:
        first = torch.empty(n, h, d, device=dev, dtype=torch.float32)
    else:
        first = torch.empty(n, h, d, d, device=dev, dtype=torch.float32)
    ks = (_hip._i64 * 3)(*k.stride()[:3])
    vs = (_hip._i64 * 3)(*v.stride()[:3])
    _hip.check(_hip.lib().tao_writer_statistics(
        k.data_ptr(), ks, v.data_ptr(), vs, n, t, h, d, mode, first.data_ptr(),
        cross.data_ptr(), mass.data_ptr() if mass is not None else None,
        _hip.stream_ptr(dev)))
    return first, cross, mass


def association_statistics(k, v, with_mass=False):
    """Raw K/V [N, T, H, D] -> fp32 gram and cross [N, H, D, D], plus the fp32
    feature mass [N, H, D] with with_mass (association_writer.py:11-18)."""
    gram, cross, mass = _statistics(k, v, 0, with_mass, "association_statistics")
    return (gram, cross, mass) if with_mass else (gram, cross)


def association_matrix(gram, cross, unchecked=False):
    """bf16 C = (gram + trace(gram)/D I)^-1 cross over [..., D, D] fp32 pairs by
    a Cholesky factor (association_writer.py:21-32). Checked mode raises
    torch.linalg.LinAlgError when a factor is not positive definite, as
    torch.linalg.cholesky does (one device synchronisation)."""
    _forward_only("association_matrix", gram, cross)
    _hip.require_device(gram)
    if gram.shape != cross.shape or gram.dim() < 2 or gram.shape[-1] != gram.shape[-2]:
        raise ValueError("association_matrix expects gram and cross of one shape [..., D, D]")
    if gram.dtype != torch.float32 or cross.dtype != torch.float32:
        raise ValueError("association_matrix expects fp32 statistics")
    d = gram.shape[-1]
    gram, cross = gram.contiguous(), cross.contiguous()
    count = gram.numel() // (d * d)
    out = torch.empty(gram.shape, device=gram.device, dtype=torch.bfloat16)
    info = None if unchecked else torch.zeros(max(count, 1), device=gram.device, dtype=torch.int32)
    _hip.check(_hip.lib().tao_association_matrix(
        gram.data_ptr(), cross.data_ptr(), count, d, out.data_ptr(),
        info.data_ptr() if info is not None else None, _hip.stream_ptr(gram.device)))
    if info is not None and count and bool((info[:count] != 0).any()):
        first = int(info[:count][info[:count] != 0][0])
        raise torch.linalg.LinAlgError(
            f"association_matrix: the leading minor of order {first} is not positive-definite")
    return out


def chronological_sum(statistics):
    """Sum the fine axis -3 in fine order, fp32 (association_writer.py:35-40)."""
    _forward_only("chronological_sum", statistics)
    _hip.require_device(statistics)
    if statistics.dim() < 3:
        raise ValueError("chronological_sum needs a fine axis at -3")
    if statistics.dtype != torch.float32:
        raise ValueError("chronological_sum expects fp32 statistics")
    x = statistics.contiguous()
    shape = x.shape
    fines = shape[-3]
    inner = shape[-2] * shape[-1]
    outer = x.numel() // max(fines * inner, 1) if fines * inner else 0
    out = torch.empty(shape[:-3] + shape[-2:], device=x.device, dtype=torch.float32)
    if fines == 0:
        raise ValueError("chronological_sum of an empty fine axis")
    _hip.check(_hip.lib().tao_chronological_sum(x.data_ptr(), outer, fines, inner,
                                                out.data_ptr(), _hip.stream_ptr(x.device)))
    return out


def feature_read_coefficients(h, read_z):
    """h [B, T, H, D], read_z broadcastable to [B, T, H, P, D]: bf16
    mixture_p * h with mixture_p = (h . exp z_p) / sum_p (h . exp z_p)
    (association_writer.py:43-53)."""
    _forward_only("feature_read_coefficients", h, read_z)
    _hip.require_device(h)
    if h.dim() != 4 or read_z.dim() != 5:
        raise ValueError("feature_read_coefficients expects h [B,T,H,D], read_z [..,P,D]")
    if h.dtype != torch.bfloat16 or read_z.dtype != torch.bfloat16:
        raise ValueError("feature_read_coefficients expects bf16 operands")
    b, t, nh, d = h.shape
    pages = read_z.shape[3]
    z = read_z.expand(b, t, nh, pages, d)
    if h.stride(-1) != 1:
        h = h.contiguous()
    if z.stride(-1) != 1:
        z = z.contiguous()
    out = torch.empty(b, t, nh, pages, d, device=h.device, dtype=torch.bfloat16)
    hs = (_hip._i64 * 3)(*h.stride()[:3])
    zs = (_hip._i64 * 4)(*z.stride()[:4])
    _hip.check(_hip.lib().tao_feature_read_coefficients(
        h.data_ptr(), hs, z.data_ptr(), zs, b, t, nh, pages, d, out.data_ptr(),
        _hip.stream_ptr(h.device)))
    return out
