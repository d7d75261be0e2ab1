"""fp32 sufficient statistics and the analytic structured-Gram association on
the HIP library.

Mirrors the reference module tao_attention/structured_writer.py (same names,
arguments, shapes and dtypes); forward-only like association_writer.
"""
import torch

from . import _hip
from .association_writer import _forward_only, _statistics

__all__ = ["structured_statistics", "structured_matrix"]


def structured_statistics(k, v):
    """k, v [N, T, H, D] -> square_mass [N, H, D], cross [N, H, D, D],
    mass [N, H, D], fp32 (structured_writer.py:5-13)."""
    square, cross, mass = _statistics(k, v, 1, True, "structured_statistics")
    return square, cross, mass


def structured_matrix(square_mass, cross, mass, count):
    """bf16 (diag(var + ridge) - var var^T / sum(var) + mass mass^T / count)^-1
    cross, by its two Sherman-Morrison steps (structured_writer.py:16-34)."""
    _forward_only("structured_matrix", square_mass, cross, mass)
    _hip.require_device(cross)
    d = cross.shape[-1]
    if (cross.dim() < 2 or cross.shape[-2] != d or square_mass.shape != cross.shape[:-1]
            or mass.shape != square_mass.shape):
        raise ValueError("structured_matrix expects square_mass/mass [..., D] and cross [..., D, D]")
    if any(t.dtype != torch.float32 for t in (square_mass, cross, mass)):
        raise ValueError("structured_matrix expects fp32 statistics")
    square_mass, cross, mass = (t.contiguous() for t in (square_mass, cross, mass))
    count_mats = cross.numel() // (d * d)
    out = torch.empty(cross.shape, device=cross.device, dtype=torch.bfloat16)
    _hip.check(_hip.lib().tao_structured_matrix(
        square_mass.data_ptr(), cross.data_ptr(), mass.data_ptr(), count_mats, d,
        float(count), out.data_ptr(), _hip.stream_ptr(cross.device)))
    return out
