"""Channel-given selected contraction on the HIP library.

Mirrors selected_fine_numerator and _SelectedContraction of the reference
module tao_attention/indirect_fine.py (:65-133): the numerator-only fine read
of the feature-mass writers, with autograd. The reference's grouped Triton
kernels (_selected_bounds, _grouped_forward, _sum_selected, _grouped_grad_a,
_shared_grad_c) and its legacy per-query kernel are replaced by the library's
query-tile MFMA kernels (tao_selected_numerator / _backward).
"""
import torch

from . import _hip

__all__ = ["selected_fine_numerator"]


def _validate(channel, selected_id, fine_c):
    b, q, h, m, d = channel.shape
    if (d not in (64, 128) or fine_c.shape[1] != h or b % fine_c.shape[0] != 0
            or fine_c.shape[3:] != (d, d)
            or selected_id.shape != (b, q, h, m)
            or channel.dtype != torch.bfloat16
            or fine_c.dtype != torch.bfloat16):
        raise ValueError("selected fine contraction requires BF16 D64 or D128 tensors")


class _SelectedContraction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, channel, selected_id, fine_c):
        _validate(channel, selected_id, fine_c)
        for t in (channel, selected_id, fine_c):
            _hip.require_device(t)
        channel = channel.contiguous()
        ids = selected_id.contiguous().to(torch.int64)
        fine_c = fine_c.contiguous()
        b, q, h, m, d = channel.shape
        out = torch.empty((b, q, h, d), device=channel.device, dtype=channel.dtype)
        _hip.check(_hip.lib().tao_selected_numerator(
            channel.data_ptr(), ids.data_ptr(), fine_c.data_ptr(), b, q, h, m,
            fine_c.shape[0], fine_c.shape[2], d, out.data_ptr(),
            _hip.stream_ptr(channel.device)))
        ctx.save_for_backward(channel, ids, fine_c)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        channel, ids, fine_c = ctx.saved_tensors
        b, q, h, m, d = channel.shape
        grad = grad_output.contiguous().to(torch.bfloat16)
        grad_channel = torch.empty_like(channel) if ctx.needs_input_grad[0] else None
        grad_fine_c = torch.empty_like(fine_c) if ctx.needs_input_grad[2] else None
        if grad_channel is not None or grad_fine_c is not None:
            _hip.check(_hip.lib().tao_selected_numerator_backward(
                channel.data_ptr(), ids.data_ptr(), fine_c.data_ptr(), grad.data_ptr(),
                b, q, h, m, fine_c.shape[0], fine_c.shape[2], d,
                grad_channel.data_ptr() if grad_channel is not None else None,
                grad_fine_c.data_ptr() if grad_fine_c is not None else None,
                _hip.stream_ptr(channel.device)))
        return grad_channel, None, grad_fine_c


def selected_fine_numerator(channel, selected_id, fine_c):
    """out[b, q, h] = bf16(sum_m channel[b, q, h, m] . C[id_m]) with
    C = fine_c[b % BB, h] (indirect_fine.py:123-133), differentiable in channel
    and fine_c."""
    return _SelectedContraction.apply(channel, selected_id, fine_c)
