"""Numeric primitives of the TaoMemory CPU oracle.

TEST INFRASTRUCTURE ONLY: the oracle is the checker. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import
anything under ``oracle/``; the product never does.

The reference computes in bf16 with one round-to-nearest-even per torch op and
fp32 inside each op (torch's bf16 elementwise/reduction semantics). Three
choices the reference leaves to its backend are fixed here, identically in the
HIP kernels, so that everything feeding routing is bit-reproducible:

* ``exp32``/``log32`` are correctly rounded fp32 (computed in fp64, rounded
  once). Any <=1 ulp fp32 implementation (torch CPU, CUDA, ROCm) agrees with
  them except within one fp32 ulp of a rounding boundary.
* ``fold_sum`` is the fp32 reduction order of a 64-lane butterfly: zero-pad
  to a power of two, then repeatedly add the upper half onto the lower half.
* ``quarter_sum`` (writer token sums) splits the axis into four contiguous
  quarters, sums each sequentially in fp32, then adds (q0+q1)+(q2+q3).
"""

import torch

BF16 = torch.bfloat16
F32 = torch.float32


def rnd(x, dtype=BF16):
    """One round-to-nearest-even to ``dtype`` (the reference's ``.to(dtype)``)."""
    return x.to(dtype)


def exp32(x):
    """Correctly rounded fp32 exp of an fp32 tensor."""
    return x.to(torch.float64).exp().to(F32)


def log32(x):
    """Correctly rounded fp32 natural log of an fp32 tensor."""
    return x.to(torch.float64).log().to(F32)


def fold_sum(x, dim=-1):
    """fp32 sum along ``dim`` in butterfly (fold-halves) order."""
    x = x.to(F32).movedim(dim, -1)
    n = x.shape[-1]
    width = 1
    while width < n:
        width *= 2
    if width != n:
        pad = torch.zeros((*x.shape[:-1], width - n), dtype=F32)
        x = torch.cat((x, pad), dim=-1)
    while x.shape[-1] > 1:
        half = x.shape[-1] // 2
        x = x[..., :half] + x[..., half:]
    return x[..., 0]


def sequential_sum(x, dim=-1):
    """fp32 left-to-right sum along ``dim``."""
    x = x.to(F32).movedim(dim, 0)
    total = torch.zeros(x.shape[1:], dtype=F32)
    for index in range(x.shape[0]):
        total = total + x[index]
    return total


def quarter_sum(x, dim):
    """fp32 sum: four contiguous quarters summed sequentially, then paired."""
    x = x.to(F32).movedim(dim, 0)
    n = x.shape[0]
    if n % 4:
        return sequential_sum(x, 0)
    parts = x.reshape(4, n // 4, *x.shape[1:])
    acc = torch.zeros((4, *x.shape[1:]), dtype=F32)
    for index in range(n // 4):
        acc = acc + parts[:, index]
    return (acc[0] + acc[1]) + (acc[2] + acc[3])


def softmax(x, dim):
    """torch ``F.softmax`` on a reduced-precision tensor, output rounded once.

    fp32 internals: max, correctly rounded exp(x - max), butterfly sum,
    division; then one rounding to x's dtype.
    """
    dtype = x.dtype
    xf = x.to(F32).movedim(dim, -1)
    top = xf.amax(-1, keepdim=True)
    e = exp32(xf - top)
    total = fold_sum(e, -1)
    return rnd(e / total.unsqueeze(-1), dtype).movedim(-1, dim)


def logsumexp(x, dim):
    """torch.logsumexp on a reduced-precision tensor (composite op).

    torch evaluates ``max + log(sum(exp(x - max)))`` as separate tensor ops
    on x's dtype, so every intermediate is rounded: r(x-m), r(exp), r(sum),
    r(log), r(log + m). Infinite maxima are replaced by 0 first.
    """
    dtype = x.dtype
    top = x.amax(dim, keepdim=True)
    top = top.masked_fill(top.abs() == float("inf"), 0)
    shifted = rnd(x.to(F32) - top.to(F32), dtype)
    e = rnd(exp32(shifted.to(F32)), dtype)
    total = rnd(fold_sum(e, dim), dtype)
    logged = rnd(log32(total.to(F32)), dtype)
    return rnd(logged.to(F32) + top.squeeze(dim).to(F32), dtype)


def bf16_bits(x):
    """int32 view of bf16 values (for bit-exact comparisons)."""
    return x.to(BF16).view(torch.int16).to(torch.int32) & 0xFFFF
