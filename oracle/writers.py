"""CPU restatement of the non-preset fine writers and the channel-given read.

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may import this module, and only as the
checker; the product never routes through it.

Restates (paths relative to the reference repository root):
  association_statistics   tao_attention/association_writer.py:11-18
  association_matrix       tao_attention/association_writer.py:21-32
  chronological_sum        tao_attention/association_writer.py:35-40
  feature_read_coefficients tao_attention/association_writer.py:43-53
  structured_statistics    tao_attention/structured_writer.py:5-13
  structured_matrix        tao_attention/structured_writer.py:16-34
  selected_fine_numerator  tao_attention/indirect_fine.py:65-133 (forward:
                           per-pair fp32 products, then an ordered sum over the
                           selection slots, _grouped_forward :136-159 and
                           _sum_selected :162-169) and its backward
                           (_grouped_grad_a :172-195, _shared_grad_c :198-227)

Every routine works in float64 on the reference's rounding points (the bf16
feature cast of u, the final bf16 cast of C and of the read output), so the
HIP path is held to the reference within the fp32-vs-fp64 gap plus one bf16
rounding of the result. Two inputs of routing are exact instead: the feature
simplex u and the feature masses are fp32 in an order this build fixes
(feature_simplex, feature_mass), so fine and page descriptors r(log mass)
are bit-reproducible.

Pinning (tests/test_oracle.py): association_matrix against numpy's dense
solve and the residual of the regularised normal equations; structured_matrix
against a dense solve of the matrix its two Sherman-Morrison steps invert
(diag(var + ridge) - var var^T / sum(var) + mass mass^T / count); statistics
against their invariants (gram symmetric with trace sum_t |u_t|^2, sum_d mass
= token count within bf16 rounding, column sums of cross = sum_d of u times
v); feature_read_coefficients against its mixture invariants; the selected
numerator against a per-query brute-force loop and one-hot channels that pick
single rows of C.
"""

import numpy as np
import torch

from .numerics import exp32, sequential_sum

BF16 = torch.bfloat16


def _bf16(x):
    return x.to(BF16).to(torch.float64)


def feature_simplex(k):
    """u = bf16(softmax_D(k.float())) (association_writer.py:14).

    The fp32 softmax's internals are the backend's; this build fixes them
    (the HIP statistics kernel computes the same): e = correctly rounded fp32
    exp(k - max); s = the D channels in 8 contiguous groups, each summed in
    channel order, then the 8 group sums pairwise,
    ((g0+g1)+(g2+g3))+((g4+g5)+(g6+g7)); u = r(e / s). Returned as fp64
    (exact: u is bf16)."""
    x = k.float()
    e = exp32(x - x.amax(-1, keepdim=True))
    d = e.shape[-1]
    groups = sequential_sum(e.reshape(*e.shape[:-1], 8, d // 8), -1)
    while groups.shape[-1] > 1:
        groups = groups[..., 0::2] + groups[..., 1::2]
    return _bf16(e / groups)


def feature_mass(u):
    """sum_t u (association_writer.py:18, structured_writer.py:9) in fp32,
    tokens in order (axis -2 of u [N, H, T, D]); the reference's fp32
    reduction order is its backend's, this build fixes token order."""
    return sequential_sum(u.float(), -2)


def association_statistics(k, v, with_mass=False):
    """k, v: [N, T, H, D] -> gram [N, H, D, D], cross [N, H, D, D] (fp64),
    optional mass [N, H, D] (fp32, feature_mass) (association_writer.py:11-18)."""
    u = feature_simplex(k).transpose(1, 2)            # [N, H, T, D]
    values = v.double().transpose(1, 2)
    gram = u.transpose(-1, -2) @ u
    cross = u.transpose(-1, -2) @ values
    if with_mass:
        return gram, cross, feature_mass(u)
    return gram, cross


def regularised_system(gram):
    """gram + (trace(gram) / D) I (association_writer.py:24-27)."""
    width = gram.shape[-1]
    ridge = gram.diagonal(dim1=-2, dim2=-1).sum(-1) / width
    return gram + ridge[..., None, None] * torch.eye(width, dtype=gram.dtype)


def association_matrix(gram, cross):
    """bf16(cholesky_solve(cross, chol(gram + tr/D I))) (association_writer.py:21-32).
    Returns the fp64 solution before the cast and the bf16 result."""
    system = regularised_system(gram.double())
    factor = torch.linalg.cholesky(system)
    solution = torch.cholesky_solve(cross.double(), factor)
    return solution, solution.to(BF16)


def chronological_sum(statistics):
    """Sum over axis -3 in fine order (association_writer.py:35-40)."""
    total = statistics.select(-3, 0).clone()
    for index in range(1, statistics.shape[-3]):
        total = total + statistics.select(-3, index)
    return total


def feature_read_coefficients(h, read_z):
    """h [B, T, H, D], read_z broadcastable to [B, T, H, P, D]:
    mixture_p = (h . exp z_p) / sum_p (h . exp z_p); out = bf16(mixture_p h)
    (association_writer.py:43-53)."""
    query = h.double().unsqueeze(-2)
    mass = (query * read_z.double().exp()).sum(-1)
    mixture = mass / mass.sum(-1, keepdim=True)
    return (mixture.unsqueeze(-1) * query).to(BF16)


def structured_statistics(k, v):
    """k, v: [N, T, H, D] -> square_mass [N, H, D], cross [N, H, D, D],
    mass [N, H, D] (structured_writer.py:5-13). The square mass and the mass
    are fp32 sums in token order (u * u is exact in fp32); cross is fp64."""
    u = feature_simplex(k).transpose(1, 2)
    values = v.double().transpose(1, 2)
    return feature_mass(u * u), u.transpose(-1, -2) @ values, feature_mass(u)


def structured_matrix(square_mass, cross, mass, count):
    """The frozen diagonal / two-rank inverse applied to cross
    (structured_writer.py:16-34). Returns the fp64 result and its bf16 cast."""
    square_mass, cross, mass = square_mass.double(), cross.double(), mass.double()
    variance = (square_mass - mass * mass / count).clamp_min(0)
    variance_sum = variance.sum(-1, keepdim=True)
    ridge = square_mass.sum(-1, keepdim=True) / mass.shape[-1]
    diagonal = variance + ridge
    zero = variance_sum == 0
    t = torch.where(zero, torch.zeros_like(variance), variance / diagonal)
    positive_sum = (variance * ridge / diagonal).sum(-1, keepdim=True)
    safe_sum = torch.where(zero, torch.ones_like(positive_sum), positive_sum)
    t_cross = (t.unsqueeze(-1) * cross).sum(-2)
    hb = (cross / diagonal.unsqueeze(-1)
          + t.unsqueeze(-1) * t_cross.unsqueeze(-2) / safe_sum.unsqueeze(-1))
    hm = mass / diagonal + t * (t * mass).sum(-1, keepdim=True) / safe_sum
    mass_hb = (mass.unsqueeze(-1) * hb).sum(-2)
    denominator = count + (mass * hm).sum(-1, keepdim=True)
    result = hb - hm.unsqueeze(-1) * mass_hb.unsqueeze(-2) / denominator.unsqueeze(-1)
    return result, result.to(BF16)


def structured_system(square_mass, mass, count):
    """The matrix structured_matrix inverts, written densely (checker):
    diag(var + ridge) - var var^T / sum(var) + mass mass^T / count, the
    rank-one var term dropped when sum(var) == 0."""
    square_mass, mass = square_mass.double(), mass.double()
    variance = (square_mass - mass * mass / count).clamp_min(0)
    ridge = square_mass.sum(-1, keepdim=True) / mass.shape[-1]
    total = variance.sum(-1, keepdim=True)
    system = torch.diag_embed(variance + ridge)
    outer = variance.unsqueeze(-1) * variance.unsqueeze(-2)
    safe = torch.where(total == 0, torch.ones_like(total), total)
    system = system - torch.where(total.unsqueeze(-1) == 0, torch.zeros_like(outer),
                                  outer / safe.unsqueeze(-1))
    return system + mass.unsqueeze(-1) * mass.unsqueeze(-2) / count


def selected_fine_numerator(channel, selected_id, fine_c):
    """channel [B, Q, H, M, D] bf16, selected_id [B, Q, H, M], fine_c
    [BB, H, S, D, D] bf16 (C[d][e], batch b reads bank b % BB):
    out[b, q, h, e] = bf16(sum_m fp32(sum_d channel[m][d] C[id_m][d][e]))
    (indirect_fine.py:123-133, :136-169)."""
    b, q, h, m, d = channel.shape
    bank_b = fine_c.shape[0]
    banks = fine_c.double()[torch.arange(b) % bank_b]            # [B, H, S, D, D]
    ids = selected_id.long()
    gathered = banks[torch.arange(b)[:, None, None, None], torch.arange(h)[None, None, :, None],
                     ids]                                         # [B, Q, H, M, D, D]
    pairs = torch.einsum("bqhmd,bqhmde->bqhme", channel.double(), gathered)
    pairs = pairs.float().double()                                # per-pair fp32 result
    return pairs.sum(3).to(BF16)


def selected_fine_numerator_loop(channel, selected_id, fine_c):
    """Per-query brute force of selected_fine_numerator (checker)."""
    b, q, h, m, d = channel.shape
    out = torch.zeros(b, q, h, d, dtype=torch.float64)
    bank_b = fine_c.shape[0]
    for bi in range(b):
        for qi in range(q):
            for hi in range(h):
                acc = torch.zeros(d, dtype=torch.float64)
                for mi in range(m):
                    seg = int(selected_id[bi, qi, hi, mi])
                    c = fine_c[bi % bank_b, hi, seg].double()
                    acc += channel[bi, qi, hi, mi].double() @ c
                out[bi, qi, hi] = acc
    return out.to(BF16)


def selected_fine_numerator_backward(channel, selected_id, fine_c, grad):
    """grad_channel[b,q,h,m,d] = sum_e grad[b,q,h,e] C[id_m][d][e] (fp32 out,
    cast to the channel dtype) and grad_fine_c[bb,h,s,d,e] = sum over the
    batches b with b % BB == bb of bf16(sum over that batch's (q, m) with
    id == s of channel[d] grad[e]) (indirect_fine.py:101-120, 172-227)."""
    b, q, h, m, d = channel.shape
    bank_b, _, s = fine_c.shape[:3]
    banks = fine_c.double()[torch.arange(b) % bank_b]
    ids = selected_id.long()
    gathered = banks[torch.arange(b)[:, None, None, None], torch.arange(h)[None, None, :, None],
                     ids]
    grad_channel = torch.einsum("bqhe,bqhmde->bqhmd", grad.double(), gathered).to(BF16)
    onehot = torch.nn.functional.one_hot(ids, s).double()        # [B, Q, H, M, S]
    per_batch = torch.einsum("bqhms,bqhmd,bqhe->bhsde", onehot, channel.double(),
                             grad.double())
    per_batch = per_batch.to(BF16).double()
    grad_c = torch.zeros(bank_b, h, s, d, d, dtype=torch.float64)
    for bi in range(b):
        grad_c[bi % bank_b] += per_batch[bi]
    return grad_channel, grad_c.float().to(BF16)


def dense_solve(system, rhs):
    """numpy's LU solve in float64 (checker, independent of Cholesky)."""
    return torch.from_numpy(np.linalg.solve(system.numpy(), rhs.numpy()))
