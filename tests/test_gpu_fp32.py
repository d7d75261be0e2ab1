"""fp32 tao_attention (BASELINE configs[0] class) against the oracle.

The oracle's training_forward on fp32 operands defines the fp32 semantics
(every rounding point of the bf16 contract at fp32; pinned against an fp64
evaluation in test_oracle.py). The HIP fp32 read must give the oracle's
routes bit for bit and outputs within the north-star fp32 tolerance, 1e-4
absolute and relative.
"""
import pytest
import torch

from oracle import tao_oracle as O
from tao_attention import TaoConfig, tao_attention
from tao_attention import training
from tao_attention.presets import index_only_page_memo

pytestmark = pytest.mark.gpu
TOL32 = dict(atol=1e-4, rtol=1e-4)


def rope(x, base=10000.0):
    """Rotary embedding over channel pairs (d, d + D/2) at positions 0..T-1."""
    t, d = x.shape[1], x.shape[-1]
    inv = base ** (-torch.arange(0, d // 2, dtype=torch.float64) * 2 / d)
    ang = torch.arange(t, dtype=torch.float64)[:, None] * inv[None, :]
    cos = torch.cat((ang.cos(), ang.cos()), -1)[None, :, None, :]
    sin = torch.cat((ang.sin(), ang.sin()), -1)[None, :, None, :]
    half = d // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), -1)
    return (x.double() * cos + rot.double() * sin).to(x.dtype)


def config0_inputs(batch=1, tokens=2048, heads=4, width=64, seed=0):
    """q/k/v/raw_q/raw_k N(0, 1) from `seed`, RoPE on q and k by
    the caller, fusion_a/b N(0, 0.02) [H, D, 3]."""
    g = torch.Generator().manual_seed(seed)
    xs = [torch.randn(batch, tokens, heads, width, generator=g) for _ in range(5)]
    fa = torch.randn(heads, width, 3, generator=g) * 0.02
    fb = torch.randn(heads, width, 3, generator=g) * 0.02
    xs[0], xs[1] = rope(xs[0]), rope(xs[1])
    return xs, fa, fb


def check_routes(sel, routes, tokens):
    """HIP selections [B, T, H, Mmax] (-1 padded) == the oracle's per-tile
    selections [B, Q, H, M], every query with history."""
    checked = 0
    for tile, want in routes.items():
        start = tile * 256
        got = sel[:, start:start + want.shape[1]].cpu().long()
        m = want.shape[-1]
        assert torch.equal(got[..., :m], want), f"tile {tile}"
        assert bool((got[..., m:] == -1).all())
        checked += want.numel()
    first = min(routes) * 256 if routes else tokens
    assert bool((sel[:, :first].cpu() == -1).all())
    assert checked > 0


@pytest.mark.parametrize("batch,tokens,heads,width,cfg,seed", [
    (1, 2048, 4, 64, index_only_page_memo(), 0),          # configs[0] itself
    (2, 3000, 2, 128, TaoConfig(), 7),                    # pages, coarse values, log 2 bias
    (1, 2900, 3, 64, index_only_page_memo(), 8),          # completed page, index-only
    (1, 2100, 2, 128, TaoConfig(), 9),                    # ragged last tile
])
def test_fp32_full_sequence_matches_oracle(batch, tokens, heads, width, cfg, seed):
    xs, fa, fb = config0_inputs(batch, tokens, heads, width, seed)
    print(f"fp32 full sequence B{batch} T{tokens} H{heads} D{width} "
          f"index_only={cfg.coarse_index_only}", flush=True)
    dev = [x.cuda() for x in xs]
    with torch.no_grad():
        out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                            fusion_b=fb.cuda(), alpha=0.5, config=cfg)
        again, sel = training.forward_f32(*dev, fa.cuda(), fb.cuda(), 0.5, cfg,
                                          return_routes=True)
    assert out.dtype == torch.float32
    assert torch.equal(out, again)
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True)
    check_routes(sel, routes, tokens)
    torch.testing.assert_close(out.cpu(), ref, **TOL32)


def test_fp32_bf16_fusion_parameters_and_strided_operands():
    """bf16 fusion parameters (upcast exactly, operator.py:23-24) and
    non-contiguous fp32 operands (token-strided views) give the same result
    as the contiguous fp32 call with the upcast parameters."""
    xs, fa, fb = config0_inputs(1, 1300, 2, 64, 11)
    fa16, fb16 = fa.to(torch.bfloat16), fb.to(torch.bfloat16)
    cfg = index_only_page_memo()
    wide = [torch.cat((x, x), -1).cuda()[..., :64] for x in xs]       # strided rows
    with torch.no_grad():
        got = tao_attention(*wide[:3], raw_q=wide[3], raw_k=wide[4], fusion_a=fa16.cuda(),
                            fusion_b=fb16.cuda(), alpha=0.5, config=cfg)
        want = tao_attention(*(x.cuda() for x in xs[:3]), raw_q=xs[3].cuda(),
                             raw_k=xs[4].cuda(), fusion_a=fa16.float().cuda(),
                             fusion_b=fb16.float().cuda(), alpha=0.5, config=cfg)
    assert torch.equal(got, want)
    ref = O.training_forward(*xs, fa16.float(), fb16.float(), 0.5,
                             O.Geometry.from_config(cfg))
    torch.testing.assert_close(got.cpu(), ref, **TOL32)


@pytest.mark.parametrize("tokens,cfg", [(2048, index_only_page_memo()), (2100, TaoConfig())])
def test_fp32_with_a_local_flash_plugin(tokens, cfg):
    """fp32 operands with a caller plugin (operator.py:40-52 passes
    local_flash to read_training at any dtype): the plugin is called with the
    reference's tiling on the fp32 operands (here the reference adapter's
    SDPA modes in fp32, recorded), the read takes its fp32 output
    (tao_full_sequence_f32_local), routes stay bit-exact and the output is
    within the fp32 tolerance of the oracle."""
    from types import SimpleNamespace
    from test_gpu_plugin import sdpa_fp32
    xs, fa, fb = config0_inputs(1, tokens, 2, 64, 21)
    dev = [x.cuda() for x in xs]
    calls = []

    def recorded(q, k, v, causal=True, window_size=(-1, 0)):
        assert q.dtype == torch.float32 and k.dtype == torch.float32
        calls.append((q.shape[1], k.shape[1]))
        return sdpa_fp32(q, k, v, causal=causal, window_size=window_size)

    plugin = SimpleNamespace(flash_attn_func=recorded)
    print(f"fp32 with plugin T{tokens} index_only={cfg.coarse_index_only}", flush=True)
    with torch.no_grad():
        out = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                            fusion_b=fb.cuda(), alpha=0.5, config=cfg, local_flash=plugin)
        own = tao_attention(*dev[:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                            fusion_b=fb.cuda(), alpha=0.5, config=cfg)
        from tao_attention.flash_attention import plugin_training_local
        local = plugin_training_local(SimpleNamespace(flash_attn_func=sdpa_fp32), *dev[:3], cfg)
        _, sel = training.forward_f32(*dev, fa.cuda(), fb.cuda(), 0.5, cfg,
                                      return_routes=True, local=local)
    assert out.dtype == torch.float32 and calls
    ref, routes = O.training_forward(*xs, fa, fb, 0.5, O.Geometry.from_config(cfg),
                                     return_routes=True)
    check_routes(sel, routes, tokens)
    torch.testing.assert_close(out.cpu(), ref, **TOL32)
    torch.testing.assert_close(out, own, **TOL32)
    with pytest.raises(ValueError):
        training.forward_f32(*dev, fa.cuda(), fb.cuda(), 0.5, cfg, local=local[:, 1:])


def test_fp32_contract_errors():
    xs, fa, fb = config0_inputs(1, 300, 2, 64, 12)
    dev = [x.cuda() for x in xs]
    leaf = dev[0].clone().requires_grad_(True)
    with pytest.raises(NotImplementedError):
        tao_attention(leaf, *dev[1:3], raw_q=dev[3], raw_k=dev[4], fusion_a=fa.cuda(),
                      fusion_b=fb.cuda(), alpha=0.5)
    with pytest.raises(TypeError):
        tao_attention(dev[0].to(torch.bfloat16), *dev[1:3], raw_q=dev[3], raw_k=dev[4],
                      fusion_a=fa.cuda(), fusion_b=fb.cuda(), alpha=0.5)
