"""Named operating presets (reference tao_attention/presets.py:5-12)."""

from .config import TaoConfig


def index_only_page_memo(*, graph=False):
    """Index-only coarse routing with the q1 page-normalisation memo.

    ``graph=True`` replays the non-refresh single-token decode step from a
    captured hipGraph; the arithmetic is the same kernels as eager execution.
    """
    return TaoConfig(coarse_index_only=True, q1_page_normalization_memo=True,
                     q1_history_region_graph=graph)
