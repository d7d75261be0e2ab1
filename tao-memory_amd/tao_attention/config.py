"""Frozen TaoMemory geometry and the routing-budget closed form.

Same fields, defaults, validation errors and ``export()`` round trip as the
reference ``TaoConfig`` (tao_attention/config.py:7-63), so snapshot dicts and
``TaoConfig(**config.export())`` move between the two implementations.
"""

from dataclasses import asdict, dataclass
from math import isqrt

WRITERS = ("softmax", "regularized_association", "feature_mass_association",
           "structured_gram_association")

_INT_FIELDS = ("fine_tokens", "local_keep", "coarse_group", "route_period",
               "layer_stagger", "budget_root_scale", "budget_offset")


@dataclass(frozen=True)
class TaoConfig:
    fine_tokens: int = 256
    local_keep: int = 512
    coarse_group: int = 8
    route_period: int = 24
    layer_stagger: int = 2
    budget_root_scale: int = 2
    budget_offset: int = 2
    fine_writer: str = "softmax"
    coarse_index_only: bool = False
    q1_page_normalization_memo: bool = False
    q1_history_region_graph: bool = False

    def __post_init__(self):
        # Checks run in the reference's order (config.py:21-36) so the same
        # bad config raises the same exception type first.
        if self.fine_writer not in WRITERS:
            raise ValueError("unsupported fine writer")
        if any(type(getattr(self, name)) is not int for name in _INT_FIELDS):
            raise TypeError("Tao geometry and budget fields must be integers")
        if self.fine_tokens <= 0 or self.local_keep <= 0:
            raise ValueError("fine_tokens and local_keep must be positive")
        if self.local_keep % self.fine_tokens:
            raise ValueError("local_keep must be a multiple of fine_tokens")
        if self.coarse_group <= 0 or self.route_period <= 0:
            raise ValueError("coarse_group and route_period must be positive")
        if (self.layer_stagger < 0 or self.budget_root_scale <= 0
                or self.budget_offset < 0):
            raise ValueError("unsupported stagger or budget policy")

    @property
    def serve_limit(self):
        """Longest exact-local span served before the oldest block seals."""
        return self.local_keep + self.fine_tokens

    @property
    def first_fine(self):
        """First absolute position that can read a sealed fine memory."""
        return self.serve_limit

    @property
    def first_coarse(self):
        """First absolute position whose history holds a completed page."""
        return self.local_keep + self.coarse_group * self.fine_tokens

    @property
    def visibility_tiles(self):
        return self.local_keep // self.fine_tokens

    def budget(self, count):
        """min(count, ceil(sqrt(scale*count)) + offset), exact integer form."""
        if count <= 0:
            return 0
        target = self.budget_root_scale * count
        root = isqrt(target)
        if root * root < target:
            root += 1
        return min(count, root + self.budget_offset)

    def export(self):
        return asdict(self)
