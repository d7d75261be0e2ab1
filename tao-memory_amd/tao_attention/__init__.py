"""TaoMemory attention on MI355X: functional API and explicit per-layer state.

Drop-in for the reference package ``tao_attention`` (same names and
signatures); the compute runs in the gfx950 HIP library libtao_hip.so.
"""

from .operator import (new_state, tao_attention, tao_attention_decode,
                       tao_attention_decode_batch, tao_attention_prefill)
from .tao_stream import StreamCache
from .config import TaoConfig
from .step_graph import WholeStepGraph

__all__ = ["new_state", "tao_attention", "tao_attention_prefill",
           "tao_attention_decode", "tao_attention_decode_batch", "StreamCache", "TaoConfig",
           "WholeStepGraph"]
