"""MI355X-native batched four-player Junqi environment.

The rules, legal-move generation, combat memory, beliefs and the 317-plane
observation run as HIP kernels in ``_build/libjunqi_amd.so`` (C ABI declared in
``include/junqi_amd.h``). Importing this package fails if that library is not
built; there is no CPU implementation behind it.
"""

from . import _lib
from ._lib import AUX_CHANNELS, SLOTS_PER_PIECE, JunqiError
from .batch import JunqiBatch, decode_table, decode_u8, generate_lineups, generate_pool, recency_table, zobrist_stream
from .gpu_rollout import GpuRollout
from .gpu_world import GpuWorld
from .history import GpuRolloutHistory

__all__ = ["JunqiBatch", "GpuRollout", "GpuWorld", "GpuRolloutHistory", "JunqiError", "AUX_CHANNELS", "SLOTS_PER_PIECE", "decode_table", "decode_u8",
           "generate_lineups", "generate_pool", "recency_table", "zobrist_stream", "_lib"]
