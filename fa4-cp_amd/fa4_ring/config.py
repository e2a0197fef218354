"""Ring configuration (interface of fa4_ring/config.py:15-33)."""

from dataclasses import dataclass
from typing import Optional

# "incremental": one in-place LSE merge after every ring step (O(1) extra state).
# "batched": every step's partial is kept and all are merged by one kernel at the end.
MERGE_MODES = ("incremental", "batched")


@dataclass
class RingConfig:
    """Zig-zag causal ring settings for one rank.

    cp_size / cp_rank: ring size and this rank's position.  causal must stay True (the
    zig-zag schedule is the causal one).  softmax_scale None means 1/sqrt(head_dim).
    deterministic is accepted for interface compatibility; every kernel here is
    deterministic (fixed reduction order, no atomics)."""

    cp_size: int
    cp_rank: int
    causal: bool = True
    softmax_scale: Optional[float] = None
    merge_mode: str = "incremental"
    deterministic: bool = False

    def __post_init__(self):
        assert self.merge_mode in MERGE_MODES, (
            f"merge_mode must be one of {MERGE_MODES}, got {self.merge_mode}")
        assert self.cp_size >= 1, "cp_size must be >= 1"
        assert 0 <= self.cp_rank < self.cp_size, (
            f"cp_rank {self.cp_rank} not in [0, {self.cp_size})")
        assert self.causal, "only the causal zig-zag ring is implemented"
