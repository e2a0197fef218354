"""fa4_ring on MI355X: one rank's causal zig-zag ring attention on gfx950 HIP kernels.

Public API (the reference package's names):
    RingConfig          configuration (cp_size, cp_rank, merge_mode, ...)
    ring_flash_attn     causal ring attention over a zig-zag local shard
    Descales            FP8 per-tensor descales (k / v indexed by source rank)
    zigzag_shard / zigzag_unshard   shard a full sequence / stitch shards back
    IncrementalMerger / BatchedMerger / make_merger   online-softmax mergers
and, for the single-GPU ring:
    LocalKVRing         every source rank's KV shard resident in HBM
    PagedKVRing         every source rank's paged K/V cache (fused sweep)
    quantize_e4m3 / quantize_ring   the FP8 producer (e4m3 shards and their descales)
    ring_flash_attn_backward / ring_flash_attn_func   the sweep's backward (the reference is
                        forward-only): functional, and as a torch.autograd function
"""

from .backward import ring_flash_attn_backward, ring_flash_attn_func
from .config import RingConfig
from .fp8 import quantize_e4m3, quantize_ring
from .merge import BatchedMerger, IncrementalMerger, make_merger
from .paged import PagedKVRing
from .ring_attention import Descales, LocalKVRing, ring_flash_attn
from .zigzag import zigzag_shard, zigzag_unshard

__all__ = [
    "RingConfig",
    "ring_flash_attn",
    "Descales",
    "LocalKVRing",
    "PagedKVRing",
    "zigzag_shard",
    "zigzag_unshard",
    "IncrementalMerger",
    "BatchedMerger",
    "make_merger",
    "quantize_e4m3",
    "quantize_ring",
    "ring_flash_attn_backward",
    "ring_flash_attn_func",
]
