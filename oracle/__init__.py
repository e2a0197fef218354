"""CPU oracle of the per-rank zig-zag ring-attention path (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this
package, and only to check or time the reference algorithm; the fa4_ring product never does.
"""
from .ring_oracle import *  # noqa: F401,F403
