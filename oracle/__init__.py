"""CPU oracle for mtlattn's varlen attention.

TEST INFRASTRUCTURE ONLY. Nothing in the product path (mtlattn_amd/, mtlattn/)
imports this package. Only tests/, __graft_entry__.smoke() and the cpu_baseline
leg of bench.py use it, and only as the checker or as the timed CPU baseline.
"""

from .reference import (  # noqa: F401
    allowed_mask,
    attended_pairs,
    brute_force,
    seq_lens,
    varlen_forward,
    varlen_forward_backward,
    varlen_forward_backward_blocked,
)
