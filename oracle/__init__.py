"""CPU oracle for rich-triplet's Q4_K / BF16 decode path -- TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker.  The product (rich-triplet_amd/) never
links or calls it.
"""
