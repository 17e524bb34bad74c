"""CPU oracle of the quantized projection hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg, as the checker.  The product (m5kernels_amd / libm5k.so) never uses it.
"""
