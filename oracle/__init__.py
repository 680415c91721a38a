"""CPU oracle for the quantized-matmul path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package; the product (zero_amd/) never does.
"""
