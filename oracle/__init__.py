"""CPU oracle of the quantized DiT hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, as the checker.  The product package never does.
"""
