"""CPU oracle for the Soklyn DenseBlock hot path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker / the CPU baseline being timed.
"""
