"""CPU oracle (test infrastructure only): restatements of the reference's PyTorch math.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import this package.
"""
