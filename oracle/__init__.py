"""Test infrastructure: the porch host evaluator (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use
this package, as the checker; the product never imports it.
"""
