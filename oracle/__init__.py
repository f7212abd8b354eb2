"""Test infrastructure: the porch host evaluator (liboracle.so).

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use
this package, to compare results against; the product never imports it.
"""
