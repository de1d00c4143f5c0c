"""CPU oracle of ditch's reference numerics — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, always as the checker (or the timed CPU baseline), never as a
path of the product.
"""
