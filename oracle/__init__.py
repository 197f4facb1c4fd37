"""CPU oracle for the MI355X rasterizer -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package; the product package blitzgs_amd never does.
"""
