"""CPU oracle of the IFKFAC curvature path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, never by the ifkfac_amd package.
"""
