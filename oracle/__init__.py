"""CPU oracle for the MoE expert hot path -- test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package; the product (tinygiant_amd) never does.  See oracle.py.
"""
