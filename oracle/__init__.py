"""CPU oracle and baseline restatements of the reference RBF attention math.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the rbf_attention_amd package.
"""
