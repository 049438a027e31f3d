"""CPU oracle and CPU baseline for the paged-KV hot path.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py.  The product package never imports it.
"""
