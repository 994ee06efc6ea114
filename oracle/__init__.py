"""Oracle: CPU restatements of the reference's decode arithmetic.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import anything under oracle/, and only as the
checker or the timed CPU baseline, never as the thing measured or shipped.
"""
