"""CPU oracle for the hot/cold sparse-FFN path.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker or the timed CPU baseline,
never by the shipped library.
"""
