"""Float64 CPU oracle for the reconstruction path -- test infrastructure only.

Imported only by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg, as the
checker or the timed CPU baseline; the cufk_amd package never imports it.
"""
