"""CPU oracle for the sparse attention path — test infrastructure only.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the reference results are compared with
or the timed CPU baseline.
"""
