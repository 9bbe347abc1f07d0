"""CPU oracle — test infrastructure only (see oracle.cpp's header).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package, and only as the checker / the timed CPU baseline.
"""
