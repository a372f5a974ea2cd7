"""CPU oracle for the gfx950 hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or the timed CPU baseline).  The shipped library and the plugin never
call it; the product path fails loudly when the HIP library is missing instead of falling back
here.
"""
