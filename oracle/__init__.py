"""CPU oracle for the path-ordered attention forward (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this package, and only as the checker or the timed CPU baseline. The product
(holonomyawareattention_amd) never imports it and fails loudly when its HIP
library is missing.
"""
