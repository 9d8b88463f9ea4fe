"""Parity oracle: CPU restatement of the reference quantized matvec (test infrastructure only).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package, and only
as the checker or the timed CPU baseline. The product (vinf_3080ti_amd) never imports it.
"""
