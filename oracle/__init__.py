"""ORACLE -- test infrastructure only, never product code.

CPU restatements of the reference's attention forward used to check the HIP
kernels of mtlflashattn_amd:
  * chunked.py    -- the reference's chunked-fp32 torch path (the oracle proper)
  * stream_ref.c  -- float64 two-pass restatement of the scalar kernel math,
                     used to pin chunked.py (stream.py wraps it)
Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this package.
"""
