"""ORACLE -- test infrastructure only.

CPU restatements of the reference's paged-attention path that tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg compare the HIP
path with.  Nothing in the product package imports this package.

  attention.py  the reference CPU kernel (C restatement + the reference's own
                build) and a float64 closed form
  packing.py    cu_seqlens / slot mapping / block tables / positions / mask /
                KV scatter, in NumPy
"""
