"""CPU oracle for the ternocl_amd HIP library -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline
leg may import this package, and only to check results against.  The product never does.

* :mod:`oracle.binding` -- numpy wrappers of ``liboracle.so`` (the C restatement
  of TernOCL's host golds, ``ternocl_oracle.c``) and, where it was built, of
  ``_ref/libternocl_ref.so`` (the reference's own host golds compiled from their
  sources, ``ref_shim.cpp``).
"""
