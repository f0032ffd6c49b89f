"""CPU oracle for the krunch hot path — TEST INFRASTRUCTURE ONLY.

Nothing in the product (`krunch_amd/`) imports, links or runs anything under
this directory. Only `tests/`, `__graft_entry__.smoke()` and the
`cpu_baseline` leg of `bench.py` use it, and only as the checker / the timed
CPU baseline — never as the thing measured on the GPU or shipped.

Each module restates one piece of the reference's algorithm for the batched
RWKV-4 compress/decompress path, citing the reference file:line it follows:

  range_coder.py  cpu_reference.py:28-234          (pure-Python integer spec)
  range_coder.c   same, in C (fast; CPU baseline)   -> oracle/lib/liboracle_rc.so
  cdf.py          cdf.py:22-74 + numpy's float32 row-sum order
  softmax.py      the build's deterministic softmax (exp2-based exp) whose
                  output feeds cdf.py's procedure; det_softmax_cdf.cu:62-185
                  is the reference counterpart
  rwkv4.py        batched_rwkv4.py:60-262 layer math with the WKV of
                  wkv_kernel.cu:52-73 (fp32 torch)

How each function is pinned (golden vectors, closed forms, library routines,
invariants) is listed in the module headers and in tests/test_oracle_*.py.
"""
