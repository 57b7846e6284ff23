"""CPU oracle of the quantized decode hot path — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this package, and only as the checker (or the timed CPU baseline), never as
the product path: the product is the HIP libraries under
dsv4-flash-gb10-runtime_amd/kernel/, which fail loudly when missing.

Contents
  mx.py        numpy restatement of the reference's CPU math (dequant + fp32
               matmul + bf16 casts), each function citing the reference
               file:line it follows;
  mx_oracle.c  independent scalar C restatement with fp64 accumulation (the
               brute-force comparator), built by the Makefile here into
               oracle/libmx_oracle.so and loaded through c_oracle.py.

Pinning (what checks each function against something other than itself) is
listed in each function's docstring; the tests under tests/ run those checks.
The reference's own CUDA sources cannot be built here (no nvcc, and a hipify
of them is excluded), so there is no oracle/_ref build.
"""
