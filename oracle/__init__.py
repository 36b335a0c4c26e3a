"""CPU oracle of the ternary BitLinear hot path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import or run anything
here, and only as the checker or the timed CPU baseline.  The product (wrinklefree-monorepo_amd/)
never imports it.  Contents:
  bitnet_oracle.py  numpy restatement of the reference algorithm (file:line citations inside)
  c/i2s_oracle.c    C restatement (scalar I2_S dot, OpenMP GEMM, quantiser)
  c/ref_shim.cpp    extern "C" wrappers over the reference's own bitnet_gemv.cpp
  Makefile          builds c/liboracle_c.so and, where the reference tree exists, _ref/*.so
  refbind.py        ctypes bindings of those libraries
"""
