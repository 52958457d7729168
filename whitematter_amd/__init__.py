"""MI355X (gfx950) implementation of whitematter's Tensor elementwise,
broadcast, reduction and softmax hot path.

- ``libwm_hip.so`` (built from csrc/): the HIP kernels behind the C ABI in
  include/wm_hip.h;
- ``core/``: the C++ ``Tensor`` with the reference's class API
  (core/tensor.h:12-137), device-resident storage, calling that ABI;
- ``_lib``: a ctypes binding of the C ABI used by the tests and the bench;
- ``synth``: the seeded input generator shared by GPU path, oracle and bench.
"""
