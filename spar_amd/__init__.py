"""Spar's MI355X (gfx950) device backend.

`spar_amd.hip` binds the C ABI (include/spar_hip.h) with ctypes; the C++ host
library (Tensor, ops, autograd) is reachable from Python as `spar_amd.spar`
once built (`python -m spar_amd.build`).
"""
