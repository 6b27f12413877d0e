"""Python access to the MI355X triton-ext extension libraries.

The product is the C-ABI in ../lib (headers in include/triton_ext/):
  libTritonExtPassInfra.so  tritonAddPluginPass / tritonRegisterPluginPass /
                            tritonEnumeratePluginPasses / TritonExtLoadPass
                            (R:infra/pass/TritonExtPassInfra.h:10-26)
  libloop_split.so          "loop_split" extension (R:pass/LoopSplit/LoopSplit.cpp)
  libarith_intensity.so     "arith_intensity" extension
  libmi355x_dot.so          "mi355x_dot" extension: gfx950 kernels + tx_dot_*

This module binds them with ctypes (the binding a Python caller such as
Triton's runtime would add) and offers `dot()` over torch device tensors.
torch is used only for device memory and streams.  There is no CPU fallback:
if libmi355x_dot.so is missing, `load()` raises.
"""
from .capi import *  # noqa: F401,F403
from .dot import (aligned_rows, attention, dot, dot_scaled, new_output, plan_for, tx_type,  # noqa: F401
                  workspace_for)
