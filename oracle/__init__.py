"""CPU oracle for the tiled dot -- TEST INFRASTRUCTURE ONLY.

Python access to liboracle.so (a C restatement of the Triton interpreter's
tiled dot, see tiled_dot.c) plus small numpy helpers.  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg import this package,
and only as the checker; the product path never does.

Function headers state which reference or third-party behaviour each part
restates, and which checks in tests/ pin it.
"""
from .oracle import *  # noqa: F401,F403
