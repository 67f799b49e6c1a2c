"""TEST INFRASTRUCTURE ONLY: the fp64 CPU oracle for the GEMM-family path.

Importable only from tests/, ``__graft_entry__.smoke()`` and bench.py's
``cpu_baseline`` leg, as the checker.
"""
from .oracle import *  # noqa: F401,F403
from .oracle import build, lib, TOL, DENSE, LOWER, UPPER  # noqa: F401
