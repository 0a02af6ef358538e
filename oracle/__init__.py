"""CPU oracle for the W4A8 MoE expert path (TEST INFRASTRUCTURE ONLY).

This package is the checker, never the product. Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it.
The shipped path (``rdna4-vllm_amd/w4a8_fp8_wmma``) never imports it and fails
loudly when its HIP library is missing.

Every function restates the arithmetic of patcarter883/rdna4-vllm's W4A8 path
(kernel and test files cited per function) in numpy. How each function is pinned
(exhaustive tables, library casts, closed forms, brute force) is listed in
``PINNING`` below and exercised by ``tests/test_oracle_*.py``.
"""
from .w4a8_oracle import *  # noqa: F401,F403
from .w4a8_oracle import PINNING  # noqa: F401
