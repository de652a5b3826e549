"""CPU oracle for the exlr8 MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker (or the timed CPU baseline).  The
product package ``mlxlr8_amd`` never imports it.

``moe_oracle.c`` (built to ``libmoe_oracle.so`` by ``oracle/Makefile``) restates the
reference operators; ``numpy_ref.py`` holds independent numpy restatements used to
pin the C code (closed forms, brute force, the reference's own known answers).
"""
from .cbind import lib, build  # noqa: F401
