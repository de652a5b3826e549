"""CPU oracle for the exlr8 MoE expert path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg
may import this package, and only as the checker (or the timed CPU baseline).  The
product package ``mlxlr8_amd`` never imports it.

``moe_oracle.c`` (built to ``libmoe_oracle.so`` by ``oracle/Makefile``) restates the
reference operators.  The checks that pin it (closed forms, brute force on small cases, the
reference's own known answers under ``tests/golden/``) live in ``tests/`` (``tests/refmath.py``
and the ``tests/test_oracle_*.py`` files).  ``native_f32`` builds the same source with fp32
accumulation for the host it runs on: the timed CPU baseline of ``bench.py``.
"""
from .cbind import lib, build, native_f32  # noqa: F401
