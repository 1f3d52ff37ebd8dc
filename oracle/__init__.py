"""CPU oracle for the KTIR execution path — TEST INFRASTRUCTURE ONLY.

This package restates, in NumPy, the reference interpreter's algorithm
(torch-spyre/ktir-cpu ``ktir_cpu/interpreter.py``, ``grid.py``, ``memory.py``,
``ops/*``, ``dialects/*``): cores run one after another in core-id order,
every op is one or a few NumPy calls, HBM is a sparse byte-addressed store.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import it, and only as the checker / baseline.  The product
(``ktir_cpu_amd``) never imports it.

Pinning status per function is recorded in ``oracle/interp.py``'s header.
"""

from .interp import OracleInterpreter, OracleTile  # noqa: F401
