"""CPU oracle for lanternl's pure-Lua path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
may import this package, and only as the checker (or the timed CPU stand-in
for the single-threaded LuaJIT path).  The product package ``lanternl_amd``
never imports it.

``oracle.py`` wraps ``liboracle.so`` (``oracle.c``, built by ``oracle/Makefile``)
with numpy float64 arrays.  Each C function cites the reference Lua it restates.
"""
from .oracle import *  # noqa: F401,F403
