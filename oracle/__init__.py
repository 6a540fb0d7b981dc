"""CPU oracle for the DetLLM integer forward pass — TEST INFRASTRUCTURE ONLY.

This package is a numpy restatement of the reference's CPU ("reference")
backend: every function cites the reference file:line it follows and
reproduces its integer semantics bit for bit (int64 two's-complement wrap on
add/mul, torch's shift clamping, Python floor division).

Who may use it: ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, and only as the checker / the timed CPU baseline. The
product package ``idempotent_llm_amd`` never imports it; its compute runs
only through the HIP library and fails loudly when that is missing.

Parity status of each function is recorded in its docstring:
  * "pinned: <how>" — checked against golden vectors written from the
    reference (tests/golden/), closed forms or brute force;
  * "parity unpinned" — no such check exists (none at present).
"""

from . import intmath, dyadic, gemm, ops, model  # noqa: F401
