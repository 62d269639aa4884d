"""CPU checkers for the LiGGUF decode path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg
import this package, and only as the checker.  ``ligguf_amd`` never does.

* ``liblg_oracle.so`` -- plain-C restatement (lg_oracle.c), always built.
* ``_ref/libligguf_ref.so`` -- the reference FAST engine compiled from its own
  sources (Makefile target ``ref``); present only where it was built.
"""
from .binding import (  # noqa: F401
    Oracle, Reference, load_oracle, load_reference, reference_available,
    ORACLE_DIR, build_oracle, build_reference,
)
