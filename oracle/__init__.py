"""CPU oracle for the DSA decode path (test infrastructure only).

This package restates, in plain numpy, what the reference computes on the DSA
decode path. It is the checker for the HIP kernels and is imported only by
``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py``. The product path (``nanoengine_amd``) never imports it.
"""
from .dsa_oracle import *  # noqa: F401,F403
