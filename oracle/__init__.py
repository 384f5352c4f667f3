"""CPU oracle for the ChebyKAN hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker or the timed
CPU baseline.  The product path (``kan_amd``) never calls into it.
"""
from .chebykan_oracle import *  # noqa: F401,F403
