"""CPU oracle for the decode hot path -- TEST INFRASTRUCTURE ONLY.

Importable only from ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``.  The shipped package never imports it.
"""

from .decode_oracle import *  # noqa: F401,F403
from .decode_oracle import PINNING  # noqa: F401
