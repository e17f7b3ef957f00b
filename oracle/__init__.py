"""CPU oracle for the out-of-core FP32 SGEMM path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of ``bench.py`` -- always as the checker or the timed
CPU baseline, never by the product path (``xvram_amd``). The C sources and the
citations of the reference algorithms they restate are in ``xvram_oracle.c``.
"""
from .oracle import *  # noqa: F401,F403
