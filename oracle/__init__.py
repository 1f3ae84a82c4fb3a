"""CPU oracle for the decode hot path — TEST INFRASTRUCTURE ONLY.

Loaded by tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline``
leg, as the checker; the product (``popcorn_amd``) never imports it.
"""
from .binding import *  # noqa: F401,F403
