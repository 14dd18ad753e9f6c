"""CPU oracle for the Mixture-of-Memory read — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline), never as the product path. ``naylis_amd`` never imports it.
"""
from .mom_oracle import *  # noqa: F401,F403
from .decoder_oracle import OracleDecoder  # noqa: F401
