"""CPU oracle for the KDA core -- test infrastructure, never part of the product path.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker or the timed CPU baseline.
"""

from .kda_oracle import (  # noqa: F401
    FP16_MAX_SAFE,
    kda_chunkwise_ref,
    kda_recurrent_f64,
    kda_recurrent_ref,
)
