"""CPU oracle for the Pairformer pair path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg import this package, and only as
the reference the results are compared with (or as the timed reference-equivalent CPU path). The product path in ``boltz_mlx_amd`` never imports it.
"""

from oracle.pairformer import *  # noqa: F401,F403
