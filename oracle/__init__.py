"""CPU oracle for the LeanSelect prefill hot path (test infrastructure only).

This package restates the reference algorithm on the CPU so the HIP kernels in
``leanselect_amd`` can be checked against it.  It is the checker, never the
product: only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of
``bench.py`` may import it.  Nothing in ``leanselect_amd`` imports it, and the
product path raises when the HIP library is missing instead of falling back
here.
"""

from .leanselect_oracle import *  # noqa: F401,F403
from .check import *  # noqa: F401,F403
from .nosa_oracle import *  # noqa: F401,F403
from .minicpm_oracle import *  # noqa: F401,F403
from .reference_path import *  # noqa: F401,F403
from .decode_oracle import *  # noqa: F401,F403
