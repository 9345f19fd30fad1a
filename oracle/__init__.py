"""CPU oracle for the paged-attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, as the checker; the product path never does.
"""
from .pa_oracle import *  # noqa: F401,F403
from .pa_oracle import lib, ref  # noqa: F401
