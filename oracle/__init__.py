"""CPU oracle for the quantized-linear hot path.

Test infrastructure only: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker and never as the thing
measured or shipped. The product package (spark-mlx-llm_amd/sparkq) does not
import it.
"""

from .oracle import *  # noqa: F401,F403
