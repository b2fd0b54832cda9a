"""MI355X (gfx950) implementation of the PLM round's dense-linear hot path.

* ``fast_gemm``   — drop-in for the reference's ``plm.fast_gemm`` (``install``, ``fast_gemm``,
                    ``hip_linear``, ``CONFIGS``, ``HALF_DTYPES``).
* ``gemm_tables`` — drop-in for ``plm.gemm_tables`` (``model_shapes``, ``load_table``, ``install``).
* ``verify``      — the fused LM-head verify step (softmax / argmax / nucleus membership).
* ``workloads``   — the measured shapes and their seeded inputs.

All compute runs in ``libplm_amd.so`` (hand-written HIP kernels, C ABI in ``include/plm_amd.h``).
"""

from . import fast_gemm, gated_lora, gemm_tables, verify, workloads  # noqa: F401
from ._lib import LIBRARY, lib  # noqa: F401
