"""gfx950 (MI355X) tile-local one-level Strassen GEMM with fused epilogues.

Drop-in for the reference's ``strassen_pallas`` GEMM path: ``strassen_matmul``
and the relayout helpers keep the reference's names, arguments and errors;
the compute is the hand-written HIP kernel in ``csrc/strassen_gemm.hip``
behind the C ABI ``include/strassen_mi355x.h``.
"""

from .layouts import (  # noqa: F401
    is_k_contiguous, k_contiguous, rope_layout_tables, rope_layout_to_heads,
    rope_scale_layout, rope_weight_layout, swiglu_weight_layout,
)
from .strassen import (  # noqa: F401
    PROFILE_INFO, TUNED_BK, TUNED_BM, TUNED_BN, VMEM_PROFILE, check_tiling,
    cubic_matmul, native_matmul, plain_weight_kernel, strassen_kernel, strassen_matmul,
    strassen_matmul_lhs_transposed,
)

from .packing import (  # noqa: F401
    ExactSchedule, PackedOperand, SplitOperand, cache_packed_weights, cubic_weight_layout, pack_activation,
    pack_operand, packed_weight_cache_info, precision_passes, strassen_weight_layout,
)
from .strassen import PlainWeightPackWarning  # noqa: F401
from .tuning import tuned_matmul  # noqa: F401

__version__ = "0.5.0"
