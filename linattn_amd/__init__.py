"""linattn_amd -- MI355X (gfx950) HIP implementation of the sparse-attention hot
path of tongxin/linattn: Quest page selection, the lightning indexer top-k, and
block-sparse prefill / paged sparse decode.

Kernel-level entry points mirror the reference's kernel modules
(src/linattn/kernels/triton/{block_sparse,quest_pages,fused_indexer}.py and
src/linattn/kernels/c_attention.py); the ``hip_*`` variants plug into the
reference's AttentionVariant contract (src/linattn/core.py:187-306) the way the
MLX adapter does (src/linattn/kernels/mlx/adapter.py:34-107).
"""

from linattn_amd._native import LIB_PATH, load  # noqa: F401
from linattn_amd.kernels import backend_for, describe_backends  # noqa: F401

__version__ = "0.1.0"
