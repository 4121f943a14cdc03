"""sparseforge_amd: MI355X-native sparse-training hot path of SparseForge.

Drop-in modules mirroring liuhanzuo/SparseForge legacy/:
  sparse_modeling  SparseLinearConfig, SparseLinear, FusedMaskedLinearSTE, Distill_Model
  utils            mask-op functions (calculate_model_mask, update_hessian_hutchinson, ...)
  adamw            AdamW with the mask-aware decay
  block_sparse     convert_to_block_sparse, BlockSparseLinear (block-sparse-16 GEMM)
All tensor work runs in the HIP library libsparseforge_amd.so (gfx950).
"""
from . import _lib  # noqa: F401

__all__ = ["_lib"]
