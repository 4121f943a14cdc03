"""Drop-in block-sparse-16 format and linear layer (legacy/triton_block_sparse.py).

Same names and signatures as the reference: convert_to_block_sparse,
get_sparsity_info, BlockSparseLinear (from_dense / from_sparse_linear),
convert_model_to_block_sparse.  The compressed layout is the reference's
(blocks [nnz, 16, 16], row_ptr int32 [nbr + 1], col_idx int32 [nnz]) plus a
block map [nbr, nbc] (block index or -1) that the MFMA kernels use to find
blocks.  Differences, by design:

* the index is built on the device (three kernels, one host sync to read
  nnz) instead of a Python loop with a sync per block;
* blocks are stored and multiplied in bf16 (or f32) on MFMA, not fp16;
* bsr_linear / BlockSparseLinear(trainable=True) also run the backward: the
  input gradient through the transposed blocks and the weight gradient as an
  SDDMM that only writes kept blocks (the reference is forward-only).
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from . import _lib as L
from . import profiling as _prof

BLOCK = 16


def convert_to_block_sparse(weight: torch.Tensor, mask: torch.Tensor, block_size: int = 16,
                            return_block_map: bool = False, blocks_dtype: Optional[torch.dtype] = None):
    """(sparse_blocks, block_row_indices, block_col_indices[, block_map]) of weight * mask (:46-103)."""
    if block_size != BLOCK:
        raise NotImplementedError(f"block_size {block_size}: only 16 is built on the MI355X path")
    out_f, in_f = weight.shape
    if out_f % block_size or in_f % block_size:
        raise ValueError(f"weight shape {tuple(weight.shape)} is not a multiple of the block size {block_size}")
    W, M = weight.detach().contiguous(), mask.detach().contiguous()
    if M.shape != W.shape:
        raise ValueError(f"mask shape {tuple(M.shape)} != weight shape {tuple(W.shape)}")
    dev = L.require_device(W, M)
    nbr, nbc = out_f // block_size, in_f // block_size
    flags = torch.empty(nbr * nbc, dtype=torch.uint8, device=dev)
    counts = torch.empty(nbr, dtype=torch.int32, device=dev)
    row_ptr = torch.empty(nbr + 1, dtype=torch.int32, device=dev)
    st = L.stream(dev)
    with _prof.region("sf_bsr_build", W.numel() * (W.element_size() + M.element_size()), "B", dev):
        L.check(L.lib().sf_bsr_count(L.ptr(W), L.dtype_code(W), L.ptr(M), L.dtype_code(M), out_f, in_f, block_size,
                                     L.ptr(flags), L.ptr(counts), st), "sf_bsr_count")
        L.check(L.lib().sf_bsr_scan(L.ptr(counts), nbr, L.ptr(row_ptr), st), "sf_bsr_scan")
        nnz = int(row_ptr[-1].item())  # the one host sync: the size of the compressed arrays
        bdt = blocks_dtype or torch.promote_types(W.dtype, M.dtype)
        blocks = torch.zeros(max(nnz, 1), block_size, block_size, dtype=bdt, device=dev)
        col_idx = torch.empty(nnz, dtype=torch.int32, device=dev)
        bmap = torch.empty(nbr, nbc, dtype=torch.int32, device=dev)
        L.check(L.lib().sf_bsr_fill(L.ptr(W), L.dtype_code(W), L.ptr(M), L.dtype_code(M), out_f, in_f, block_size,
                                    L.ptr(flags), L.ptr(row_ptr), L.ptr(col_idx) if nnz else None, L.ptr(blocks),
                                    L.dtype_code(blocks), L.ptr(bmap), st), "sf_bsr_fill")
    if return_block_map:
        return blocks, row_ptr, col_idx, bmap
    return blocks, row_ptr, col_idx


def block_map_from_csr(row_ptr: torch.Tensor, col_idx: torch.Tensor, num_block_cols: int) -> torch.Tensor:
    """[nbr, nbc] block map of any CSR block index (validated on the host first)."""
    rp = row_ptr.detach().to("cpu", torch.int64)
    nnz = col_idx.numel()
    if rp.numel() < 1 or int(rp[0]) != 0 or bool((rp[1:] < rp[:-1]).any()) or int(rp[-1]) != nnz:
        raise ValueError("block_row_indices must be a non-decreasing scan from 0 to len(block_col_indices)")
    dev = L.require_device(row_ptr, col_idx if nnz else None) if nnz else row_ptr.device
    nbr = rp.numel() - 1
    bmap = torch.empty(nbr, num_block_cols, dtype=torch.int32, device=dev)
    L.check(L.lib().sf_bsr_block_map(L.ptr(row_ptr.contiguous()), L.ptr(col_idx.contiguous()) if nnz else None, nbr,
                                     num_block_cols, L.ptr(bmap), L.stream(dev)), "sf_bsr_block_map")
    return bmap


def get_sparsity_info(block_row_indices: torch.Tensor, num_block_cols: int) -> dict:
    """(:106-120)"""
    num_block_rows = len(block_row_indices) - 1
    num_nonzero_blocks = int(block_row_indices[-1].item())
    total_blocks = num_block_rows * num_block_cols
    block_sparsity = 1 - num_nonzero_blocks / total_blocks
    return {
        "num_block_rows": num_block_rows,
        "num_block_cols": num_block_cols,
        "num_nonzero_blocks": num_nonzero_blocks,
        "total_blocks": total_blocks,
        "block_sparsity": block_sparsity,
        "theoretical_speedup": 1 / (1 - block_sparsity) if block_sparsity < 1 else float("inf"),
    }


# ---------------------------------------------------------------------------
# products
# ---------------------------------------------------------------------------
def bsr_transpose(blocks: torch.Tensor, bmap: torch.Tensor):
    """(blocks_t, bmap_t) of W^T: every block transposed (same order, so the indices stay valid) and the
    map transposed to [nbc, nbr]."""
    dev = L.require_device(blocks, bmap)
    nbr, nbc = bmap.shape
    bt = torch.empty_like(blocks)
    mt = torch.empty(nbc, nbr, dtype=torch.int32, device=dev)
    with _prof.region("sf_bsr_transpose", 2 * blocks.numel() * blocks.element_size() + 8 * bmap.numel(), "B", dev):
        L.check(L.lib().sf_bsr_transpose(L.ptr(blocks), L.dtype_code(blocks), blocks.shape[0], L.ptr(bmap), nbr, nbc,
                                         L.ptr(bt), L.ptr(mt), L.stream(dev)), "sf_bsr_transpose")
    return bt, mt


def _bsr_gemm(A: torch.Tensor, blocks: torch.Tensor, bmap: torch.Tensor, n_out: int, transposed: bool,
              out_dtype: torch.dtype) -> torch.Tensor:
    """A [M, K] . B^T with B = W (transposed=False, W [n_out, K]) or B = W^T (True, W [K, n_out]).

    bf16 products whose K is a multiple of 64 run the exact-skip kernel; the input gradient
    (transposed) then multiplies by the transposed block matrix (sf_bsr_transpose) with it."""
    dev = L.require_device(A, blocks, bmap)
    if blocks.dtype != A.dtype:
        raise TypeError(f"bsr: blocks dtype {blocks.dtype} != activation dtype {A.dtype}")
    M, K = A.shape
    if transposed and A.dtype == torch.bfloat16 and out_dtype == torch.bfloat16 and K % 64 == 0 and \
            tuple(bmap.shape) == (K // BLOCK, n_out // BLOCK):
        bt, mt = bsr_transpose(blocks, bmap)
        return _bsr_gemm(A, bt, mt, n_out, False, out_dtype)
    C = torch.empty(M, n_out, dtype=out_dtype, device=dev)
    d = L.GemmDesc()
    d.dtype = L.dtype_code(A)
    d.a_layout = L.LAYOUT_K
    d.b_layout = L.LAYOUT_MN if transposed else L.LAYOUT_K
    d.M, d.N, d.K1, d.K2 = M, n_out, K, 0
    d.A1, d.lda1 = L.ptr(A), K
    d.B1, d.ldb1 = L.ptr(blocks), 16
    d.bscale = 1.0
    d.C, d.ldc, d.c_dtype = L.ptr(C), n_out, L.dtype_code(C)
    d.b_format = L.BFMT_BSR16
    d.b_map, d.b_map_rows, d.b_map_cols = L.ptr(bmap), bmap.shape[0], bmap.shape[1]
    ws_bytes = L.lib().sf_gemm_workspace_size(L.byref(d))
    ws = None
    if ws_bytes:
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        d.workspace, d.workspace_bytes = ws.data_ptr(), ws_bytes
    with _prof.region("sf_gemm_bsr", 2.0 * M * n_out * K, "FLOP", dev):
        L.check(L.lib().sf_gemm(L.byref(d), L.stream(dev)), "sf_gemm (block-sparse)")
    return C


def bsr_sddmm(gy: torch.Tensor, x: torch.Tensor, bmap: torch.Tensor, nnz: int, out_dtype: torch.dtype) -> torch.Tensor:
    """gy^T x at the kept blocks of bmap: [max(nnz, 1), 16, 16] (the weight gradient of a block-sparse linear)."""
    dev = L.require_device(gy, x, bmap)
    T, out_f = gy.shape
    in_f = x.shape[1]
    blocks = torch.zeros(max(nnz, 1), 16, 16, dtype=out_dtype, device=dev)
    d = L.GemmDesc()
    d.dtype = L.dtype_code(gy)
    d.a_layout, d.b_layout = L.LAYOUT_MN, L.LAYOUT_MN
    d.M, d.N, d.K1, d.K2 = out_f, in_f, T, 0
    d.A1, d.lda1 = L.ptr(gy), out_f
    d.B1, d.ldb1 = L.ptr(x), in_f
    d.bscale = 1.0
    d.c_dtype = L.dtype_code(blocks)
    d.ldc = in_f
    d.c_blocks, d.c_map = L.ptr(blocks), L.ptr(bmap)
    d.c_map_rows, d.c_map_cols = bmap.shape[0], bmap.shape[1]
    with _prof.region("sf_gemm_bsr", 2.0 * out_f * in_f * T, "FLOP", dev):
        L.check(L.lib().sf_gemm(L.byref(d), L.stream(dev)), "sf_gemm (block-sparse SDDMM)")
    return blocks


class _BsrLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, blocks, bmap, out_f, in_f):
        ctx.save_for_backward(x2, blocks, bmap)
        ctx.out_f, ctx.in_f = out_f, in_f
        return _bsr_gemm(x2, blocks, bmap, out_f, False, x2.dtype)

    @staticmethod
    def backward(ctx, gy):
        x2, blocks, bmap = ctx.saved_tensors
        gy = gy.contiguous().to(x2.dtype)
        gx = _bsr_gemm(gy, blocks, bmap, ctx.in_f, True, x2.dtype) if ctx.needs_input_grad[0] else None
        gb = bsr_sddmm(gy, x2, bmap, blocks.shape[0], blocks.dtype) if ctx.needs_input_grad[1] else None
        return gx, gb, None, None, None


def bsr_linear(x: torch.Tensor, blocks: torch.Tensor, block_map: torch.Tensor, out_features: int,
               in_features: int, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x W^T (+ bias) for a block-sparse-16 W, with gradients for x and for the kept blocks."""
    if tuple(block_map.shape) != (out_features // BLOCK, in_features // BLOCK) or out_features % BLOCK or \
            in_features % BLOCK:
        raise ValueError(f"block map {tuple(block_map.shape)} does not tile a {out_features} x {in_features} weight "
                         f"in {BLOCK} x {BLOCK} blocks")
    if x.shape[-1] != in_features:
        raise ValueError(f"input feature size {x.shape[-1]} != in_features {in_features}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, in_features).to(blocks.dtype).contiguous()
    y = _BsrLinear.apply(x2, blocks, block_map, out_features, in_features)
    if bias is not None:
        y = y + bias.to(y.dtype)
    return y.view(*lead, out_features)


class BlockSparseLinear(nn.Module):
    """Block-sparse linear layer (:290-470) on the MFMA block-sparse GEMM."""

    def __init__(self, sparse_blocks: torch.Tensor, block_row_indices: torch.Tensor,
                 block_col_indices: torch.Tensor, in_features: int, out_features: int,
                 bias: Optional[torch.Tensor] = None, block_size: int = 16, block_map: Optional[torch.Tensor] = None,
                 trainable: bool = False):
        super().__init__()
        if block_size != BLOCK:
            raise NotImplementedError(f"block_size {block_size}: only 16 is built on the MI355X path")
        self.in_features = in_features
        self.out_features = out_features
        self.block_size = block_size
        if trainable:
            self.sparse_blocks = nn.Parameter(sparse_blocks.contiguous())
        else:
            self.register_buffer("sparse_blocks", sparse_blocks.contiguous())
        self.register_buffer("block_row_indices", block_row_indices.contiguous())
        self.register_buffer("block_col_indices", block_col_indices.contiguous())
        nnz = int(block_row_indices[-1].item())
        if sparse_blocks.dim() != 3 or tuple(sparse_blocks.shape[1:]) != (block_size, block_size) or \
                sparse_blocks.shape[0] < max(nnz, 1) or block_col_indices.numel() != nnz:
            raise ValueError(f"sparse_blocks {tuple(sparse_blocks.shape)} / block_col_indices "
                             f"{tuple(block_col_indices.shape)} do not match the index's {nnz} blocks")
        if out_features % block_size or in_features % block_size or \
                block_row_indices.numel() != out_features // block_size + 1:
            raise ValueError("block_row_indices does not match out_features / block_size")
        if block_map is None:
            block_map = block_map_from_csr(self.block_row_indices, self.block_col_indices, in_features // block_size)
        self.register_buffer("block_map", block_map.contiguous())
        if bias is not None:
            self.register_buffer("bias", bias.contiguous())
        else:
            self.bias = None
        self.sparsity_info = get_sparsity_info(block_row_indices, in_features // block_size)

    @classmethod
    def from_dense(cls, weight: torch.Tensor, mask: torch.Tensor, bias: Optional[torch.Tensor] = None,
                   block_size: int = 16, dtype: torch.dtype = torch.bfloat16, trainable: bool = False):
        out_f, in_f = weight.shape
        blocks, rp, ci, bmap = convert_to_block_sparse(weight, mask, block_size, return_block_map=True)
        return cls(blocks.to(dtype), rp, ci, in_f, out_f, bias.to(dtype) if bias is not None else None, block_size,
                   block_map=bmap, trainable=trainable)

    @classmethod
    def from_sparse_linear(cls, sparse_linear_module, block_size: int = 16, dtype: torch.dtype = torch.bfloat16):
        weight = sparse_linear_module.weight.data
        mask = sparse_linear_module.hard_mask if hasattr(sparse_linear_module, "hard_mask") else \
            sparse_linear_module.mask.data
        bias = sparse_linear_module.bias.data if sparse_linear_module.bias is not None else None
        return cls.from_dense(weight, mask, bias, block_size, dtype)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return bsr_linear(x, self.sparse_blocks, self.block_map, self.out_features, self.in_features, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, block_size={self.block_size}, "
                f"sparsity={self.sparsity_info['block_sparsity']:.1%}, "
                f"nnz_blocks={self.sparsity_info['num_nonzero_blocks']}")


def convert_model_to_block_sparse(model: nn.Module, block_size: int = 16, target_modules: Optional[list] = None,
                                  verbose: bool = True, dtype: torch.dtype = torch.bfloat16) -> nn.Module:
    """Replace every SparseLinear-like module (has `mask` and `weight`) by a BlockSparseLinear (:476-525).

    dtype (an addition to the reference's signature) is the block storage and compute dtype."""
    converted = 0
    for name, module in list(model.named_modules()):
        if hasattr(module, "hard_mask") or (hasattr(module, "mask") and hasattr(module, "weight")):
            if target_modules is not None and not any(t in name for t in target_modules):
                continue
            try:
                parent_name = ".".join(name.split(".")[:-1])
                attr = name.split(".")[-1]
                parent = model.get_submodule(parent_name) if parent_name else model
                layer = BlockSparseLinear.from_sparse_linear(module, block_size, dtype)
                setattr(parent, attr, layer)
                if verbose:
                    info = layer.sparsity_info
                    print(f"[convert] {name}: sparsity={info['block_sparsity']:.1%}, "
                          f"nnz_blocks={info['num_nonzero_blocks']}/{info['total_blocks']}")
                converted += 1
            except Exception as e:  # the reference reports and continues
                if verbose:
                    print(f"[convert] {name}: FAILED - {e}")
    if verbose:
        print(f"[convert] Total converted: {converted} layers")
    return model
