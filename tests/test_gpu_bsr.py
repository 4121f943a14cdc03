"""GPU parity of the block-sparse-16 path (sf_bsr_* build kernels, block-sparse sf_gemm modes).

Bar: the compressed index (row_ptr, col_idx, block map) and the blocks are
bit-exact against oracle/bsr.py and the reference's own output
(tests/golden/ref_bsr_basic_f32.npz); products (y = x W^T, dx = dy W, the
SDDMM weight gradient at kept blocks) against the float64 oracle, elementwise
(conftest.gemm_err): bf16 within 2^-7 of each element plus 2^-12 of the output
scale, f32 within 1e-5 of the output scale.
"""
import numpy as np
import pytest
import torch

from conftest import BF16_ULP, gemm_err, load_golden
from oracle import bsr as ob

pytestmark = pytest.mark.gpu


def _bs():
    from sparseforge_amd import block_sparse as bs

    return bs


def _block_mask(g, out_f, in_f, density, elem_zero=0.0):
    bm = torch.rand(out_f // 16, in_f // 16, generator=g) < density
    M = bm.repeat_interleave(16, 0).repeat_interleave(16, 1).float()
    if elem_zero:
        M = M * (torch.rand(out_f, in_f, generator=g) >= elem_zero).float()
    return M


def _check_index(bs, W, M, dev):
    blocks, rp, ci, bmap = bs.convert_to_block_sparse(W.to(dev), M.to(dev), return_block_map=True)
    sw = (W * M).float().numpy()  # the product rounds in the promoted dtype, as the kernel's
    eb, erp, eci = ob.convert(sw, np.ones_like(sw))
    assert np.array_equal(rp.cpu().numpy(), erp) and np.array_equal(ci.cpu().numpy(), eci)
    assert np.array_equal(blocks.float().cpu().numpy(), eb, equal_nan=True)
    nbr, nbc = W.shape[0] // 16, W.shape[1] // 16
    assert np.array_equal(bmap.cpu().numpy(), ob.block_map(erp, eci, nbr, nbc))
    return blocks, rp, ci, bmap


def test_convert_matches_reference_golden(cuda_device):
    bs = _bs()
    r = load_golden("bsr_basic_f32")
    blocks, rp, ci = bs.convert_to_block_sparse(torch.from_numpy(r["W"]).to(cuda_device),
                                                torch.from_numpy(r["mask"]).to(cuda_device))
    assert np.array_equal(rp.cpu().numpy(), r["row_ptr"]) and np.array_equal(ci.cpu().numpy(), r["col_idx"])
    assert np.array_equal(blocks.cpu().numpy(), r["blocks"])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape,density", [((64, 96), 0.5), ((4096, 8192), 0.25), ((8192, 272), 0.6)])
def test_convert_bit_exact(cuda_device, dtype, shape, density):
    """Random block patterns with zeros inside kept blocks; 512 block columns / rows cross the 256-wide scans."""
    bs = _bs()
    g = torch.Generator().manual_seed(shape[0] + shape[1])
    W = torch.randn(*shape, generator=g).to(dtype)
    M = _block_mask(g, *shape, density, elem_zero=0.3).to(dtype)
    _check_index(bs, W, M, cuda_device)


def test_convert_nan_zero_and_soft_mask(cuda_device):
    bs = _bs()
    W = torch.ones(32, 48)
    W[3, 20] = float("nan")   # block (0, 1) holds a NaN: dropped
    W[16:32, 32:48] = 0.0     # block (1, 2) zero in W though kept by the mask: dropped
    M = torch.ones(32, 48)
    M[16:32, 0:16] = 0.0      # block (1, 0) pruned by the mask
    blocks, rp, ci, bmap = _check_index(bs, W, M, cuda_device)
    assert rp.tolist() == [0, 2, 3] and ci.tolist() == [0, 2, 1]
    # a soft mask: the kept values are the bf16 products
    g = torch.Generator().manual_seed(5)
    Wb = torch.randn(64, 64, generator=g).bfloat16()
    Ms = (torch.rand(64, 64, generator=g) * _block_mask(g, 64, 64, 0.5)).bfloat16()
    _check_index(bs, Wb, Ms, cuda_device)
    # nothing kept: one zero block and an empty index
    blocks, rp, ci = bs.convert_to_block_sparse(torch.zeros(32, 48, device=cuda_device),
                                                torch.ones(32, 48, device=cuda_device))
    assert tuple(blocks.shape) == (1, 16, 16) and not blocks.any() and rp.tolist() == [0, 0, 0] and ci.numel() == 0
    info = bs.get_sparsity_info(rp, 3)
    assert info["num_nonzero_blocks"] == 0 and info["block_sparsity"] == 1.0 and info["theoretical_speedup"] == float("inf")


def test_block_map_from_csr_and_validation(cuda_device):
    bs = _bs()
    rp = torch.tensor([0, 2, 2, 3], dtype=torch.int32, device=cuda_device)
    ci = torch.tensor([1, 3, 0], dtype=torch.int32, device=cuda_device)
    m = bs.block_map_from_csr(rp, ci, 4)
    assert np.array_equal(m.cpu().numpy(), ob.block_map(rp.cpu().numpy(), ci.cpu().numpy(), 3, 4))
    with pytest.raises(ValueError):
        bs.block_map_from_csr(torch.tensor([0, 3, 2], dtype=torch.int32, device=cuda_device), ci, 4)
    with pytest.raises(ValueError):
        bs.block_map_from_csr(torch.tensor([0, 1, 2, 4], dtype=torch.int32, device=cuda_device), ci, 4)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("T,out_f,in_f,density", [(512, 1024, 768, 0.5), (300, 272, 208, 0.25),
                                                  (1024, 2048, 4096, 0.5), (256, 512, 512, 0.0)])
def test_products(cuda_device, dtype, T, out_f, in_f, density):
    bs = _bs()
    g = torch.Generator().manual_seed(T + out_f + in_f)
    W = torch.randn(out_f, in_f, generator=g).to(dtype)
    M = _block_mask(g, out_f, in_f, density).to(dtype)
    x = torch.randn(T, in_f, generator=g).to(dtype)
    gy = torch.randn(T, out_f, generator=g).to(dtype)
    d = lambda t: t.to(cuda_device)
    blocks, rp, ci, bmap = bs.convert_to_block_sparse(d(W), d(M), return_block_map=True)
    nnz = ci.numel()
    eb, erp, eci = ob.convert((W * M).float().numpy(), np.ones((out_f, in_f), np.float32))
    xn, gyn = x.double().numpy(), gy.double().numpy()

    xg = d(x).requires_grad_(True)
    bp = blocks.clone().requires_grad_(True)
    y = bs.bsr_linear(xg, bp, bmap, out_f, in_f)
    ref_y = ob.forward(xn, eb, erp, eci, out_f, in_f)
    y.backward(d(gy))
    ref_dx = ob.input_grad(gyn, eb, erp, eci, out_f, in_f)
    if nnz == 0:
        assert not y.any() and not xg.grad.any() and not bp.grad.any()
        return
    assert gemm_err(y, ref_y, dtype) <= 1.0
    assert gemm_err(xg.grad, ref_dx, dtype) <= 1.0
    ref_dw = ob.sddmm_grad(gyn, xn, erp, eci)
    assert gemm_err(bp.grad[:nnz], ref_dw, dtype) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_block_sparse_linear_module(cuda_device, dtype):
    """from_dense / from_sparse_linear / convert_model_to_block_sparse against the dense masked layer."""
    bs = _bs()
    g = torch.Generator().manual_seed(3)
    out_f, in_f = 384, 256
    W = torch.randn(out_f, in_f, generator=g)
    M = _block_mask(g, out_f, in_f, 0.4)
    b = torch.randn(out_f, generator=g)
    x = torch.randn(2, 50, in_f, generator=g).to(dtype)
    prod = x.double() @ (W * M).to(dtype).double().t()
    ref = prod + b.to(dtype).double()
    # the bias is added to the rounded product, as the reference's layer adds it: one more half ulp
    extra = prod.abs() * BF16_ULP / 2 if dtype == torch.bfloat16 else None

    layer = bs.BlockSparseLinear.from_dense(W.to(cuda_device), M.to(cuda_device), b.to(cuda_device), dtype=dtype)
    got = layer(x.to(cuda_device))
    assert got.shape == (2, 50, out_f) and gemm_err(got, ref, dtype, extra) <= 1.0
    assert "sparsity=" in layer.extra_repr()

    class Holder(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.proj = torch.nn.Linear(in_f, out_f)
            self.proj.weight.data.copy_(W)
            self.proj.bias.data.copy_(b)
            self.proj.mask = torch.nn.Parameter(M.clone(), requires_grad=False)

    model = Holder().to(cuda_device)
    bs.convert_model_to_block_sparse(model, verbose=False, dtype=dtype)
    assert isinstance(model.proj, bs.BlockSparseLinear)
    assert gemm_err(model.proj(x.to(cuda_device)), ref, dtype, extra) <= 1.0


def test_rejects_bad_operands(cuda_device):
    bs = _bs()
    blocks, rp, ci, bmap = bs.convert_to_block_sparse(torch.ones(32, 32, device=cuda_device),
                                                      torch.ones(32, 32, device=cuda_device), return_block_map=True)
    with pytest.raises(TypeError):  # the products take one element dtype
        bs._bsr_gemm(torch.ones(4, 32, device=cuda_device), blocks.bfloat16(), bmap, 32, False, torch.float32)
    with pytest.raises(ValueError):  # a map that does not tile the weight
        bs.bsr_linear(torch.ones(4, 32, device=cuda_device), blocks, bmap[:1], 32, 32)
    with pytest.raises(ValueError):
        bs.bsr_linear(torch.ones(4, 48, device=cuda_device), blocks, bmap, 32, 32)
    with pytest.raises(ValueError):
        bs.convert_to_block_sparse(torch.ones(30, 32, device=cuda_device), torch.ones(30, 32, device=cuda_device))
    with pytest.raises(ValueError):
        bs.BlockSparseLinear(blocks[:1], rp, ci, 32, 32)  # fewer blocks than the index lists


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_bsr_transpose(cuda_device, dtype):
    """sf_bsr_transpose: every block transposed in place order and the map transposed, so the pair is the
    block-sparse form of (W . M)^T (the input gradient's operand)."""
    bs = _bs()
    g = torch.Generator().manual_seed(11)
    out_f, in_f = 160, 96
    W = torch.randn(out_f, in_f, generator=g).to(dtype)
    M = _block_mask(g, out_f, in_f, 0.4).to(dtype)
    blocks, rp, ci, bmap = bs.convert_to_block_sparse(W.to(cuda_device), M.to(cuda_device), return_block_map=True)
    bt, mt = bs.bsr_transpose(blocks, bmap)
    assert torch.equal(mt, bmap.t().contiguous())
    assert torch.equal(bt, blocks.transpose(1, 2).contiguous())
    Wt, Mt = (W * M).t().contiguous(), M.t().contiguous()
    b2, _rp2, _ci2, m2 = bs.convert_to_block_sparse(Wt.to(cuda_device), Mt.to(cuda_device), return_block_map=True)
    # the transposed pair describes the same matrix as converting (W . M)^T directly
    dense = torch.zeros(in_f // 16, out_f // 16, 16, 16, dtype=dtype, device=cuda_device)
    dense2 = torch.zeros_like(dense)
    kept = mt >= 0
    dense[kept] = bt[mt[kept].long()]
    dense2[m2 >= 0] = b2[m2[m2 >= 0].long()]
    assert torch.equal(dense, dense2)
