"""The skinny bf16 products of sf_gemm (one side of C at most 64: the SLoRB terms) against float32 products.

The SLoRB bypass of SparseLinear (legacy/sparse_modeling.py:790-794 and its
autograd) multiplies by the rank-r projections: z = x P^T and dz = dy S
(N = r), dP = dz^T x (M = r) and dS = dy^T z (N = r).  These run on a
128 x 64-tile kernel with split-K; C's short side may be its columns or its
rows.  Bar: bf16 outputs within 2^-8 of each element's magnitude plus 1e-3
of the output scale (one bf16 rounding of an f32 sum), f32 outputs within
1e-5 of the scale; the split-K reduce's epilogue (accumulate) applies.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lin():
    from sparseforge_amd import linear as lin

    return lin


def _check(got, ref, bf16_out=True):
    ref = ref.float()
    scale = float(ref.abs().max())
    err = (got.float() - ref).abs()
    if bf16_out:
        bound = 2.0 ** -8 * ref.abs() + 1e-3 * scale
    else:
        bound = torch.full_like(ref, 1e-5 * scale)
    assert bool((err <= bound).all()), float((err / (bound + 1e-30)).max())


def _rand(g, *shape, dev, s=1.0):
    return (torch.randn(*shape, generator=g, device=dev) * s).to(torch.bfloat16)


@pytest.mark.parametrize("T,K,r", [(8192, 4096, 64), (8192, 11008, 64), (1000, 200, 64), (777, 4096, 32),
                                   (8192, 520, 48)])
def test_z_and_dz_products(cuda_device, T, K, r):
    """z = x P^T (A K-contiguous, B K-contiguous) and dz = dy S (B N-contiguous), N = r."""
    lin = _lin()
    g = torch.Generator(device=cuda_device).manual_seed(T + K + r)
    x = _rand(g, T, K, dev=cuda_device)
    P = _rand(g, r, K, dev=cuda_device, s=0.05)
    S = _rand(g, K, r, dev=cuda_device, s=0.05)
    _check(lin.mm_nt(x, P), x.float() @ P.float().t())
    _check(lin.mm_nn(x, S), x.float() @ S.float())
    _check(lin.mm_nt(x, P, out_dtype=torch.float32), x.float() @ P.float().t(), bf16_out=False)


@pytest.mark.parametrize("T,N,r", [(8192, 4096, 64), (8192, 11008, 64), (1000, 200, 64), (4096, 776, 16)])
def test_dP_and_dS_products(cuda_device, T, N, r):
    """dP = dz^T x (C's rows are the short side: M = r) and dS = dy^T z (N = r); both operands
    M/N-contiguous, K = tokens."""
    lin = _lin()
    g = torch.Generator(device=cuda_device).manual_seed(T * 3 + N + r)
    dz = _rand(g, T, r, dev=cuda_device)
    x = _rand(g, T, N, dev=cuda_device)
    _check(lin.mm_tn(dz, x), dz.float().t() @ x.float())
    _check(lin.mm_tn(x, dz), x.float().t() @ dz.float())
    _check(lin.mm_tn(dz, x, out_dtype=torch.float32), dz.float().t() @ x.float(), bf16_out=False)


def test_both_sides_short_and_accumulate(cuda_device):
    lin = _lin()
    g = torch.Generator(device=cuda_device).manual_seed(5)
    a = _rand(g, 48, 4096, dev=cuda_device)
    b = _rand(g, 56, 4096, dev=cuda_device)
    _check(lin.mm_nt(a, b), a.float() @ b.float().t())
    # accumulate: C += A B^T through the split-K reduce's epilogue (the ggy += u S^T term of the HVP)
    x = _rand(g, 2048, 4096, dev=cuda_device)
    P = _rand(g, 64, 4096, dev=cuda_device, s=0.05)
    c0 = torch.randn(2048, 64, generator=g, device=cuda_device)
    c = c0.clone()
    lin.mm_nt(x, P, out=c, accumulate=True)
    _check(c, c0 + x.float() @ P.float().t(), bf16_out=False)
