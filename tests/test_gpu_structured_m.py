"""structured N:M with a group size other than 4 is refused on the device, loudly, in every entry point.

The reference projects any N:M (legacy/sparse_modeling.py:720-735 hard mask, :1164-1185
structured gate, :1531-1565 structured_topn penalty; SparseLinearConfig.N / M at :149-150).
The device kernels build groups of 4 only (the torch.topk tie order for k of 4 is a fixed
function of the group's weak ordering); any other M raises NotImplementedError naming the
supported shape, instead of silently projecting groups of 4.  Parts that never project (the
soft-mask forward at hardening_x = 1, the dense forward) run for any M.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev, N, M):
    from sparseforge_amd import sparse_modeling as sm

    cfg = sm.SparseLinearConfig(mask_type="structured", hard_mask_type="match", mask_metric="hessian_obd", N=N, M=M,
                                sparsity_warmup_steps=0, mask_update_period=1)
    lin = sm.SparseLinear(64, 32, sparselinear_config=cfg, bias=False).to(dev)
    g = torch.Generator().manual_seed(4)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(32, 64, generator=g) * 0.02)
        lin.mask.copy_(torch.rand(32, 64, generator=g))
        lin.hessian_diag.copy_(torch.rand(32, 64, generator=g) + 0.1)
    return lin


@pytest.mark.parametrize("N,M", [(2, 8), (4, 8), (1, 2)])
def test_structured_group_other_than_4_is_refused(cuda_device, N, M):
    lin = _layer(cuda_device, N, M)
    x = torch.randn(16, 64, device=cuda_device)
    # no projection: the soft-mask forward runs for any group size
    lin.hardening_x = 1.0
    y = lin(x)
    assert torch.isfinite(y).all()
    ref = x @ (lin.weight * lin.mask).t()
    assert torch.allclose(y, ref, rtol=1e-5, atol=1e-5)
    # every projection of groups of M refuses the shape
    lin.hardening_x = 0.5
    with pytest.raises(NotImplementedError, match=f"M={M}"):
        lin(x)
    with pytest.raises(NotImplementedError, match=f"M={M}"):
        lin._hard_mask_from_soft(lin.mask)
    with pytest.raises(NotImplementedError, match=f"M={M}"):
        lin.compute_gate_target(step=1)
    before = lin.mask.detach().clone()
    with pytest.raises(NotImplementedError, match=f"M={M}"):
        lin.update_mask(step=1)
    assert torch.equal(lin.mask, before), "a refused update leaves the mask unchanged"
