"""The mixed-mode effective mask a SparseLinear keeps between forwards is rebuilt whenever the mask changes.

The reference projects hard(mask) on every forward (legacy/sparse_modeling.py:759-771); the
build keeps the projection (or hx * mask + (1 - hx) * hard(mask)) per layer while the mask's
storage, version counter and the projection parameters are unchanged.  Each case below runs a
forward, changes something the projection depends on (the library's fused mask update writing the
mask in place, a torch in-place write, a new hardening_x, a block hard type's whole-tensor
projection) and checks that the next forward is bit-identical to the same layer's forward with
the cache emptied first.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _layer(dev, dtype, hard_mask_type="nm_2_4", in_f=128, out_f=64, **kw):
    from sparseforge_amd import sparse_modeling as sm

    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type=hard_mask_type,
                                mask_metric="hessian_ratio", sparsity_warmup_steps=0, mask_update_period=1,
                                tau_sample_size=1 << 20, **kw)
    lin = sm.SparseLinear(in_f, out_f, sparselinear_config=cfg, bias=True).to(dtype).to(dev)
    g = torch.Generator().manual_seed(5)
    with torch.no_grad():
        lin.weight.copy_((torch.randn(out_f, in_f, generator=g) * 0.02).to(dtype))
        lin.mask.copy_(torch.rand(out_f, in_f, generator=g).to(dtype))
        lin.hessian_diag.copy_((torch.rand(out_f, in_f, generator=g) * 1e-3 + 1e-6).to(dtype))
    return lin


def _fresh(lin, x):
    """The layer's forward with its effective-mask cache emptied first (what the reference computes)."""
    lin.__dict__.get("_eff_cache", {}).clear()
    with torch.no_grad():
        return lin(x).clone()


def _cached(lin, x):
    with torch.no_grad():
        return lin(x).clone()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("hx", [0.0, 0.4])
def test_cache_follows_library_mask_update(cuda_device, dtype, hx):
    lin = _layer(cuda_device, dtype)
    lin.hardening_x = hx
    x = torch.randn(96, 128, device=cuda_device).to(dtype)
    y0 = _cached(lin, x)
    assert lin._eff_cache, "mixed mode keeps its effective mask"
    assert torch.equal(_cached(lin, x), y0), "same mask: same output"
    before = lin.mask.detach().clone()
    lin.update_mask(step=1)  # the fused device update writes the mask through its raw pointer
    lin.hardening_x = hx     # (the update also advances hardening_x on its schedule: pin it)
    assert not torch.equal(lin.mask, before)
    y1 = _cached(lin, x)
    assert torch.equal(y1, _fresh(lin, x))
    assert not torch.equal(y1, y0)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_cache_follows_torch_inplace_write_and_hx(cuda_device, dtype):
    lin = _layer(cuda_device, dtype)
    lin.hardening_x = 0.0
    x = torch.randn(64, 128, device=cuda_device).to(dtype)
    y0 = _cached(lin, x)
    with torch.no_grad():
        lin.mask.copy_(1.0 - lin.mask)  # reverses every group's order: a different 2:4 projection
    y1 = _cached(lin, x)
    assert torch.equal(y1, _fresh(lin, x)) and not torch.equal(y1, y0)
    lin.hardening_x = 0.5
    y2 = _cached(lin, x)
    assert torch.equal(y2, _fresh(lin, x)) and not torch.equal(y2, y1)


def test_cache_follows_block_hard_type(cuda_device):
    lin = _layer(cuda_device, torch.float32, hard_mask_type="block16", in_f=64, out_f=48)
    lin.hardening_x = 0.0
    x = torch.randn(32, 64, device=cuda_device)
    y0 = _cached(lin, x)
    assert "hard" in lin._eff_cache
    with torch.no_grad():
        lin.mask.copy_(torch.flip(lin.mask, dims=[1]))
    y1 = _cached(lin, x)
    assert torch.equal(y1, _fresh(lin, x)) and not torch.equal(y1, y0)


def test_cache_gradients_match_uncached(cuda_device):
    """Forward + backward through the cached byte mask (hx = 0, bf16: the 2:4 sparse forward) equal the
    uncached call's, and the saved tensors survive a mask update between two steps."""
    lin = _layer(cuda_device, torch.bfloat16, in_f=256, out_f=128)
    lin.hardening_x = 0.0
    x = torch.randn(128, 256, device=cuda_device).to(torch.bfloat16)
    gy = torch.randn(128, 128, device=cuda_device).to(torch.bfloat16)
    grads = []
    for clear in (True, False, False):
        if clear:
            lin.__dict__.get("_eff_cache", {}).clear()
        lin.weight.grad = None
        y = lin(x)
        y.backward(gy)
        grads.append((y.detach().clone(), lin.weight.grad.clone()))
    for y, gw in grads[1:]:
        assert torch.equal(y, grads[0][0]) and torch.equal(gw, grads[0][1])
