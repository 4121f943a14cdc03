"""init_SLoRB (legacy/sparse_modeling.py:830-872) against the reference's own output (CPU).

The fixtures record, for "sum" and "mean" initialisation and f32 / bf16 layers, the projection P
(the block-sum matrix: row r has ones on inputs [r k, (r + 1) k)) and the SLoRB weight S (the sum or
mean over each block of k inputs of the pruned part W (1 - mask)) that the reference computes from a
random weight and soft mask.  init_SLoRB is host torch code, so it runs here on CPU tensors.
Bar: bit for bit (P is 0/1; S is the same reduction over the same values in the same dtype).
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden


@pytest.mark.parametrize("case", ["slorb_init_sum_f32", "slorb_init_mean_f32", "slorb_init_mean_bf16"])
def test_init_slorb_matches_reference(case):
    from sparseforge_amd import sparse_modeling as sm

    r = load_golden(case)
    kw = ast.literal_eval(str(r["cfg"]))
    dtype = torch.bfloat16 if "bfloat16" in str(r["dtype"]) else torch.float32
    out_f, in_f = r["W"].shape
    layer = sm.SparseLinear(in_f, out_f, sparselinear_config=sm.SparseLinearConfig(**kw), bias=False).to(dtype)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(r["W"]).to(dtype))
        layer.mask.copy_(torch.from_numpy(r["mask"]).to(dtype))
    layer.init_SLoRB()
    assert layer.x_proj.dtype == dtype and layer.SLoRB_Weight.dtype == dtype
    assert layer.x_proj.requires_grad == bool(kw["trainable_projection"])
    np.testing.assert_array_equal(layer.x_proj.detach().float().numpy(), r["P"])
    np.testing.assert_array_equal(layer.SLoRB_Weight.detach().float().numpy(), r["S"])


def test_init_slorb_projection_of_linear_golden():
    """The linear fixture's P (ref_linear_slorb_f32, written after the reference's init_SLoRB) is what
    init_SLoRB builds for that layer."""
    from sparseforge_amd import sparse_modeling as sm

    r = load_golden("linear_slorb_f32")
    kw = ast.literal_eval(str(r["cfg"]))
    layer = sm.SparseLinear(32, 20, sparselinear_config=sm.SparseLinearConfig(**kw), bias=True)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(r["W"]))
        layer.mask.copy_(torch.from_numpy(r["mask"]))
    layer.init_SLoRB()
    np.testing.assert_array_equal(layer.x_proj.detach().numpy(), r["P"])
