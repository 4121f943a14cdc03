"""The cfg1 chain at full size on the GPU, stage by stage against the oracle.

cfg1 (GPT-2-small MLP, fp32): W [3072, 768] ~ N(0, 0.02), x [8 x 1024 tokens, 768] ~ N(0, 1), seed 0;
the Hessian diagonal from 4 Rademacher probes of Hutchinson's estimator on the quadratic loss
1/2 ||y - t||^2 (update_hessian_hutchinson, legacy/utils.py:714-869); scores |W| sqrt(H); the
structured 2:4 soft mask at temperature 0.5 from those scores (_compute_joint_gate_target,
legacy/utils.py:536-613) and its hard top-2 projection (_hard_mask_from_soft,
legacy/sparse_modeling.py:720-735); then the SparseLinear forward and backward with SLoRB rank 16
(:737-796, :56-132) under the soft mask (hardening_x = 1) and the hard mask (hardening_x = 0).

Each stage takes the device's output of the stage before it, so each bar is that stage's own:
* Hessian diagonal after each probe: within 1e-5 of its largest value of oracle.hutchinson
  (update of quadratic_hvp = v X^T X under the straight-through backward), the probes injected;
* scores: |W| sqrt(H) in float32 (torch on the device) within one ulp of numpy's correctly rounded
  value; the gate stage then takes the device's scores;
* gate target: within 1e-6 of oracle.masks.joint_gate_target;
* hard top-2: the device's projection of its own soft mask bit for bit equal to the oracle's
  projection of it; against the oracle's own soft mask only near-ties may differ;
* forward / dX / dW / db / dP / dS: float32, within 1e-5 of each output's scale against float64
  products of the same operands (oracle.linear).
"""
import numpy as np
import pytest
import torch

from conftest import gemm_err
from oracle import hutchinson as oh
from oracle import linear as ol
from oracle import masks as om
from test_gpu_masks import _hard_parity

pytestmark = pytest.mark.gpu

OUT, IN, TOKENS, RANK, PROBES = 3072, 768, 8 * 1024, 16, 4


def test_cfg1_chain_full_size(cuda_device):
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd import utils as U

    print("[cfg1] building W [3072, 768], x [8192, 768], SLoRB rank 16", flush=True)
    kw = dict(mask_type="structured", N=2, M=4, hard_mask_type="match", mask_metric="hessian_ratio",
              sparsity_warmup_steps=0, mask_update_period=1, temp_init=0.5, beta=0.99, SLoRB=True,
              SLoRB_k=IN // RANK, SLoRB_init_type="mean", trainable_projection=True)
    cfg = sm.SparseLinearConfig(**kw)
    cfg.enable_hutchinson = True
    layer = sm.SparseLinear(IN, OUT, sparselinear_config=cfg, bias=True).to(cuda_device)
    g = torch.Generator().manual_seed(0)
    W = torch.randn(OUT, IN, generator=g) * 0.02
    x = torch.randn(TOKENS, IN, generator=g)
    t = torch.randn(TOKENS, OUT, generator=g)
    S0 = torch.randn(OUT, RANK, generator=g) * 0.01
    b0 = torch.randn(OUT, generator=g) * 0.01
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.bias.copy_(b0)
        layer.initialize()
        layer.hessian_diag.zero_()
        layer.init_SLoRB()
        layer.SLoRB_Weight.copy_(S0)
    assert layer.x_proj.shape == (RANK, IN) and layer.SLoRB_Weight.shape == (OUT, RANK)
    xd = x.to(cuda_device)

    # 1. Hutchinson: four probes on one graph (retain_graph), as four update_hessian_hutchinson calls
    loss = 0.5 * ((layer(xd) - t.to(cuda_device)) ** 2).sum()
    H = np.zeros((OUT, IN), np.float32)
    xn = x.numpy()
    for j in range(PROBES):
        v = (torch.randint(0, 2, (OUT, IN), generator=g).float() * 2 - 1)
        U.update_hessian_hutchinson(torch.nn.Sequential(layer), loss, probes=[v])
        H = oh.update(H, oh.quadratic_hvp(xn, v.numpy()).astype(np.float32), v.numpy(), 0.99)
        got = layer.hessian_diag.detach().cpu().numpy()
        err = float(np.abs(got - H).max() / np.abs(H).max())
        print(f"[cfg1] Hutchinson probe {j}: max rel err {err:.2e}", flush=True)
        assert err <= 1e-5, (j, err)
    layer.zero_grad(set_to_none=True)
    del loss

    # 2. scores |W| sqrt(H) from the device's H
    Hd = layer.hessian_diag.detach()
    scores = layer.weight.detach().abs() * torch.sqrt(Hd)
    Hn, Wn = Hd.cpu().numpy(), layer.weight.detach().cpu().numpy()
    s_ref = (np.abs(Wn) * np.sqrt(Hn)).astype(np.float32)
    s_dev = scores.cpu().numpy()
    np.testing.assert_allclose(s_dev, s_ref, rtol=2.0 ** -23, atol=0)

    # 3. structured 2:4 soft mask at T = 0.5 from the scores
    G = U._compute_joint_gate_target(layer, scores, 0)
    assert layer._temperature(0) == 0.5
    G_ref = om.joint_gate_target(om.full_config(**kw), 0, s_dev, layer.mask.detach().cpu().numpy(), None, None)
    Gn = G.cpu().numpy()
    d = float(np.abs(Gn - G_ref).max())
    print(f"[cfg1] gate target max |d| {d:.2e}", flush=True)
    assert d <= 1e-6

    # 4. hard top-2 of each group of 4
    hard = layer._hard_mask_from_soft(G).cpu().numpy()
    assert np.array_equal(hard, om.hard_mask_from_soft(Gn, "structured", 2, 4))
    assert (hard.reshape(OUT, IN // 4, 4).sum(-1) == 2).all()
    _hard_parity(Gn, G_ref, 1e-6, 0, 0, "cfg1 top-2")

    # 5. forward / backward with SLoRB under the soft mask and under the hard mask
    with torch.no_grad():
        layer.mask.copy_(G)
    P, S = layer.x_proj.detach().cpu().numpy(), layer.SLoRB_Weight.detach().cpu().numpy()
    gy = torch.randn(TOKENS, OUT, generator=g)
    for hx in (1.0, 0.0):
        print(f"[cfg1] SparseLinear fwd/bwd at hardening_x={hx}", flush=True)
        layer.hardening_x = hx
        layer.zero_grad(set_to_none=True)
        xg = xd.clone().requires_grad_(True)
        y = layer(xg)
        y.backward(gy.to(cuda_device))
        E = ol.effective_mask(Gn, hx, "structured", 2, 4)
        y_ref = ol.forward(xn, Wn, E, b0.numpy(), 1.0, P, S, dtype=np.float64)
        g_ref = ol.backward(xn, Wn, E, gy.numpy(), True, P, S, dtype=np.float64)
        for name, got, ref in (("y", y, y_ref), ("dx", xg.grad, g_ref["dx"]), ("dW", layer.weight.grad, g_ref["dW"]),
                               ("db", layer.bias.grad, g_ref["db"]), ("dP", layer.x_proj.grad, g_ref["dP"]),
                               ("dS", layer.SLoRB_Weight.grad, g_ref["dS"])):
            err = gemm_err(got, torch.from_numpy(np.asarray(ref)), torch.float32)
            assert err <= 1.0, (hx, name, err)
