"""GPU checks at the benchmark's full sizes, through size-independent properties and torch's
own float32 GPU results (the float64 CPU oracle would take minutes at these sizes).

* SparseLinear fwd / dX / dW / dP / dS at the q/k/v/o, gate/up and down shapes of a
  LLaMA-2-7B layer (T = 8192) with the hard 2:4 mask and SLoRB rank 64: against torch
  float32 products of the same bf16 operands, each element within bf16 rounding
  (2^-7 of its magnitude plus 2^-12 of the output scale, plus one ulp of each term of
  the bf16 SLoRB intermediates z = X P^T and dz = dY S).
* the fused mask update over a full [11008, 4096] layer: the new mask stays in [0, 1], its
  hard 2:4 projection keeps exactly two of every four, and the flip count equals the number
  of changed hard-mask entries counted independently.
* the distillation KL over the full [16384, 32000] logits: against torch's float32
  log-softmax KL rounded to the logits' dtype, within one bf16 ulp.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu


def within_bf16_rounding(got, ref, extra=None) -> float:
    """Largest ratio of |got - ref| to the elementwise bound 2^-7 |ref| + 2^-12 max|ref|: a bf16 result
    of a float32 accumulation is within half an ulp (2^-9 relative) of the exact value; a dropped 8-wide
    k chunk at K = 4096 moves an element by about 4e-2 of the output scale, 160 times the absolute term.
    `extra`: the elementwise effect of one ulp (2^-7 relative at most) of a bf16 intermediate, whose two
    float32 accumulations may round to neighbouring bf16 values."""
    got, ref = got.detach().float(), ref.detach().float()
    bound = ref.abs() * 2.0 ** -7 + ref.abs().max() * 2.0 ** -12
    if extra is not None:
        bound = bound + extra
    return float(((got - ref).abs() / bound).max())


@pytest.mark.parametrize("in_f,out_f", [(4096, 4096), (4096, 11008), (11008, 4096)])
def test_sparse_linear_full_shape(cuda_device, in_f, out_f):
    """The seven cfg2 shapes (q/k/v/o, gate/up, down) with SLoRB at rank 64 (the block-sum projection of
    init_SLoRB, k = in / 64): forward, dX, dW, dP, dS against torch float32 products."""
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd.linear import masked_linear

    print(f"[fullsize] linear {in_f}->{out_f} + SLoRB r=64", flush=True)
    T, R = 8192, 64
    k = in_f // R
    g = torch.Generator(device=cuda_device).manual_seed(in_f + out_f)
    x = torch.randn(T, in_f, generator=g, device=cuda_device).to(torch.bfloat16).requires_grad_(True)
    W = (torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02).to(torch.bfloat16).requires_grad_(True)
    P = torch.zeros(R, in_f, device=cuda_device)
    P[torch.arange(R, device=cuda_device)[:, None], torch.arange(R, device=cuda_device)[:, None] * k
      + torch.arange(k, device=cuda_device)] = 1.0
    P = P.to(torch.bfloat16).requires_grad_(True)
    S = (torch.randn(out_f, R, generator=g, device=cuda_device) * 0.01).to(torch.bfloat16).requires_grad_(True)
    soft = torch.rand(out_f, in_f, generator=g, device=cuda_device)
    y = masked_linear(x, W, None, soft, "mix", 0.0, L.HARD_NM_TAIL_KEEP, 2, 1.0, P=P, S=S)
    gy = torch.randn(T, out_f, generator=g, device=cuda_device).to(torch.bfloat16)
    y.backward(gy)
    E = K.hard_mask(soft, L.HARD_NM_TAIL_KEEP, 2, 4).float()
    Wm = W.detach().float() * E
    xf, gyf, Pf, Sf = x.detach().float(), gy.float(), P.detach().float(), S.detach().float()
    z = xf @ Pf.t()
    dz = gyf @ Sf
    # each bf16 result within rounding of the float32 product, the SLoRB intermediates z and dz rounded to
    # bf16 first as the bf16 path (and the reference under autocast) stores them
    zb, dzb = z.bfloat16().float(), dz.bfloat16().float()
    ulp = 2.0 ** -7
    checks = (("y", y, xf @ Wm.t() + zb @ Sf.t(), (zb.abs() @ Sf.abs().t()) * ulp),
              ("dX", x.grad, gyf @ Wm + dzb @ Pf, (dzb.abs() @ Pf.abs()) * ulp),   # dY (W . M) + (dY S) P
              ("dW", W.grad, gyf.t() @ xf, None),                                   # dY^T X (unmasked)
              ("dP", P.grad, dzb.t() @ xf, (dzb.abs().t() @ xf.abs()) * ulp),       # (dY S)^T X
              ("dS", S.grad, gyf.t() @ zb, (gyf.abs().t() @ zb.abs()) * ulp))       # dY^T (X P^T)
    for name, got, ref, extra in checks:
        err = within_bf16_rounding(got, ref, extra)
        assert err <= 1.0, (name, err)


def test_update_mask_full_layer_properties(cuda_device):
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd import sparse_modeling as sm

    print("[fullsize] update_mask 11008x4096", flush=True)
    out_f, in_f = 11008, 4096
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                sparsity_warmup_steps=0, mask_update_period=1, tau_sample_size=262144,
                                temp_init=0.5)
    cfg.enable_hutchinson = True
    layer = sm.SparseLinear(in_f, out_f, sparselinear_config=cfg, bias=False).to(cuda_device)
    g = torch.Generator(device=cuda_device).manual_seed(5)
    with torch.no_grad():
        layer.weight.copy_(torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02)
        layer.hessian_diag.copy_(torch.rand(out_f, in_f, generator=g, device=cuda_device) * 1e-3 + 1e-6)
        layer.mask.copy_(torch.rand(out_f, in_f, generator=g, device=cuda_device))
    before = K.hard_mask(layer.mask.detach().contiguous(), L.HARD_NM_TAIL_KEEP, 2, 4)
    layer.update_mask(10)
    m = layer.mask.detach()
    assert bool(((m >= 0) & (m <= 1)).all())
    after = K.hard_mask(m.contiguous(), L.HARD_NM_TAIL_KEEP, 2, 4)
    kept = after.view(out_f, in_f // 4, 4).sum(-1)
    assert bool((kept == 2).all())
    changed = int((before != after).sum())
    assert int(layer.weight.flipped_mask) == changed


def test_distill_kl_full_logits(cuda_device):
    from sparseforge_amd.distill import chunked_kl_loss

    print("[fullsize] kl 16384x32000", flush=True)
    g = torch.Generator(device=cuda_device).manual_seed(9)
    s = (torch.randn(16384, 32000, generator=g, device=cuda_device) * 4).to(torch.bfloat16)
    t = (torch.randn(16384, 32000, generator=g, device=cuda_device) * 4).to(torch.bfloat16)
    loss = chunked_kl_loss(s, t, 2)
    ref = 0.0
    for i in range(0, 16384, 2048):  # torch float32 log-softmax KL per 2048-row chunk (the reference's chunking)
        ls = torch.log_softmax(s[i:i + 2048].float() / 2, -1)
        lt = torch.log_softmax(t[i:i + 2048].float() / 2, -1)
        ref += float((lt.exp() * (lt - ls)).sum(dtype=torch.float64))
    ref = ref * 4 / 16384
    # the loss comes back in the logits' dtype (bf16 here), as the reference returns it
    want = float(torch.tensor(ref, dtype=torch.float32).to(loss.dtype))
    assert float(loss) == pytest.approx(want, rel=8e-3)  # within one bf16 ulp of the rounded float32 value


@pytest.mark.parametrize("density", [0.5, 0.25])
def test_block_sparse_full_shape(cuda_device, density):
    """cfg4: the block-sparse-16 forward, input gradient and SDDMM weight gradient at W [11008, 4096],
    x [8192, 4096] (bf16), against torch float32 products of the dense masked weight; each bf16 result
    within rounding of the float32 product, elementwise."""
    from sparseforge_amd import block_sparse as bs

    print(f"[fullsize] block-sparse d={density}", flush=True)
    out_f, in_f, T = 11008, 4096, 8192
    bm = torch.rand(out_f // 16, in_f // 16, generator=torch.Generator().manual_seed(1)) < density
    g = torch.Generator(device=cuda_device).manual_seed(3)
    W = (torch.randn(out_f, in_f, generator=g, device=cuda_device) * 0.02).to(torch.bfloat16)
    M = bm.to(cuda_device).repeat_interleave(16, 0).repeat_interleave(16, 1).to(torch.bfloat16)
    x = torch.randn(T, in_f, generator=g, device=cuda_device).to(torch.bfloat16)
    gy = torch.randn(T, out_f, generator=g, device=cuda_device).to(torch.bfloat16)
    blocks, rp, ci, bmap = bs.convert_to_block_sparse(W, M, return_block_map=True)
    nnz = ci.numel()
    y = bs._bsr_gemm(x, blocks, bmap, out_f, False, torch.bfloat16)
    dx = bs._bsr_gemm(gy, blocks, bmap, in_f, True, torch.bfloat16)
    dwb = bs.bsr_sddmm(gy, x, bmap, nnz, torch.bfloat16)
    Wm = (W * M).float()
    xf, gyf = x.float(), gy.float()
    assert within_bf16_rounding(y, xf @ Wm.t()) <= 1.0
    assert within_bf16_rounding(dx, gyf @ Wm) <= 1.0
    dW = gyf.t() @ xf
    # the kept blocks of dW in CSR order (row-major over block rows, ascending columns)
    rows = torch.repeat_interleave(torch.arange(out_f // 16, device=cuda_device), (rp[1:] - rp[:-1]).long())
    ref_blocks = dW.view(out_f // 16, 16, in_f // 16, 16).permute(0, 2, 1, 3)[rows, ci.long()]
    assert within_bf16_rounding(dwb[:nnz], ref_blocks) <= 1.0
