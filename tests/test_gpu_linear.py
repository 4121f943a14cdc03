"""GPU parity of the masked linear GEMMs (K1-K5) against a float64 CPU reference.

Bar (conftest.gemm_err): each bf16 result within 2^-7 of its own magnitude plus
2^-12 of the output scale of the float64 product of the same operands, the
operands rounded as the kernels and the reference round them (W.E, then W.E.s,
in the weight dtype; the SLoRB intermediates z = x P^T and dz = dy S in the
activation dtype, with one ulp of slack each); float32 results within 1e-5 of
the output scale.  Gradients follow the reference's STE semantics (dW unmasked,
no weight scale in dx, legacy/sparse_modeling.py:96-132).
"""
import numpy as np
import pytest
import torch

from conftest import BF16_ULP, bias_slack, gemm_err, load_golden

pytestmark = pytest.mark.gpu


def _lin():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import linear as lin

    return L, lin


def rel_err(got: torch.Tensor, ref: torch.Tensor) -> float:
    got = got.detach().double().cpu()
    ref = ref.detach().double().cpu()
    return float((got - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(256, 512, 384), (300, 136, 72), (1024, 768, 3072), (64, 4096, 8)])
def test_gemm_layouts(cuda_device, dtype, shape):
    L, lin = _lin()
    M, K, N = shape
    g = torch.Generator().manual_seed(M + K + N)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(N, K, generator=g).to(dtype)
    Bt = B.t().contiguous()
    At = A.t().contiguous()
    ref = A.double() @ B.double().t()
    d = lambda t: t.to(cuda_device)
    assert gemm_err(lin.mm_nt(d(A), d(B)), ref, dtype) <= 1.0
    assert gemm_err(lin.mm_nn(d(A), d(Bt)), ref, dtype) <= 1.0
    vec = 8 if dtype == torch.bfloat16 else 4
    if M % vec:
        # an M-contiguous operand needs M to be a multiple of the 16-byte vector: rejected on the host
        with pytest.raises(ValueError, match="multiples"):
            lin.mm_tn(d(At), d(Bt))
    else:
        assert gemm_err(lin.mm_tn(d(At), d(Bt)), ref, dtype) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gemm_mask_scale_bias_and_segment(cuda_device, dtype):
    L, lin = _lin()
    g = torch.Generator().manual_seed(1)
    T, IN, OUT, R = 320, 256, 200, 16
    x = torch.randn(T, IN, generator=g).to(dtype)
    W = torch.randn(OUT, IN, generator=g).to(dtype)
    E = (torch.rand(OUT, IN, generator=g)).to(dtype)
    z = torch.randn(T, R, generator=g).to(dtype)
    S = torch.randn(OUT, R, generator=g).to(dtype)
    b = torch.randn(OUT, generator=g).to(dtype)
    d = lambda t: t.to(cuda_device)
    got = lin.mm_nt(d(x), d(W), bmask=d(E), bscale=1.5, A2=d(z), B2=d(S), K2=R, bias=d(b))
    # the masked operand as the reference forms it (legacy/sparse_modeling.py:79-81): w = W * E, then
    # w * scale, each rounded to the weight dtype
    Wm = W * E
    prod = x.double() @ (Wm * 1.5).double().t() + z.double() @ S.double().t()
    assert gemm_err(got, prod + b.double(), dtype, bias_slack(prod, dtype)) <= 1.0
    dx = lin.mm_nn(d(x[:, :OUT].contiguous()), d(W), bmask=d(E))
    assert gemm_err(dx, x[:, :OUT].double() @ Wm.double(), dtype) <= 1.0


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("shape", [(256, 512, 384), (300, 136, 72), (1024, 768, 3072)])
def test_gemm_byte_and_mask(cuda_device, dtype, shape):
    """A uint8 and-mask (0xFF keep / 0x00 prune) equals multiplying by the 0/1 mask, in both B layouts."""
    L, lin = _lin()
    M, K, N = shape
    g = torch.Generator().manual_seed(11 + M)
    A = torch.randn(M, K, generator=g).to(dtype)
    B = torch.randn(N, K, generator=g).to(dtype)
    keep = torch.rand(N, K, generator=g) < 0.5
    E8 = (keep.to(torch.uint8) * 255)
    ref = A.double() @ (B.double() * keep.double()).t()
    d = lambda t: t.to(cuda_device)
    got = lin.mm_nt(d(A), d(B), bmask=d(E8))
    assert gemm_err(got, ref, dtype) <= 1.0
    # input-grad layout: C = G . (B.E) with B [N, K] read N-contiguous
    G = torch.randn(M, N, generator=g).to(dtype)
    got2 = lin.mm_nn(d(G), d(B), bmask=d(E8))
    ref2 = G.double() @ (B.double() * keep.double())
    assert gemm_err(got2, ref2, dtype) <= 1.0
    # the same with the mask also given K-major ([K, N] here: B's columns are the GEMM's n)
    got3 = lin.mm_nn(d(G), d(B), bmask=d(E8), bmask_t=lin.transpose_u8(d(E8)))
    assert gemm_err(got3, ref2, dtype) <= 1.0


@pytest.mark.parametrize("shape", [(64, 64), (3, 5), (130, 67), (4096, 11008), (11008, 4096), (1, 1000)])
def test_transpose_u8_exact(cuda_device, shape):
    L, lin = _lin()
    g = torch.Generator().manual_seed(shape[0] * 7 + shape[1])
    E = torch.randint(0, 256, shape, generator=g, dtype=torch.int32).to(torch.uint8)
    got = lin.transpose_u8(E.to(cuda_device)).cpu()
    assert torch.equal(got, E.t().contiguous())


@pytest.mark.parametrize("M,N,K", [(512, 768, 1024), (300, 272, 208), (1024, 4096, 11008)])
def test_gemm_input_grad_kmajor_mask(cuda_device, M, N, K):
    """dx = G (W.E) with the byte mask copied K-major (bf16 direct kernel, transposed weight reads)."""
    L, lin = _lin()
    g = torch.Generator().manual_seed(M + N + K)
    G = torch.randn(M, K, generator=g).bfloat16()
    W = torch.randn(K, N, generator=g).bfloat16()   # [out = K, in = N]
    keep = torch.rand(K, N, generator=g) < 0.5
    E8 = keep.to(torch.uint8) * 255
    d = lambda t: t.to(cuda_device)
    got = lin.mm_nn(d(G), d(W), bmask=d(E8), bmask_t=lin.transpose_u8(d(E8)))
    ref = G.double() @ (W.double() * keep.double())
    assert gemm_err(got, ref, torch.bfloat16) <= 1.0
    plain = lin.mm_nn(d(G), d(W))
    assert gemm_err(plain, G.double() @ W.double(), torch.bfloat16) <= 1.0


@pytest.mark.parametrize("mdt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols", [64, 66, 4096])
def test_effective_mask_hard_bytes_bit_exact(cuda_device, mdt, cols):
    """sf_effective_mask(SF_EFF_HARD, uint8) is 0xFF exactly where the oracle's 2:4 projection keeps."""
    L, lin = _lin()
    from oracle import masks as om

    g = torch.Generator().manual_seed(cols)
    soft = torch.rand(37, cols, generator=g).to(mdt)
    soft[3, :8] = 1.0  # all-tie groups keep columns 2, 3
    got = lin.effective_mask(soft.to(cuda_device), torch.uint8, "hard", 0.0, L.HARD_NM_TAIL_KEEP, 2).cpu()
    ref = om.hard_mask_from_soft(soft.float().numpy(), "nm_2_4")
    assert torch.equal(got, torch.from_numpy((ref > 0.5).astype(np.uint8) * 255))


def _dense_reference(x, W, b, E, s, P, S, gy):
    """float64 products of FusedMaskedLinearSTE + SLoRB forward / backward (legacy/sparse_modeling.py:72-132,
    :790-794) over the operands rounded as the layer rounds them: w = W * E, then w * s, in the weight
    dtype (:79-81); z = x P^T and dz = dy S stored in the activation dtype.  Returns the references and,
    for bf16, the elementwise slack of one ulp of z or dz (two float32 sums may round to neighbours)."""
    dt = x.dtype
    Wm = W * E
    Ws = Wm * s if s != 1.0 else Wm
    xd, gyd, Pd, Sd = x.double(), gy.double(), P.double(), S.double()
    z = (xd @ Pd.t()).to(dt).double()
    dz = (gyd @ Sd).to(dt).double()
    prod = xd @ Ws.double().t() + z @ Sd.t()
    y = prod + b.double() if b is not None else prod
    # STE: dW = gy^T x (unmasked), dx = gy (W.E) without s
    ref = dict(y=y, dx=gyd @ Wm.double() + dz @ Pd, dW=gyd.t() @ xd, db=gyd.sum(0), dP=dz.t() @ xd,
               dS=gyd.t() @ z)
    u = BF16_ULP if dt == torch.bfloat16 else 0.0
    # y: the bias is added to the rounded product (as the reference's out + bias)
    slack = dict(y=u * (z.abs() @ Sd.abs().t()) + (u / 2 * prod.abs() if b is not None else 0.0),
                 dx=u * (dz.abs() @ Pd.abs()), dP=u * (dz.abs().t() @ xd.abs()), dS=u * (gyd.abs().t() @ z.abs()))
    return ref, slack


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mode", ["soft", "mix", "hard", "none"])
def test_sparse_linear_fwd_bwd(cuda_device, dtype, mode):
    """SparseLinear (soft / mixed / hard effective mask, SLoRB rank 16, bias, weight scaling) forward and
    backward against the float64 products of the same rounded operands.  The mixed mask is formed as the
    reference forms it, hx * M + (1 - hx) * hard(M) with each op rounded to the mask dtype (:759-771),
    and must equal the layer's own effective mask bit for bit."""
    from sparseforge_amd import _lib as L
    from sparseforge_amd import linear as lin
    from sparseforge_amd import sparse_modeling as sm
    from oracle import masks as om

    torch.manual_seed(0)
    IN, OUT, T = 256, 192, 160
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", SLoRB=True, SLoRB_k=16,
                                SLoRB_init_type="sum", trainable_projection=True, weight_scaling=True,
                                mode="dense_forward" if mode == "none" else "sparse_forward")
    layer = sm.SparseLinear(IN, OUT, sparselinear_config=cfg, bias=True).to(dtype).to(cuda_device)
    g = torch.Generator().manual_seed(5)
    W = (torch.randn(OUT, IN, generator=g) * 0.02).to(dtype)
    b = (torch.randn(OUT, generator=g) * 0.1).to(dtype)
    M = torch.rand(OUT, IN, generator=g).to(dtype)
    with torch.no_grad():
        layer.weight.copy_(W)
        layer.bias.copy_(b)
        layer.mask.copy_(M)
        layer.init_SLoRB()
        layer.SLoRB_Weight.copy_((torch.randn(OUT, IN // 16, generator=g) * 0.01).to(dtype))
    hx = {"soft": 1.0, "mix": 0.3, "hard": 0.0, "none": 1.0}[mode]
    if mode == "hard":
        cfg.weight_scaling = False  # hx = 0 without scaling: the byte and-mask path
    layer.hardening_x = hx
    x = torch.randn(2, T // 2, IN, generator=g).to(dtype)
    gy = torch.randn(2, T // 2, OUT, generator=g).to(dtype)
    xd = x.to(cuda_device).requires_grad_(True)
    y = layer(xd)
    y.backward(gy.to(cuda_device))
    if mode == "none":
        E, s = torch.ones(OUT, IN, dtype=dtype), 1.0
    elif mode == "soft":
        E, s = M, 1.0
    else:
        hard = torch.from_numpy(om.hard_mask_from_soft(M.float().numpy(), "nm_2_4")).to(dtype)
        E = hx * M + (1 - hx) * hard
        s = 1.0 + (1.0 - hx) * (2.0 - 1.0) if cfg.weight_scaling else 1.0
        if mode == "mix":
            got_E = lin.effective_mask(layer.mask.detach(), dtype, "mix", hx, L.HARD_NM_TAIL_KEEP, 2).cpu()
            assert torch.equal(got_E, E)
    ref, slack = _dense_reference(x.reshape(T, IN), W, b, E, s, layer.x_proj.detach().cpu(),
                                  layer.SLoRB_Weight.detach().cpu(), gy.reshape(T, OUT))
    for name, got, extra in (("y", y.reshape(T, OUT), slack["y"]), ("dx", xd.grad.reshape(T, IN), slack["dx"]),
                             ("dW", layer.weight.grad, None), ("db", layer.bias.grad, None),
                             ("dP", layer.x_proj.grad, slack["dP"]), ("dS", layer.SLoRB_Weight.grad, slack["dS"])):
        err = gemm_err(got, ref[name], dtype, extra)
        assert err <= 1.0, (name, err)


def test_sparse_linear_matches_reference_golden(cuda_device):
    """FusedMaskedLinearSTE + SLoRB outputs/grads written by the reference code."""
    from sparseforge_amd import sparse_modeling as sm

    r = load_golden("linear_slorb_f32")
    import ast

    kw = ast.literal_eval(str(r["cfg"]))
    cfg = sm.SparseLinearConfig(**kw)
    layer = sm.SparseLinear(32, 20, sparselinear_config=cfg, bias=True).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(r["W"]))
        layer.bias.copy_(torch.from_numpy(r["bias"]))
        layer.mask.copy_(torch.from_numpy(r["mask"]))
        layer.x_proj.copy_(torch.from_numpy(r["P"]))
        layer.SLoRB_Weight.copy_(torch.from_numpy(r["S"]))
    for j in range(3):
        layer.hardening_x = float(r[f"hx{j}"])
        x = torch.from_numpy(r[f"x{j}"]).to(cuda_device).requires_grad_(True)
        y = layer(x)
        y.backward(torch.from_numpy(r[f"gy{j}"]).to(cuda_device))
        for name, got in (("y", y), ("dx", x.grad), ("dW", layer.weight.grad), ("db", layer.bias.grad),
                          ("dP", layer.x_proj.grad), ("dS", layer.SLoRB_Weight.grad)):
            ref = torch.from_numpy(r[f"{name}{j}"])
            assert rel_err(got, ref) < 1e-5, (j, name, rel_err(got, ref))
        layer.zero_grad(set_to_none=True)


def test_double_backward_hvp_matches_reference(cuda_device):
    """Hutchinson HVP through the custom backward equals the reference's (v X^T X, unmasked)."""
    from sparseforge_amd import sparse_modeling as sm

    r = load_golden("hutch_quadratic_f32")
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                beta=0.98)
    layer = sm.SparseLinear(48, 24, sparselinear_config=cfg, bias=False).to(cuda_device)
    with torch.no_grad():
        layer.weight.copy_(torch.from_numpy(r["W"]))
        layer.mask.copy_(torch.from_numpy(r["mask"]))
    x = torch.from_numpy(r["x"]).to(cuda_device)
    y = torch.from_numpy(r["y"]).to(cuda_device)
    H = torch.from_numpy(r["init_H"]).double()
    for j in range(3):
        v = torch.from_numpy(r[f"v{j}"]).to(cuda_device)
        loss = 0.5 * ((layer(x) - y) ** 2).sum()
        (g,) = torch.autograd.grad(loss, [layer.weight], create_graph=True)
        (hvp,) = torch.autograd.grad((g * v).sum(), [layer.weight])
        est = (hvp * v).clamp_min(0).double().cpu()
        H = 0.98 * H + 0.02 * est
        assert rel_err(H, torch.from_numpy(r[f"H{j}"])) < 1e-5
        H = torch.from_numpy(r[f"H{j}"]).double()


def test_cpu_tensor_raises():
    from sparseforge_amd import linear as lin

    with pytest.raises(RuntimeError, match="GPU only"):
        lin.mm_nt(torch.ones(8, 8), torch.ones(8, 8))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gemm_split_k_skinny(cuda_device, dtype):
    """GEMMs with few output tiles and long K split K over f32 partials; the
    reduce applies bias / accumulation, and the second K segment runs once."""
    L, lin = _lin()
    g = torch.Generator().manual_seed(23)
    d = lambda t: t.to(cuda_device)
    # SLoRB-shaped products: z = x P^T (N = 64), dP = dz^T x (M = 64, K = T)
    T, IN, R, OUT = 4096, 1024, 64, 320
    x = torch.randn(T, IN, generator=g).to(dtype)
    P = torch.randn(R, IN, generator=g).to(dtype)
    dz = torch.randn(T, R, generator=g).to(dtype)
    desc = L.GemmDesc()
    desc.dtype, desc.M, desc.N, desc.K1 = L.dtype_code(x), T, R, IN
    assert L.lib().sf_gemm_workspace_size(L.byref(desc)) > 0  # this shape splits
    assert gemm_err(lin.mm_nt(d(x), d(P)), x.double() @ P.double().t(), dtype) <= 1.0
    assert gemm_err(lin.mm_tn(d(dz), d(x)), dz.double().t() @ x.double(), dtype) <= 1.0
    # second segment + bias on the last split, then accumulate into an existing C
    W = torch.randn(OUT, IN, generator=g).to(dtype)
    S = torch.randn(OUT, R, generator=g).to(dtype)
    z = torch.randn(256, R, generator=g).to(dtype)
    xa = x[:256].contiguous()
    b = torch.randn(OUT, generator=g).to(dtype)
    ref = xa.double() @ W.double().t() + z.double() @ S.double().t() + b.double()
    got = lin.mm_nt(d(xa), d(W), A2=d(z), B2=d(S), K2=R, bias=d(b))
    assert gemm_err(got, ref, dtype, bias_slack(ref - b.double(), dtype)) <= 1.0
    base = torch.randn(256, OUT, generator=g).to(dtype)
    acc = d(base.clone())
    lin.mm_nt(d(xa), d(W), out=acc, accumulate=True)
    # C += A B^T into a bf16 C rounds the product to bf16 before the sum (as torch's C += A @ B does)
    prod = xa.double() @ W.double().t()
    assert gemm_err(acc, base.double() + prod, dtype, bias_slack(prod, dtype)) <= 1.0


def test_gemm_split_k_deterministic(cuda_device):
    L, lin = _lin()
    g = torch.Generator().manual_seed(29)
    x = torch.randn(8192, 64, generator=g).bfloat16().to(cuda_device)
    y = torch.randn(8192, 512, generator=g).bfloat16().to(cuda_device)
    r1 = lin.mm_tn(x, y)
    r2 = lin.mm_tn(x, y)
    assert torch.equal(r1, r2)


def test_mfma_probe_runs(cuda_device):
    """The sustained-rate probe bench.py reports beside the peak: runs and yields finite checksums."""
    L, _ = _lin()
    out = torch.empty(8 * 256, dtype=torch.float32, device=cuda_device)
    L.check(L.lib().sf_mfma_probe(10, 8, L.ptr(out), L.stream(cuda_device)), "sf_mfma_probe")
    torch.cuda.synchronize()
    assert torch.isfinite(out).all() and (out != 0).any()


@pytest.mark.parametrize("tag,tol", [("f32", 1e-5), ("bf16", 2e-2)])
def test_fused_masked_linear_ste_apply_decay_matches_reference(cuda_device, tag, tol):
    """The drop-in FusedMaskedLinearSTE.apply(x, W, b, mask, decay, scale) against the reference's
    own outputs with decay = 0.05 and scale = 1.7 (legacy/sparse_modeling.py:56-132): forward,
    backward and the Hessian-vector product by double backward (the SR-STE decay epilogue of the
    weight-gradient GEMM and its elementwise second derivative)."""
    from sparseforge_amd.sparse_modeling import FusedMaskedLinearSTE

    r = load_golden(f"ste_decay_{tag}")
    dt = torch.float32 if tag == "f32" else torch.bfloat16
    d = lambda k: torch.from_numpy(r[k]).to(cuda_device).to(dt)  # noqa: E731
    x = d("x").requires_grad_(True)
    W = d("W").requires_grad_(True)
    b = d("b").requires_grad_(True)
    mask = torch.from_numpy(r["mask"]).to(cuda_device)
    decay, scale = float(r["decay"]), float(r["scale"])
    y = FusedMaskedLinearSTE.apply(x, W, b, mask, decay, scale)
    y.backward(d("gy"))
    ref = lambda k: torch.from_numpy(r[k])  # noqa: E731
    sy = sw = None
    if tag == "bf16":
        # both sides round x w^T before adding the bias, and gy^T x and decay * W before adding the decay
        # term (:84-87, :123-125), each product from its own float32 sum: the rounded products may be
        # neighbours, one ulp apart
        term = decay * ref("W").double() * (ref("mask") < 0.5)
        sy = (ref("y").double() - ref("b").double()).abs() * BF16_ULP
        sw = (ref("dW").double().abs() + 2 * term.abs()) * BF16_ULP
    for name, got, extra in (("y", y, sy), ("dx", x.grad, None), ("dW", W.grad, sw), ("db", b.grad, None)):
        err = gemm_err(got, ref(name), dt, extra)
        assert err <= 1.0, (name, err)
    Wh = d("W").requires_grad_(True)
    yh = FusedMaskedLinearSTE.apply(d("x"), Wh, d("b"), mask, decay, scale)
    loss = 0.5 * ((yh.float() - d("t").float()) ** 2).sum()
    (g,) = torch.autograd.grad(loss, Wh, create_graph=True)
    (hvp,) = torch.autograd.grad((g * d("v")).sum(), Wh)
    # a chain of products whose bf16 intermediates (the residual y - t, the gradient) both sides round:
    # checked against the output scale
    assert rel_err(hvp, ref("hvp")) < (3e-5 if tag == "f32" else tol)
    if tag == "f32":
        # the decay terms themselves: below the bars above (about 1e-4 of dW's scale), so checked
        # as residuals against the closed forms; mask == 0.5 is kept (the test is mask < 0.5)
        x64 = torch.from_numpy(r["x"]).double().reshape(-1, 64)
        gy64 = torch.from_numpy(r["gy"]).double().reshape(-1, 48)
        M = torch.from_numpy(r["mask"]).double()
        v = torch.from_numpy(r["v"]).double()
        term = decay * torch.from_numpy(r["W"]).double() * (M < 0.5)
        resid = W.grad.double().cpu() - gy64.t() @ x64
        assert (resid - term).abs().max() < 1e-6 * ref("dW").abs().max()
        h_resid = hvp.double().cpu() - v @ (x64.t() @ x64)
        assert (h_resid - decay * v * (M < 0.5)).abs().max() < 2e-5 * ref("hvp").abs().max()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decay_epilogue_through_split_k(cuda_device, dtype):
    """dW = gy^T x + decay W [E < 0.5] when the weight gradient has few output tiles and a long
    token dimension (48 x 64 over 4096 tokens): the products run split K and the ordered reduce
    pass applies the decay term.  Checked against the float64 oracle; the f32 case also checks the
    term as a residual (it is about 1e-4 of dW's scale)."""
    from oracle import linear as ol
    from sparseforge_amd.sparse_modeling import FusedMaskedLinearSTE

    g = torch.Generator().manual_seed(91)
    T, IN, OUT = 4096, 64, 48
    x = torch.randn(T, IN, generator=g).to(dtype)
    W = (torch.randn(OUT, IN, generator=g) * 0.02).to(dtype)
    M = torch.rand(OUT, IN, generator=g)
    gy = torch.randn(T, OUT, generator=g).to(dtype)
    decay = 0.25
    xd, Wd = x.to(cuda_device).requires_grad_(True), W.to(cuda_device).requires_grad_(True)
    y = FusedMaskedLinearSTE.apply(xd, Wd, None, M.to(cuda_device), decay, 1.0)
    y.backward(gy.to(cuda_device))
    Mw = M.to(dtype).double().numpy()  # the reference casts the mask to the weight dtype
    ref = ol.backward(x.double().numpy(), W.double().numpy(), Mw, gy.double().numpy(), False, decay=decay,
                      dtype=np.float64)
    assert gemm_err(Wd.grad, torch.from_numpy(ref["dW"]), dtype) <= 1.0
    # dx reads w = W * E rounded to the weight dtype, as the reference forms it (:112-113)
    assert gemm_err(xd.grad, gy.double() @ (W * M.to(dtype)).double(), dtype) <= 1.0
    if dtype == torch.float32:
        st = torch.from_numpy(gy.double().numpy().T @ x.double().numpy())
        term = decay * W.double() * torch.from_numpy(Mw < 0.5)
        assert ((Wd.grad.double().cpu() - st) - term).abs().max() < 1e-6 * st.abs().max()
        assert term.abs().max() > 1e-3
