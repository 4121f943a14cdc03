"""GPU parity of the fused mask-aware AdamW (sf_adamw_step) against the oracle
and the reference's golden outputs (legacy/adamw.py:65-176).

Bar: the f32 path is bit-exact against the oracle (same per-op roundings,
IEEE sqrt and division); against the reference's CPU outputs within 1e-6.
"""
import ast

import numpy as np
import pytest
import torch

from conftest import load_golden

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("name", ["adamw_plain", "adamw_decay_l1", "adamw_amsgrad"])
def test_dropin_adamw_matches_golden_and_oracle(cuda_device, name):
    from oracle import adamw as oa
    from sparseforge_amd.adamw import AdamW

    r = load_golden(name)
    h = ast.literal_eval(str(r["cfg"]))
    w = torch.nn.Parameter(torch.from_numpy(r["init_w"]).to(cuda_device))
    w.mask = torch.from_numpy(r["mask"]).to(cuda_device)
    b = torch.nn.Parameter(torch.from_numpy(r["init_b"]).to(cuda_device))
    opt = AdamW([w, b], **h)
    n = sum(1 for k in r if k.startswith("decay"))
    ow, ob = r["init_w"], r["init_b"]
    sw = [np.zeros_like(ow) for _ in range(3)]
    sb = [np.zeros_like(ob) for _ in range(3)]
    decays = {"adamw_decay_l1": (None, 3e-4, 5e-4, 0.0), "adamw_amsgrad": (1e-3, 1e-3, 1e-3)}.get(name, (None,) * n)
    for j in range(n):
        w.grad = torch.from_numpy(r[f"gw{j}"]).to(cuda_device)
        b.grad = torch.from_numpy(r[f"gb{j}"]).to(cuda_device)
        opt.step(decay=decays[j])
        assert opt.decay == float(r[f"decay{j}"])
        kw = dict(lr=h["lr"], betas=h["betas"], eps=h["eps"], weight_decay=h["weight_decay"], decay=opt.decay,
                  l1=h["adaptive_l1_decay"], amsgrad=h["amsgrad"])
        ow, sw[0], sw[1], sw[2] = oa.step(ow, r[f"gw{j}"], sw[0], sw[1], sw[2], r["mask"], j + 1, **kw)
        ob, sb[0], sb[1], sb[2] = oa.step(ob, r[f"gb{j}"], sb[0], sb[1], sb[2], None, j + 1, **kw)
        st = opt.state[w]
        got = {"w": w.detach().cpu().numpy(), "b": b.detach().cpu().numpy(), "m": st["exp_avg"].cpu().numpy(),
               "v": st["exp_avg_sq"].cpu().numpy()}
        assert np.array_equal(got["w"], ow) and np.array_equal(got["b"], ob)
        assert np.array_equal(got["m"], sw[0]) and np.array_equal(got["v"], sw[1])
        for key in ("w", "b", "m", "v"):
            np.testing.assert_allclose(got[key], r[f"{key}{j}"], rtol=0, atol=1e-6)
        assert st["step"] == j + 1


@pytest.mark.parametrize("n", [1, 7, 4096 * 3 + 5, 1_000_003])
def test_fused_step_bit_exact_vs_oracle(cuda_device, n):
    from oracle import adamw as oa
    from sparseforge_amd.adamw import adamw_step_

    rng = np.random.default_rng(n)
    p = (rng.standard_normal(n) * 0.05).astype(np.float32)
    m = (rng.standard_normal(n) * 1e-3).astype(np.float32)
    v = (rng.random(n) * 1e-5).astype(np.float32)
    x = v + (rng.random(n) * 1e-6).astype(np.float32)
    g = (rng.standard_normal(n) * 1e-2).astype(np.float32)
    mask = rng.random(n).astype(np.float32)
    d = lambda a: torch.from_numpy(a.copy()).to(cuda_device)
    tp, tm, tv, tx = d(p), d(m), d(v), d(x)
    adamw_step_(tp, d(g), tm, tv, tx, d(mask), 7, 1e-3, (0.9, 0.95), 1e-8, 0.1, decay=2e-4, l1=1e-3, amsgrad=True,
                apply_l1=True)
    rp, rm, rv, rx = oa.step(p.reshape(1, -1), g, m, v, x, mask, 7, 1e-3, (0.9, 0.95), 1e-8, 0.1, decay=2e-4, l1=1e-3,
                             amsgrad=True)
    assert np.array_equal(tp.cpu().numpy(), rp.reshape(-1))
    assert np.array_equal(tm.cpu().numpy(), rm.reshape(-1)) and np.array_equal(tv.cpu().numpy(), rv.reshape(-1))
    assert np.array_equal(tx.cpu().numpy(), rx.reshape(-1))


def test_master_weights_with_bf16_copy_and_bf16_grad(cuda_device):
    """f32 master + bf16 gradient + bf16 working copy (the 7B arena layout)."""
    from oracle import adamw as oa
    from oracle.numerics import round_bf16
    from sparseforge_amd.adamw import adamw_step_

    rng = np.random.default_rng(3)
    n = 65536 + 3
    p = (rng.standard_normal(n) * 0.05).astype(np.float32)
    g = round_bf16((rng.standard_normal(n) * 1e-3).astype(np.float32))
    mask = rng.random(n).astype(np.float32)
    tp = torch.from_numpy(p.copy()).to(cuda_device)
    tg = torch.from_numpy(g).to(cuda_device).bfloat16()
    tm, tv = torch.zeros(n, device=cuda_device), torch.zeros(n, device=cuda_device)
    w16 = torch.empty(n, dtype=torch.bfloat16, device=cuda_device)
    adamw_step_(tp, tg, tm, tv, None, torch.from_numpy(mask).to(cuda_device), 1, 1e-3, (0.9, 0.999), 1e-8, 0.0,
                decay=1e-3, bf16_copy=w16)
    rp, rm, rv, _ = oa.step(p, g, np.zeros(n, np.float32), np.zeros(n, np.float32), None, mask, 1, 1e-3, (0.9, 0.999),
                            1e-8, 0.0, decay=1e-3)
    assert np.array_equal(tp.cpu().numpy(), rp) and np.array_equal(tm.cpu().numpy(), rm)
    assert torch.equal(w16.cpu(), torch.from_numpy(rp).bfloat16())


def test_adamw_rejects_bad_hyperparameters():
    from sparseforge_amd.adamw import AdamW

    p = [torch.nn.Parameter(torch.zeros(2))]
    with pytest.raises(ValueError, match="learning rate"):
        AdamW(p, lr=-1)
    with pytest.raises(ValueError, match="beta parameter at index 1"):
        AdamW(p, betas=(0.9, 1.0))


@pytest.mark.parametrize("amsgrad,l1,sdt", [(False, 0.0, torch.float32), (True, 2e-3, torch.float32),
                                           (False, 1e-3, torch.bfloat16)])
def test_multi_tensor_step_equals_per_tensor_step(cuda_device, amsgrad, l1, sdt):
    """sf_adamw_step_multi over 97 tensors (three launches of at most 40) equals sf_adamw_step per
    tensor bit for bit: ragged sizes, an empty tensor, unaligned views (vector accesses off), f32 and
    bf16 gradients and masks, tensors without a mask, 1-D tensors (no L1 term), bf16 copies."""
    from sparseforge_amd.adamw import TensorStep, adamw_step_, adamw_step_multi_

    g = torch.Generator(device=cuda_device).manual_seed(41)
    dev = cuda_device
    sizes = [0, 1, 3, 4, 5, 1023, 1024, 1025, 4099, 65537, 300_001] + [int(x) for x in
                                                                       torch.randint(1, 20000, (86,), generator=g,
                                                                                     device=dev).cpu()]

    def make(k, n):
        off = 1 if k % 5 == 3 else 0  # an unaligned view: element offset 1
        mk = lambda dt, s=1.0: (torch.randn(n + off, generator=g, device=dev) * s).to(dt)[off:]  # noqa: E731
        p = mk(torch.float32, 0.05)
        gr = mk(torch.bfloat16 if k % 2 else torch.float32, 1e-3)
        m = mk(sdt, 1e-3)
        v = mk(sdt, 1e-3).abs()
        vmax = (v.float() * 1.5).to(sdt) if amsgrad else None
        mask = None if k % 7 == 0 else mk(torch.bfloat16 if k % 3 else torch.float32).sigmoid()
        copy = torch.empty(n, dtype=torch.bfloat16, device=dev) if k % 4 == 1 else None
        return dict(p=p, g=gr, m=m, v=v, vmax=vmax, mask=mask, copy=copy, l1=(k % 6 != 5))

    tensors = [make(k, n) for k, n in enumerate(sizes)]
    clones = [{k: (x.clone() if isinstance(x, torch.Tensor) else x) for k, x in t.items()} for t in tensors]
    hp = dict(lr=1e-3, betas=(0.9, 0.95), eps=1e-8, weight_decay=0.1, decay=6e-5, l1=l1, amsgrad=amsgrad)
    for t in clones:
        if t["p"].numel():
            adamw_step_(t["p"], t["g"], t["m"], t["v"], t["vmax"], t["mask"], 3, hp["lr"], hp["betas"], hp["eps"],
                        hp["weight_decay"], decay=hp["decay"] if t["mask"] is not None else 0.0, l1=l1,
                        amsgrad=amsgrad, apply_l1=t["l1"], bf16_copy=t["copy"])
    items = [TensorStep(t["p"], t["g"], t["m"], t["v"], t["vmax"], t["mask"], t["copy"], apply_l1=t["l1"])
             for t in tensors]
    adamw_step_multi_(items, 3, **hp)
    torch.cuda.synchronize()
    for k, (a, b) in enumerate(zip(tensors, clones)):
        for key in ("p", "m", "v", "vmax", "copy"):
            if a[key] is not None:
                assert torch.equal(a[key], b[key]), (k, key, sizes[k])
