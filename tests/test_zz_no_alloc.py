"""sf_tau_quantile_noalloc (the entry point that allocates nothing) against sf_tau_quantile.

Both are called through the C ABI on the same device inputs; the threshold must
be bit-identical.  Two calls in a row, the second on a smaller layer with a
smaller sample, show that the shared static scratch carries nothing over.  The
maximum sample is accepted and one element more is rejected on the host
before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _lib():
    from sparseforge_amd import _lib as L

    L.load()
    return L


def _params(L, rows, cols):
    p = L.MaskParams()
    p.rows, p.cols = rows, cols
    p.metric = L.METRIC["hessian_ratio"]
    p.gate = L.GATE_UNSTRUCTURED
    p.n_keep, p.m_group = 2, 4
    p.hard_kind, p.hard_n, p.hard_m = L.HARD_NM_TAIL_KEEP, 2, 4
    p.score_dtype = L.DT_F32
    p.temperature = 0.5
    p.eps_metric = 1e-8
    p.movement_temp = 1.0
    p.mask_lr = 0.1
    return p


def _case(L, dev, rows, cols, sample, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    W = (torch.randn(rows, cols, generator=g, device=dev) * 0.02).to(torch.bfloat16)
    H = torch.rand(rows, cols, generator=g, device=dev) * 1e-3 + 1e-6
    idx = torch.randint(0, rows * cols, (sample,), generator=g, device=dev, dtype=torch.int64)
    p = _params(L, rows, cols)
    ws = torch.empty(L.lib().sf_mask_workspace_size(rows, cols, sample), dtype=torch.uint8, device=dev)
    stats = torch.empty(2, dtype=torch.float32, device=dev)
    st = L.stream(dev)
    L.check(L.lib().sf_score_stats(ctypes.byref(p), W.data_ptr(), L.DT_BF16, H.data_ptr(), L.DT_F32, None, L.DT_F32,
                                   stats.data_ptr(), ws.data_ptr(), ws.numel(), st), "sf_score_stats")
    return p, W, H, idx, ws, stats


def _tau_pair(L, dev, p, W, H, idx, ws, stats, q):
    st = L.stream(dev)
    ref = torch.full((1,), float("nan"), dtype=torch.float32, device=dev)
    got = torch.full((1,), float("nan"), dtype=torch.float32, device=dev)
    m = idx.numel()
    L.check(L.lib().sf_tau_quantile(ctypes.byref(p), W.data_ptr(), L.DT_BF16, H.data_ptr(), L.DT_F32, None, L.DT_F32,
                                    stats.data_ptr(), idx.data_ptr(), m, q, ref.data_ptr(), ws.data_ptr(), ws.numel(),
                                    st), "sf_tau_quantile")
    L.check(L.lib().sf_tau_quantile_noalloc(ctypes.byref(p), W.data_ptr(), L.DT_BF16, H.data_ptr(), L.DT_F32, None,
                                            L.DT_F32, stats.data_ptr(), idx.data_ptr(), m, q, got.data_ptr(), st),
            "sf_tau_quantile_noalloc")
    torch.cuda.synchronize(dev)
    return ref.item(), got.item()


def test_noalloc_tau_equals_workspace_tau_on_two_calls(cuda_device):
    L = _lib()
    dev = cuda_device
    # first call: a 4096 x 4096 layer, the 262 144-element sample of the paper config
    big = _case(L, dev, 4096, 4096, 262144, 5)
    # second call: a smaller layer and sample (the scratch keeps the first call's keys beyond it)
    small = _case(L, dev, 300, 200, 20000, 6)
    for case in (big, small):
        for q in (0.5, 0.37):
            ref, got = _tau_pair(L, dev, *case, q)
            assert np.float32(ref).tobytes() == np.float32(got).tobytes(), (ref, got)
            assert np.isfinite(got)


def test_noalloc_tau_sample_limit(cuda_device):
    L = _lib()
    dev = cuda_device
    rows, cols = 1024, 2048  # numel 2 Mi > the maximum sample
    p, W, H, _idx, ws, stats = _case(L, dev, rows, cols, 16, 7)
    g = torch.Generator(device=dev).manual_seed(8)
    idx_max = torch.randint(0, rows * cols, (L.TAU_NOALLOC_MAX_SAMPLE,), generator=g, device=dev, dtype=torch.int64)
    ws_max = torch.empty(L.lib().sf_mask_workspace_size(rows, cols, idx_max.numel()), dtype=torch.uint8, device=dev)
    ref, got = _tau_pair(L, dev, p, W, H, idx_max, ws_max, stats, 0.5)
    assert np.float32(ref).tobytes() == np.float32(got).tobytes()
    tau = torch.empty(1, dtype=torch.float32, device=dev)
    rc = L.lib().sf_tau_quantile_noalloc(ctypes.byref(p), W.data_ptr(), L.DT_BF16, H.data_ptr(), L.DT_F32, None,
                                         L.DT_F32, stats.data_ptr(), idx_max.data_ptr(),
                                         L.TAU_NOALLOC_MAX_SAMPLE + 1, 0.5, tau.data_ptr(), L.stream(dev))
    assert rc == L.SF_ERR_INVALID
    assert "exceeds the static scratch maximum" in L.last_error()
