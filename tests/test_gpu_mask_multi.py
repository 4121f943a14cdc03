"""The batched mask update (sf_update_mask_multi) against the single-layer entry points.

calculate_model_mask (legacy/utils.py:184-310) updates every SparseLinear
with update_mask (legacy/sparse_modeling.py:1242-1666); the batched call runs
score statistics, tau selection and the fused update of up to 28 layers per
launch.  Bar: bit-exact equality with sf_score_stats + sf_tau_quantile +
sf_update_mask layer by layer (which the reference goldens and the oracle pin
elsewhere) -- stats, tau, masks, frozen flags and flip counts -- across batch
boundaries (33 layers), ragged and empty layers, sampled and full tau samples,
f32 and bf16 masks, structured gates, frozen flags and freezing; the stages
run one call at a time equal the stages run together; and calculate_model_mask
on a model equals update_mask layer by layer.
"""
import pytest
import torch

pytestmark = pytest.mark.gpu

SHAPES = [(64, 256), (96, 1023), (33, 66), (128, 4096), (17, 7), (0, 8), (256, 512), (40, 4), (1, 1021)]


def _lib():
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K

    return L, K


def _params(L, case):
    p = L.MaskParams()
    p.n_keep, p.m_group = 2, 4
    p.hard_kind, p.hard_n, p.hard_m = L.HARD_NM_TAIL_KEEP, 2, 4
    p.eps_metric, p.movement_temp, p.mask_lr = 1e-8, 1.0, 0.1
    p.temperature = 0.3
    if case == "unstructured":
        p.metric, p.gate, p.score_dtype = L.METRIC["hessian_ratio"], L.GATE_UNSTRUCTURED, L.DT_F32
        p.penalty, p.penalty_coef = L.PENALTY_NM_2_4, 0.01
    elif case == "structured_bf16":
        p.metric, p.gate, p.score_dtype = L.METRIC["hessian_obd"], L.GATE_STRUCTURED, L.DT_BF16
        p.beta_struct = 0.3
        p.penalty, p.penalty_coef = L.PENALTY_MID, 0.02
        p.binarize = 0.05
    else:  # frozen: magnitude scores, frozen flags, freezing snaps, threshold flips
        p.metric, p.gate, p.score_dtype = L.METRIC["magnitude"], L.GATE_UNSTRUCTURED, L.DT_F32
        p.hard_kind = L.HARD_THRESHOLD
        p.has_frozen = 1
        p.apply_freeze, p.freeze_low, p.freeze_high, p.snap_high = 1, 0.05, 0.95, 1
    return p


def _layers(case, dev, n=33, seed=0):
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for i in range(n):
        rows, cols = SHAPES[i % len(SHAPES)]
        if case == "structured_bf16" and cols % 4:
            cols += 4 - cols % 4  # the structured gate needs whole groups
        wdt = torch.float32 if case == "frozen" else torch.bfloat16
        mdt = torch.bfloat16 if case == "structured_bf16" else torch.float32
        W = (torch.randn(rows, cols, generator=g, device=dev) * 0.02).to(wdt)
        H = None
        if case != "frozen":
            H = (torch.rand(rows, cols, generator=g, device=dev) * 1e-3 + 1e-6)
            H = H.to(torch.bfloat16 if case == "structured_bf16" else torch.float32)
        M = torch.rand(rows, cols, generator=g, device=dev).to(mdt)
        F = None
        if case == "frozen":
            F = (torch.rand(rows, cols, generator=g, device=dev) < 0.1).float()
        idx = None
        if rows * cols > 600 and i % 2 == 0:
            idx = torch.randint(0, rows * cols, (4099,), generator=g, device=dev)
        out.append((W, H, M, F, idx))
    return out


def _clone(layers):
    return [tuple(t.clone() if t is not None else None for t in l) for l in layers]


def _single(L, K, p0, q, layers):
    """sf_score_stats + sf_tau_quantile + sf_update_mask layer by layer."""
    stats, taus, flips = [], [], []
    for W, H, M, F, idx in layers:
        rows, cols = W.shape
        if rows * cols == 0:
            stats.append(None), taus.append(None), flips.append(None)
            continue
        p = L.MaskParams.from_buffer_copy(p0)
        p.rows, p.cols = rows, cols
        ops = K.MaskOperands(weight=W, mask=M, hessian=H, frozen=F)
        st = K.score_stats(p, ops)
        tau = K.tau_quantile(p, ops, st, q, idx) if p.gate == L.GATE_UNSTRUCTURED else None
        fl = torch.zeros(1, dtype=torch.int64, device=W.device)
        K.update_mask(p, ops, st, tau, fl)
        stats.append(st), taus.append(tau), flips.append(fl)
    return stats, taus, flips


def _multi(L, K, p0, q, layers, stage_list=None):
    dev = layers[0][0].device
    n = len(layers)
    stats = torch.full((n, 2), float("nan"), device=dev)
    tau = torch.full((n,), float("nan"), device=dev)
    flips = torch.zeros(n, dtype=torch.int64, device=dev)
    jobs = [K.MaskJob(K.MaskOperands(weight=W, mask=M, hessian=H, frozen=F), idx, stats[i], tau[i:i + 1],
                      flips[i:i + 1]) for i, (W, H, M, F, idx) in enumerate(layers)]
    for stg in stage_list or [L.MULTI_ALL]:
        K.update_mask_multi(p0, q, jobs, stg)
    return stats, tau, flips


@pytest.mark.parametrize("case", ["unstructured", "structured_bf16", "frozen"])
def test_multi_equals_single_layer_calls(cuda_device, case):
    L, K = _lib()
    p0 = _params(L, case)
    layers = _layers(case, cuda_device)
    a, b = _clone(layers), _clone(layers)
    s_stats, s_tau, s_flips = _single(L, K, p0, 0.37, a)
    m_stats, m_tau, m_flips = _multi(L, K, p0, 0.37, b)
    torch.cuda.synchronize()
    unstructured = p0.gate == L.GATE_UNSTRUCTURED
    for i, ((W, H, M, F, idx), (_, _, M2, F2, _)) in enumerate(zip(a, b)):
        if W.numel() == 0:
            assert torch.isnan(m_stats[i]).all() and m_flips[i] == 0, i  # empty layers are skipped
            continue
        assert torch.equal(m_stats[i], s_stats[i]), (case, i, m_stats[i], s_stats[i])
        if unstructured:
            assert torch.equal(m_tau[i:i + 1], s_tau[i]), (case, i)
        assert torch.equal(M2, M), (case, i, W.shape)
        if F is not None:
            assert torch.equal(F2, F), (case, i)
        assert int(m_flips[i]) == int(s_flips[i]), (case, i)
    assert int(m_flips.sum()) > 0


def test_multi_stages_one_call_at_a_time(cuda_device):
    L, K = _lib()
    p0 = _params(L, "unstructured")
    layers = _layers("unstructured", cuda_device, n=12, seed=3)
    a, b = _clone(layers), _clone(layers)
    s1 = _multi(L, K, p0, 0.5, a)
    s2 = _multi(L, K, p0, 0.5, b, [L.MULTI_STATS, L.MULTI_TAU, L.MULTI_UPDATE])
    torch.cuda.synchronize()
    for x, y in zip(s1, s2):
        assert torch.equal(torch.nan_to_num(x, 7.0), torch.nan_to_num(y, 7.0))
    for la, lb in zip(a, b):
        assert torch.equal(la[2], lb[2])


def test_multi_pipelined_schedule_equals_serial(cuda_device):
    """Four batches (100 layers, sampled and full tau samples): with the full workspace the batches' tau
    selections run on the side stream beside the next batch's statistics, and batch b + 2 reuses batch b's
    regions; with the serial minimum the stages run batch after batch.  Both equal the single-layer calls,
    over two updates in a row (the second starts from the first's masks)."""
    L, K = _lib()
    p0 = _params(L, "unstructured")
    layers = _layers("unstructured", cuda_device, n=100, seed=11)
    a, b, c = _clone(layers), _clone(layers), _clone(layers)
    n = len(layers)
    jobs_of = lambda ls, st, ta, fl: [K.MaskJob(K.MaskOperands(weight=W, mask=M, hessian=H, frozen=F), idx, st[i],
                                                ta[i:i + 1], fl[i:i + 1]) for i, (W, H, M, F, idx) in enumerate(ls)]
    outs = []
    for ls, small in ((b, False), (c, True)):
        st = torch.full((n, 2), float("nan"), device=cuda_device)
        ta = torch.full((n,), float("nan"), device=cuda_device)
        fl = torch.zeros(n, dtype=torch.int64, device=cuda_device)
        jobs = jobs_of(ls, st, ta, fl)
        table = K._layer_table(jobs)
        full = L.lib().sf_update_mask_multi_workspace_size(table, n)
        ws = K.multi_workspace(jobs, cuda_device)
        assert ws.numel() == full
        if small:  # the serial layout's size: below what the pipelined schedule needs
            ws = ws[:full - 4096 * 4]
        for step in range(2):
            p = L.MaskParams.from_buffer_copy(p0)
            p.temperature = 0.3 if step == 0 else 0.05
            K.update_mask_multi(p, 0.37, jobs, L.MULTI_ALL, ws)
        outs.append((st, ta, fl))
    want = []
    for step in range(2):
        p = L.MaskParams.from_buffer_copy(p0)
        p.temperature = 0.3 if step == 0 else 0.05
        want.append(_single(L, K, p, 0.37, a))
    torch.cuda.synchronize()
    s_stats, s_tau, _ = want[1]
    for st, ta, fl in outs:
        for i, ((W, _, M, _, _), (_, _, M2, _, _), (_, _, M3, _, _)) in enumerate(zip(a, b, c)):
            if W.numel() == 0:
                continue
            assert torch.equal(st[i], s_stats[i]), i
            assert torch.equal(ta[i:i + 1], s_tau[i]), i
            total_flips = int(want[0][2][i]) + int(want[1][2][i])
            assert int(fl[i]) == total_flips, i
    for (W, _, M, _, _), (_, _, M2, _, _), (_, _, M3, _, _) in zip(a, b, c):
        assert torch.equal(M2, M) and torch.equal(M3, M)


def test_multi_rejects_bad_calls(cuda_device):
    L, K = _lib()
    p0 = _params(L, "unstructured")
    (W, H, M, F, idx), = _layers("unstructured", cuda_device, n=1)
    job = K.MaskJob(K.MaskOperands(weight=W, mask=M, hessian=H), idx, torch.empty(2, device=cuda_device),
                    None, None)
    with pytest.raises(ValueError, match="tau"):
        K.update_mask_multi(p0, 0.5, [job])  # the unstructured gate writes tau
    job.tau = torch.empty(1, device=cuda_device)
    with pytest.raises(ValueError, match="stage"):
        K.update_mask_multi(p0, 0.5, [job], 8)
    other = K.MaskJob(K.MaskOperands(weight=W.float(), mask=M, hessian=H), idx, torch.empty(2, device=cuda_device),
                      torch.empty(1, device=cuda_device), None)
    with pytest.raises(ValueError, match="dtypes differ"):
        K.update_mask_multi(p0, 0.5, [job, other])


def _model(dev, seed):
    from sparseforge_amd import sparse_modeling as sm

    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                sparsity_warmup_steps=0, mask_update_period=1, mask_penalty_mode="nm_2_4",
                                mask_penalty_lr=0.1, mask_lr=0.1, temp_init=0.5, tau_sample_size=5000)
    cfg.enable_hutchinson = True
    g = torch.Generator(device=dev).manual_seed(seed)
    shapes = [(256, 128), (128, 256), (384, 128), (128, 384), (130, 96), (64, 64)] * 6  # 36 layers: two batches
    mods = torch.nn.Sequential(*[sm.SparseLinear(i, o, sparselinear_config=cfg, bias=False, device=dev)
                                 for i, o in shapes])
    with torch.no_grad():
        for m in mods:
            m.weight.copy_(torch.randn(m.weight.shape, generator=g, device=dev) * 0.02)
            m.hessian_diag.copy_(torch.rand(m.weight.shape, generator=g, device=dev) * 1e-3 + 1e-6)
            m.mask.copy_(torch.rand(m.weight.shape, generator=g, device=dev))
    return mods


def test_calculate_model_mask_batches_like_update_mask(cuda_device):
    from sparseforge_amd import utils as U

    a, b = _model(cuda_device, 1), _model(cuda_device, 1)
    torch.manual_seed(123)
    U.calculate_model_mask(a, step=5, lambda_mid=0.05)
    torch.manual_seed(123)
    for m in b:
        m.update_mask(5, lambda_mid=0.05)
    torch.cuda.synchronize()
    for ma, mb in zip(a, b):
        assert torch.equal(ma.mask, mb.mask), ma.weight.shape
        assert int(ma.weight.flipped_mask) == int(mb.weight.flipped_mask)
        assert ma.hardening_x == mb.hardening_x
    assert sum(int(m.weight.flipped_mask) for m in a) > 0


def test_calculate_model_mask_mixed_paths_draw_in_module_order(cuda_device):
    """Layers on the staged path (block16 hard type) interleaved with layers on the batched path (nm_2_4),
    all with sampled unstructured tau: calculate_model_mask draws every layer's tau sample in module
    order, so its masks equal one update_mask per layer after the same seed, bit for bit."""
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd import utils as U

    def model():
        g = torch.Generator(device=cuda_device).manual_seed(4)
        mods = []
        for k, (i, o) in enumerate([(256, 128), (128, 256), (384, 128), (128, 384), (256, 256), (64, 64)] * 2):
            cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="block16" if k % 2 else "nm_2_4",
                                        mask_metric="hessian_ratio", sparsity_warmup_steps=0, mask_update_period=1,
                                        mask_lr=0.1, temp_init=0.5, tau_sample_size=3000)
            cfg.enable_hutchinson = True
            m = sm.SparseLinear(i, o, sparselinear_config=cfg, bias=False, device=cuda_device)
            with torch.no_grad():
                m.weight.copy_(torch.randn(m.weight.shape, generator=g, device=cuda_device) * 0.02)
                m.hessian_diag.copy_(torch.rand(m.weight.shape, generator=g, device=cuda_device) * 1e-3 + 1e-6)
                m.mask.copy_(torch.rand(m.weight.shape, generator=g, device=cuda_device))
            mods.append(m)
        return torch.nn.Sequential(*mods)

    a, b = model(), model()
    torch.manual_seed(321)
    U.calculate_model_mask(a, step=5)
    torch.manual_seed(321)
    for m in b:
        m.update_mask(5)
    torch.cuda.synchronize()
    for k, (ma, mb) in enumerate(zip(a, b)):
        assert torch.equal(ma.mask, mb.mask), (k, ma.weight.shape)
        assert int(ma.weight.flipped_mask) == int(mb.weight.flipped_mask), k


# shapes whose groups are all vector-loadable, so the batched update reads the tau sample's keys from its
# statistics pass: windows of 1024 elements, partial last windows, one-window and sub-window layers
VEC_SHAPES = [(64, 256), (96, 1020), (33, 68), (128, 4096), (40, 4), (256, 512), (1, 1024), (3, 8), (130, 96)]


def _vec_layers(K, dev, n, seed, sampling):
    """sampling(i, numel, g) -> the layer's sample indices (or None for every element)."""
    g = torch.Generator(device=dev).manual_seed(seed)
    out = []
    for i in range(n):
        rows, cols = VEC_SHAPES[i % len(VEC_SHAPES)]
        W = (torch.randn(rows, cols, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        H = torch.rand(rows, cols, generator=g, device=dev) * 1e-3 + 1e-6
        M = torch.rand(rows, cols, generator=g, device=dev)
        out.append((W, H, M, None, sampling(i, rows * cols, g)))
    return out


def _sorted_sampling(K, dev):
    def f(i, numel, g):
        kind = i % 5
        if kind == 0:
            return None  # every element
        if kind == 1:  # the library's sorted sampler
            return K.sample_indices_sorted(4099, [numel], [77 + i], dev)[0]
        if kind == 2:  # sorted torch.randint draws (duplicates), with out-of-range ends that clamp
            v = torch.sort(torch.randint(0, numel, (3001,), generator=g, device=dev)).values
            return torch.cat([torch.tensor([-3], device=dev), v, torch.tensor([numel + 5], device=dev)])
        if kind == 3:  # unsorted: gathered by the statistics workgroups
            return torch.randint(0, numel, (2048,), generator=g, device=dev)
        # sorted, denser than one sample per element (many samples per window)
        return K.sample_indices_sorted(3 * numel, [numel], [5 + i], dev)[0]
    return f


@pytest.mark.parametrize("n_layers", [9, 61])
def test_multi_fold_equals_single_layer_calls(cuda_device, n_layers):
    """Every layer vector-loadable: the statistics pass writes the keys of sorted samples from its own
    windows, unsorted samples are gathered by the same workgroups, full samples are written in element
    order.  Stats, tau, masks and flip counts equal the single-layer calls (whose tau gathers every sample
    at random) bit for bit; 61 layers run three batches on the pipelined schedule."""
    L, K = _lib()
    p0 = _params(L, "unstructured")
    layers = _vec_layers(K, cuda_device, n_layers, 21, _sorted_sampling(K, cuda_device))
    a, b = _clone(layers), _clone(layers)
    for q in (0.37, 0.81):
        s_stats, s_tau, s_flips = _single(L, K, p0, q, a)
        m_stats, m_tau, m_flips = _multi(L, K, p0, q, b)
        torch.cuda.synchronize()
        for i, ((W, _, M, _, idx), (_, _, M2, _, _)) in enumerate(zip(a, b)):
            assert torch.equal(m_stats[i], s_stats[i]), (q, i, W.shape)
            assert torch.equal(m_tau[i:i + 1], s_tau[i]), (q, i, W.shape, None if idx is None else idx.numel())
            assert torch.equal(M2, M), (q, i, W.shape)
            assert int(m_flips[i]) == int(s_flips[i]), (q, i)


def test_multi_fold_nan_scores(cuda_device):
    """A NaN weight makes its score NaN: the folded keys carry it, and tau is NaN as with the gather."""
    L, K = _lib()
    p0 = _params(L, "unstructured")
    layers = _vec_layers(K, cuda_device, 4, 5, lambda i, numel, g: K.sample_indices_sorted(
        max(numel // 2, 1), [numel], [i], cuda_device)[0])
    W = layers[0][0]
    W.view(-1)[layers[0][4][7]] = float("nan")
    a, b = _clone(layers), _clone(layers)
    _s, s_tau, _f = _single(L, K, p0, 0.5, a)
    _s2, m_tau, _f2 = _multi(L, K, p0, 0.5, b)
    torch.cuda.synchronize()
    assert torch.isnan(m_tau[0]) and torch.isnan(s_tau[0])
    for i in range(1, 4):
        assert torch.equal(m_tau[i:i + 1], s_tau[i]), i


def test_calculate_model_mask_large_sample_fallback(cuda_device, monkeypatch):
    """Samples at or above the sorted sampler's bound come from a seeded torch.randint (unsorted); the
    batched update gathers them, and calculate_model_mask still equals update_mask layer by layer.  The
    bound is lowered below the models' 5000-element sample to take that path on small layers."""
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd import utils as U

    monkeypatch.setattr(sm, "SORTED_SAMPLE_MAX", 1000)
    rows = sm.draw_samples(5000, [7000, 9000], [3, 4], cuda_device)
    assert rows.shape == (2, 5000) and int(rows[0].max()) < 7000 and int(rows[1].max()) < 9000
    assert not bool((rows[0][1:] >= rows[0][:-1]).all())  # unsorted: the gather path
    assert torch.equal(rows, sm.draw_samples(5000, [7000, 9000], [3, 4], cuda_device))  # seeded
    a, b = _model(cuda_device, 2), _model(cuda_device, 2)
    torch.manual_seed(99)
    U.calculate_model_mask(a, step=5, lambda_mid=0.05)
    torch.manual_seed(99)
    for m in b:
        m.update_mask(5, lambda_mid=0.05)
    torch.cuda.synchronize()
    for ma, mb in zip(a, b):
        assert torch.equal(ma.mask, mb.mask), ma.weight.shape
        assert int(ma.weight.flipped_mask) == int(mb.weight.flipped_mask)
