#!/usr/bin/env python3
"""Benchmark of the SparseForge sparse-training hot path on one MI355X.

Metric (the reference's headline benchmark): SparseLinear fwd+bwd TFLOP/s at LLaMA-2-7B shapes;
2:4 mask-update HBM GB/s.

* ``value`` -- one step = forward + backward of the seven SparseLinear layers
  of a LLaMA-2-7B decoder layer (q/k/v/o [4096, 4096], gate/up
  [11008, 4096], down [4096, 11008]) over T = 8192 tokens in bf16, with the
  hard 2:4 mask of the layer's soft mask (hardening_x = 0) and the SLoRB
  bypass at rank 64.  The forward writes W * E and its packed 2:4 form with
  one elementwise pass, keeps W * E for the input gradient and runs its
  product on the 2:4 sparse MFMA (``sparse_forward``); the gradient products
  and the SLoRB products run on sf_gemm (``roofline``: its own FLOPs over its
  own device time).  Throughput counts the algorithmic (dense) 6 T in out +
  6 T r (in + out) FLOPs per linear; ``per_linear`` times each linear alone.
* ``gemm_vs_hipblaslt`` -- the three big products (fwd, dx, dW) of each 7B
  linear shape through sf_gemm and through torch.matmul (hipBLASLt), and the
  layer's 21 products summed.
* ``hutchinson_probe_layer`` -- one Hutchinson probe of the same seven linears
  (create_graph gradients, probe dot, double backward, accumulator updates).
* ``mask_update`` -- one step = the periodic mask update of every linear of
  the 7B model (32 layers x 7 linears, 6.48 G params; bf16 W, fp32
  Hutchinson accumulator and soft mask): score statistics, tau quantile over
  a 262 144-element sample, then the fused gate + EMA + flip-count pass, at a
  temperature taken from a 1.0 -> 0.01 geometric schedule over 10 steps;
  the 224 layers share their parameters, so the update is batched as
  calculate_model_mask batches it (sf_update_mask_multi, 28 layers per
  launch).  GB/s counts 20 B per parameter (stats pass: W 2 + H 4; update pass: W 2 +
  H 4 + mask read 4 + mask write 4).  ``hbm_sustained`` is what a stream of
  the same traffic with token arithmetic sustains (sf_hbm_probe).
* ``hutchinson`` -- the accumulator update of every linear of the 7B arena
  (f32 accumulator read and written, bf16 Hessian-vector product, probe
  regenerated): 10 B per parameter.
* ``adamw`` -- one step = the fused mask-aware AdamW update of every masked
  linear of the 7B model (f32 master weight, bf16 gradient, f32 moments and
  soft mask, bf16 working copy written back) in one multi-tensor call: 32 B
  per parameter.
* ``block_sparse`` -- fwd + dx + SDDMM dW of a block-sparse-16 linear at the
  gate/up shape, block densities 0.5 and 0.25, kept-block FLOPs.
* ``distill_kl`` -- the fused distillation KL of Distill_Model: forward and
  student gradient over bf16 logits [16384, 32000]; GB/s counts 10 B per
  logit (forward reads s, t; backward reads s, t and writes ds).
* ``sparse24_forward`` -- inference forward of a finalized decoder layer: the
  seven linears with hard 2:4 weights packed (kept values + 2-bit indices)
  through gfx950's sparse MFMA, beside the dense forward of the same weights;
  dense-equivalent 2 T in out FLOPs against the 2:4-sparse MFMA peak.
* ``e2e_1p1b`` -- cfg5: sparse retraining steps of a random-init
  LLaMA-architecture 1.1B model (batch 8 x 2048) with distillation, one
  Hutchinson probe, mask-aware AdamW and the periodic mask update; tokens/s
  and a per-phase breakdown.
* ``roofline`` -- the dominant kernel (the sf_gemm MFMA GEMM): algorithmic
  FLOPs of the step over the summed device time of its sf_gemm launches,
  timed with HIP events on the launch stream inside the timed region.
  ``peak`` is the published dense bf16 figure; ``mfma_sustained`` is what an
  MFMA-only loop (sf_mfma_probe, operands distributed like the GEMM's, no
  memory traffic) sustains on the same GPU.
* ``cpu_baseline`` -- the numpy oracle on the host cores: the linear leg's
  products through the BLAS threads on a bounded token sample, the HBM legs
  as one worker process per core (up to 16) each on its own slice, timed
  before the GPU is initialised (rank 0, N = 1 only).

    python bench.py [--gpus 1] [--steps 10] [--warmup 3]
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

HIDDEN, FFN, TOKENS, RANK, LAYERS = 4096, 11008, 8192, 64, 32
# (name, in, out) of the seven linears of one LLaMA-2-7B decoder layer
LINEARS = [("q_proj", HIDDEN, HIDDEN), ("k_proj", HIDDEN, HIDDEN), ("v_proj", HIDDEN, HIDDEN),
           ("o_proj", HIDDEN, HIDDEN), ("gate_proj", HIDDEN, FFN), ("up_proj", HIDDEN, FFN),
           ("down_proj", FFN, HIDDEN)]
PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_BF16_SPARSE_TFLOPS = 5000.0  # MI355X 2:4-sparse bf16 MFMA (dense-equivalent FLOPs: twice the dense rate)
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
MASK_BYTES_PER_PARAM = 20   # stats pass 6 B + update pass 14 B
ADAMW_BYTES_PER_PARAM = 32  # master r/w 8, grad 2, m r/w 8, v r/w 8, mask 4, bf16 copy 2
ALL_LEGS = ("linear", "blas", "mask", "hutch", "adamw", "bsr", "kl", "s24", "e2e")
HUTCH_BYTES_PER_PARAM = 10  # accumulator f32 r/w 8, Hessian-vector product bf16 2 (probe regenerated)


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


TRAFFIC_SUMMARY = os.path.join("profiles", "hbm_traffic_7b_layer.md")


def profiled_traffic() -> dict:
    """Per-launch HBM bytes measured by the rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (copy-calibrated) recorded in the committed traffic summary; {} when absent."""
    out = {}
    try:
        with open(os.path.join(REPO, TRAFFIC_SUMMARY)) as f:
            for line in f:
                if line.startswith("bench-traffic:"):
                    for kv in line.split(":", 1)[1].split():
                        k, v = kv.split("=")
                        out[k] = float(v) if "." in v else int(v)
    except OSError:
        pass
    return out


def flops_fwd_bwd(tokens: int, in_f: int, out_f: int, rank: int = 0) -> int:
    """Algorithmic FLOPs of one SparseLinear fwd+bwd: y, dX and dW are 2 T in out each, and the four
    rank-r SLoRB products (z, dz, dP, dS) add 6 T r (in + out)."""
    return 6 * tokens * in_f * out_f + 6 * tokens * rank * (in_f + out_f)


def step_flops(tokens: int) -> float:
    return float(sum(flops_fwd_bwd(tokens, i, o, RANK) for _, i, o in LINEARS))


# ---------------------------------------------------------------------------
# SparseLinear fwd+bwd leg
# ---------------------------------------------------------------------------
def build_layer(torch, sm, dev, tokens: int):
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                SLoRB=True, SLoRB_init_type="sum", trainable_projection=True,
                                sparsity_warmup_steps=0, tau_sample_size=262144)
    cfg.enable_hutchinson = True
    g = torch.Generator(device=dev).manual_seed(0)
    mods, xs, gys = [], [], []
    for name, fin, fout in LINEARS:
        cfg.SLoRB_k = fin // RANK
        lin = sm.SparseLinear(fin, fout, sparselinear_config=cfg, bias=False, device=dev, dtype=torch.bfloat16)
        with torch.no_grad():
            lin.weight.copy_(torch.randn(fout, fin, generator=g, device=dev) * 0.02)
            # stand-in Hutchinson accumulator: positive Hessian-diagonal estimates
            lin.hessian_diag.copy_(torch.rand(fout, fin, generator=g, device=dev) * 1e-3 + 1e-6)
            lin.initialize()
            lin.mask.copy_(lin.compute_gate_target(step=100))  # soft mask from Hessian-weighted scores
            lin.init_SLoRB()
            lin.SLoRB_Weight.copy_(torch.randn(fout, fin // lin.SLoRB_k, generator=g, device=dev) * 0.01)
        lin.hardening_x = 0.0  # E = hard 2:4 projection of the soft mask
        mods.append(lin)
        xs.append((torch.randn(tokens, fin, generator=g, device=dev)).to(torch.bfloat16).requires_grad_(True))
        gys.append(torch.randn(tokens, fout, generator=g, device=dev).to(torch.bfloat16))
    return mods, xs, gys


def linear_step(mods, xs, gys):
    for lin, x, gy in zip(mods, xs, gys):
        lin.weight.grad = None
        lin.x_proj.grad = None
        lin.SLoRB_Weight.grad = None
        x.grad = None
        y = lin(x)
        y.backward(gy)


# ---------------------------------------------------------------------------
# mask-update leg (7B arena)
# ---------------------------------------------------------------------------
def build_arena(torch, dev, layers: int):
    g = torch.Generator(device=dev).manual_seed(1)
    arena = []
    for _ in range(layers):
        for _name, fin, fout in LINEARS:
            W = (torch.randn(fout, fin, generator=g, device=dev) * 0.02).to(torch.bfloat16)
            H = torch.rand(fout, fin, generator=g, device=dev) * 1e-3 + 1e-6
            M = torch.rand(fout, fin, generator=g, device=dev)
            arena.append((W, H, M))
    return arena


def mask_params(L, rows, cols, temperature):
    p = L.MaskParams()
    p.rows, p.cols = rows, cols
    p.metric = L.METRIC["hessian_ratio"]
    p.gate = L.GATE_UNSTRUCTURED
    p.n_keep, p.m_group = 2, 4
    p.hard_kind, p.hard_n, p.hard_m = L.HARD_NM_TAIL_KEEP, 2, 4
    p.penalty = L.PENALTY_NONE
    p.score_dtype = L.DT_F32
    p.temperature = temperature
    p.eps_metric = 1e-8
    p.movement_temp = 1.0
    p.mask_lr = 0.1
    return p


def mask_jobs(torch, K, arena, sample_idx):
    """The arena's layers as batched-update jobs (per-layer stats / tau / flip outputs)."""
    dev = arena[0][0].device
    n = len(arena)
    stats = torch.empty((n, 2), dtype=torch.float32, device=dev)
    tau = torch.empty(n, dtype=torch.float32, device=dev)
    flips = torch.zeros(n, dtype=torch.int64, device=dev)
    jobs = [K.MaskJob(K.MaskOperands(weight=W, mask=M, hessian=H), sample_idx[tuple(W.shape)], stats[i],
                      tau[i:i + 1], flips[i:i + 1]) for i, (W, H, M) in enumerate(arena)]
    return jobs, K.multi_workspace(jobs, dev)


def mask_step(L, K, jobs, ws, step: int, stages=None):
    """One mask update of every linear of the arena: what calculate_model_mask does for layers that share
    their parameters, sf_update_mask_multi over the whole arena (stats, tau select and fused update of
    28 layers per launch).  stages: run only these stages (SF_MULTI_*), to time each alone."""
    temperature = 1.0 * (0.01 ** (min(step, 9) / 9.0))
    p = mask_params(L, 0, 0, temperature)
    K.update_mask_multi(p, 0.5, jobs, L.MULTI_ALL if stages is None else stages, ws)


# ---------------------------------------------------------------------------
# CPU baseline: the numpy oracle on a bounded token sample
# ---------------------------------------------------------------------------
BSR_SHAPE = (11008, 4096)  # gate/up projection of LLaMA-2-7B, 688 x 256 blocks of 16 x 16


def bsr_leg(torch, dev, tokens: int, density: float, steps: int, warmup: int) -> dict:
    """Block-sparse-16 linear at the gate/up shape: build the index, then fwd + dx + SDDMM dW per step."""
    from sparseforge_amd import block_sparse as bs
    from sparseforge_amd import profiling as prof

    out_f, in_f = BSR_SHAPE
    bm = torch.rand(out_f // 16, in_f // 16, generator=torch.Generator().manual_seed(1)) < density
    gen = torch.Generator(device=dev).manual_seed(3)
    W = (torch.randn(out_f, in_f, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
    M = bm.to(dev).repeat_interleave(16, 0).repeat_interleave(16, 1).to(torch.bfloat16)
    x = torch.randn(tokens, in_f, generator=gen, device=dev).to(torch.bfloat16)
    gy = torch.randn(tokens, out_f, generator=gen, device=dev).to(torch.bfloat16)
    bs.convert_to_block_sparse(W, M, return_block_map=True)  # warmup
    torch.cuda.synchronize()
    with prof.kernel_timer() as bt:
        t0 = time.perf_counter()
        blocks, rp, ci, bmap = bs.convert_to_block_sparse(W, M, return_block_map=True)
        torch.cuda.synchronize()
        build_ms = (time.perf_counter() - t0) * 1e3
    nnz = ci.numel()

    def step():
        bs._bsr_gemm(x, blocks, bmap, out_f, False, torch.bfloat16)
        bs._bsr_gemm(gy, blocks, bmap, in_f, True, torch.bfloat16)
        bs.bsr_sddmm(gy, x, bmap, nnz, torch.bfloat16)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    with prof.kernel_timer() as kt:
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    flops = 3 * 2.0 * tokens * nnz * 256  # kept blocks only
    gk = kt.summary()["sf_gemm_bsr"]
    kernel_tflops = flops * steps / (gk.total_ms * 1e-3) / 1e12
    build_bytes = W.numel() * 4 + nnz * 256 * 2  # read W and M (bf16), write the kept blocks
    res = {"density": density, "nnz_blocks": nnz, "total_blocks": bm.numel(), "tokens": tokens,
           "value": round(flops * steps / el / 1e12, 3), "unit": "TFLOP/s (kept blocks, fwd + dx + SDDMM dW)",
           "ms_per_step": round(el * 1e3 / steps, 4),
           "roofline": {"bound": "mfma", "kernel": "sf_gemm (block-sparse modes)", "achieved": round(kernel_tflops, 3),
                        "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                        "frac": round(kernel_tflops / PEAK_BF16_TFLOPS, 4), "launches": gk.launches,
                        "avg_launch_ms": round(gk.avg_ms, 4)},
           "build": {"ms": round(build_ms, 3), "GB/s": round(build_bytes / (build_ms * 1e-3) / 1e9, 2),
                     "kernel_ms": round(bt.summary()["sf_bsr_build"].total_ms, 3)}}
    log(f"bsr d={density}: nnz {nnz}/{bm.numel()}, {res['value']:.1f} TFLOP/s, kernels {kernel_tflops:.1f} TFLOP/s; "
        f"build {build_ms:.2f} ms")
    return res


KL_SHAPE = (8 * 2048, 32000)  # student / teacher logits of the distillation config (batch 8 x seq 2048, vocab 32000)


def kl_leg(torch, dev, steps: int, warmup: int = 2) -> dict:
    """Distillation KL forward + student gradient over bf16 logits [16384, 32000]."""
    from sparseforge_amd import profiling as prof
    from sparseforge_amd.distill import chunked_kl_loss

    gen = torch.Generator(device=dev).manual_seed(5)
    s = (torch.randn(KL_SHAPE, generator=gen, device=dev) * 4).to(torch.bfloat16).requires_grad_(True)
    t = (torch.randn(KL_SHAPE, generator=gen, device=dev) * 4).to(torch.bfloat16)

    def step():
        s.grad = None
        chunked_kl_loss(s, t, 2).backward()

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()
    with prof.kernel_timer() as kt:
        t0 = time.perf_counter()
        for _ in range(steps):
            step()
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    n = s.numel()
    nbytes = n * 2 * (2 + 3)  # forward reads s, t; backward reads s, t and writes ds (bf16)
    ks = kt.summary()
    f, b = ks["sf_kl_forward"], ks["sf_kl_backward"]
    res = {"value": round(nbytes * steps / el / 1e9, 2), "unit": "GB/s", "shape": list(KL_SHAPE), "dtype": "bf16",
           "ms_per_step": round(el * 1e3 / steps, 4), "bytes_per_element": 10,
           "roofline": {"bound": "hbm", "kernel": "sf_kl_forward", "achieved": round(f.rate / 1e9, 2),
                        "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(f.rate / 1e9 / PEAK_HBM_GBS, 4),
                        "traffic": profiled_traffic().get("sf_kl_forward_bytes_per_launch"), "traffic_unit": "B/launch",
                        "avg_launch_ms": round(f.avg_ms, 4)},
           "backward": {"kernel": "sf_kl_backward", "achieved": round(b.rate / 1e9, 2), "unit": "GB/s",
                        "avg_launch_ms": round(b.avg_ms, 4)}}
    log(f"kl: {res['ms_per_step']:.3f} ms/step (fwd + grad), {res['value']:.0f} GB/s; sf_kl_forward "
        f"{f.rate / 1e9:.0f} GB/s, sf_kl_backward {b.rate / 1e9:.0f} GB/s")
    return res


def sparse24_leg(torch, dev, tokens: int, steps: int, warmup: int = 2) -> dict:
    """Inference forward of a finalized 7B decoder layer: the seven linears with hard 2:4 weights packed
    (sf_pack_2to4) through the sparse-MFMA product, beside the dense forward of the same weights."""
    from sparseforge_amd import _lib as L
    from sparseforge_amd import finalize as F
    from sparseforge_amd import kernels as K
    from sparseforge_amd import linear as lin
    from sparseforge_amd import profiling as prof

    gen = torch.Generator(device=dev).manual_seed(11)
    layers = []
    for _name, fin, fout in LINEARS:
        W = (torch.randn(fout, fin, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        M = K.hard_mask(torch.rand(fout, fin, generator=gen, device=dev), L.HARD_NM_TAIL_KEEP, 2, 4).to(torch.bfloat16)
        Wm = lin.apply_mask(W, M)
        layers.append((F.pack_2to4(W, M), Wm, torch.randn(tokens, fin, generator=gen, device=dev).to(torch.bfloat16)))
    flops = sum(2.0 * tokens * fin * fout for _n, fin, fout in LINEARS)

    def run(sparse: bool):
        for p, Wm, x in layers:
            F.gemm_2to4(x, p) if sparse else lin.mm_nt(x, Wm)

    res = {}
    for sparse in (True, False):
        for _ in range(warmup):
            run(sparse)
        torch.cuda.synchronize()
        with prof.kernel_timer() as kt:
            t0 = time.perf_counter()
            for _ in range(steps):
                run(sparse)
            torch.cuda.synchronize()
            el = time.perf_counter() - t0
        k = kt.summary()["sf_gemm_2to4" if sparse else "sf_gemm"]
        res[sparse] = (el, flops * steps / (k.total_ms * 1e-3) / 1e12, k)
    el, ktf, k = res[True]
    del_, dtf, _ = res[False]
    out = {"value": round(flops * steps / el / 1e12, 3),
           "unit": "TFLOP/s (dense-equivalent 2 T in out of the seven forwards)",
           "ms_per_step": round(el * 1e3 / steps, 4), "tokens": tokens,
           "dense_forward": {"value": round(flops * steps / del_ / 1e12, 3), "kernel_tflops": round(dtf, 3),
                             "ms_per_step": round(del_ * 1e3 / steps, 4)},
           "speedup_vs_dense": round(del_ / el, 3),
           "roofline": {"bound": "mfma (2:4 sparse)", "kernel": "sf_gemm_2to4 (gemm24_kernel, v_smfmac_f32_32x32x32_bf16)",
                        "achieved": round(ktf, 3), "peak": PEAK_BF16_SPARSE_TFLOPS,
                        "unit": "TFLOP/s dense-equivalent", "frac": round(ktf / PEAK_BF16_SPARSE_TFLOPS, 4),
                        "frac_of_dense_peak": round(ktf / PEAK_BF16_TFLOPS, 4), "launches": k.launches,
                        "avg_launch_ms": round(k.avg_ms, 4)}}
    log(f"2:4 forward: {out['value']:.0f} TFLOP/s dense-equivalent ({out['ms_per_step']:.3f} ms), dense "
        f"{out['dense_forward']['value']:.0f} TFLOP/s, x{out['speedup_vs_dense']:.2f}")
    return out


E2E_BATCH, E2E_SEQ, E2E_START = 8, 2048, 5000


def e2e_leg(torch, dev, steps: int, warmup: int, micro: int, layers: int = 22) -> dict:
    """cfg5: sparse retraining steps of a random-init LLaMA-architecture ~1.1B student (22 layers, hidden 2048,
    FFN 5632, 32 heads, vocab 32000, bf16; every decoder projection a SparseLinear, unstructured soft mask with
    the hard 2:4 projection, SLoRB rank 64, hessian_ratio + Hutchinson) distilled from a dense random-init
    teacher of the same shape, batch 8 x seq 2048 as 8 / micro micro-batches, in the paper's schedule
    (mask update every 10 steps after step 2000, hardening from 2000 over 15000 steps) starting at step 5000:
    the timed window holds one mask update per 10 steps.  Each step: forward (student + teacher + CE + KL +
    penalties), one Hutchinson probe on the last micro-batch, backward, clipping, AdamW(decay), mask update."""
    from sparseforge_amd import sparse_modeling as sm
    from sparseforge_amd.adamw import AdamW
    from sparseforge_amd.llama import LlamaDecoder, LlamaShape
    from sparseforge_amd.retrain import PHASES, RetrainConfig, RetrainStep, optimizer_groups
    from sparseforge_amd.schedules import hardening_coefficient

    if E2E_BATCH % micro:
        raise ValueError("--e2e-micro must divide the batch of 8")
    shape = LlamaShape(num_hidden_layers=layers)
    cfg = sm.SparseLinearConfig(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                                sparsity_ratio=0.5, beta=0.98, mask_update_period_before=30,
                                mask_update_period_after=10, mask_update_switch_step=2000, mask_lr=0.1,
                                temp_init=1.0, temp_decay=0.97, temp_min=0.05, sparsity_warmup_steps=500,
                                tau_sample_size=262144, mask_penalty_lr=0.1, mask_penalty_mode="nm_2_4",
                                mask_hardening_start=2000, mask_hardening_duration=15000, SLoRB=True,
                                SLoRB_init_type="sum", trainable_projection=True)
    cfg.enable_hutchinson = True
    g = torch.Generator(device=dev).manual_seed(21)
    student = LlamaDecoder(shape, cfg, RANK, dev, torch.bfloat16)
    student.init_random(g)
    teacher = LlamaDecoder(shape, None, RANK, dev, torch.bfloat16)
    teacher.init_random(g)
    teacher.requires_grad_(False)
    hx = hardening_coefficient(cfg, E2E_START - 10)
    with torch.no_grad():  # mid-training state: soft masks from Hessian-weighted scores, hardening under way
        for m in student.modules():
            if isinstance(m, sm.SparseLinear):
                m.hessian_diag.copy_(torch.rand(m.mask.shape, generator=g, device=dev) * 1e-3 + 1e-6)
                m.mask.copy_(m.compute_gate_target(step=E2E_START - 10))
                m.hardening_x = hx
    n_student = sum(p.numel() for p in student.parameters() if p.requires_grad)
    n_sparse = sum(m.weight.numel() for m in student.modules() if isinstance(m, sm.SparseLinear))
    opt = AdamW(optimizer_groups(student, 0.1), lr=1e-4, betas=(0.9, 0.95))
    rc = RetrainConfig(grad_accum=E2E_BATCH // micro, lr=1e-4)
    step = RetrainStep(student, teacher, opt, rc, timed=True)
    tok = torch.Generator(device=dev).manual_seed(22)

    def batches():
        out = []
        for _ in range(rc.grad_accum):
            seq = torch.randint(0, shape.vocab_size, (micro, E2E_SEQ + 1), generator=tok, device=dev)
            out.append((seq[:, :-1].contiguous(), seq[:, 1:].contiguous()))
        return out

    data = [batches() for _ in range(steps + warmup)]
    it = E2E_START - warmup
    log(f"e2e: {shape.num_hidden_layers} layers, {n_student / 1e9:.3f} G trainable params "
        f"({n_sparse / 1e9:.3f} G in SparseLinear), micro-batch {micro} x {E2E_SEQ}, {rc.grad_accum} micro-batches")
    for k in range(warmup):
        step(it, data[k])
        it += 1
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    phases = {n: 0.0 for n in PHASES}
    losses = []
    t0 = time.perf_counter()
    for k in range(steps):
        r = step(it, data[warmup + k])
        it += 1
        losses.append(r.loss)
        for n, ms in r.phase_ms().items():  # waits for the step's last event (the next step is not queued yet)
            phases[n] += ms
    torch.cuda.synchronize()
    el = time.perf_counter() - t0
    tokens = E2E_BATCH * E2E_SEQ * steps
    # Model FLOPs of a step (the usual convention: 2 per multiply-add of a matrix product, the Hutchinson
    # probe's extra forward / double backward not counted): the student's forward + backward (3x its
    # forward) over every linear (projections, SLoRB factors, lm_head) and the attention products (q k^T
    # and p v over the full S x S square, as eager attention computes them), the teacher's forward.
    h, f_, v_, L_ = shape.hidden_size, shape.intermediate_size, shape.vocab_size, shape.num_hidden_layers
    proj = 4 * h * h + 3 * h * f_
    slorb = RANK * (4 * (h + h) + 3 * (h + f_))
    attn = 2 * 2 * E2E_SEQ * h  # q k^T and p v per token and layer
    per_token_fwd_student = 2 * (L_ * (proj + slorb) + h * v_) + L_ * attn
    per_token_fwd_teacher = 2 * (L_ * proj + h * v_) + L_ * attn
    model_flops = (3 * per_token_fwd_student + per_token_fwd_teacher) * E2E_BATCH * E2E_SEQ
    res = {"value": round(tokens / el, 1), "unit": "tokens/s", "steps": steps, "warmup": warmup,
           "model_tflop_per_step": round(model_flops / 1e12, 2),
           "mfu": round(model_flops * steps / el / (PEAK_BF16_TFLOPS * 1e12), 4),
           "ms_per_step": round(el * 1e3 / steps, 2), "batch": E2E_BATCH, "seq_len": E2E_SEQ, "micro_batch": micro,
           "grad_accum": rc.grad_accum, "layers": shape.num_hidden_layers, "trainable_params": n_student,
           "sparse_params": n_sparse, "first_iter": E2E_START, "hardening_x": round(hx, 4),
           "mask_updates_in_window": sum(1 for i in range(E2E_START, E2E_START + steps) if i % 10 == 0),
           "phase_ms_per_step": {n: round(v / steps, 2) for n, v in phases.items()},
           "peak_mem_gib": round(torch.cuda.max_memory_allocated(dev) / 2 ** 30, 1),
           "loss_first_last": [round(losses[0], 4), round(losses[-1], 4)],
           "data": "synthetic token ids uniform over the vocabulary; random-init student and teacher"}
    log(f"e2e: {res['ms_per_step']:.0f} ms/step, {res['value']:.0f} tokens/s, MFU {res['mfu']:.3f} "
        f"({res['model_tflop_per_step']} TFLOP of model work a step); phases {res['phase_ms_per_step']}; "
        f"peak {res['peak_mem_gib']} GiB")
    del step, opt, student, teacher, data
    return res


def mfma_sustained(torch, dev, iters: int = 4000, blocks: int = 1024, reps: int = 6) -> float:
    """TFLOP/s of sf_mfma_probe (MFMA-only loop, bf16 register operands distributed like the GEMM's):
    the rate this GPU sustains on the bf16 MFMA pipe alone, best of `reps` after a clock ramp-up."""
    from sparseforge_amd import _lib as L

    out = torch.empty(blocks * 256, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev)
    flops = blocks * 4.0 * iters * 16 * 32768
    best = 0.0
    for r in range(reps + 3):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        L.check(L.lib().sf_mfma_probe(iters, blocks, L.ptr(out), L.stream(dev)), "sf_mfma_probe")
        e1.record(st)
        e1.synchronize()
        if r >= 3:
            best = max(best, flops / (e0.elapsed_time(e1) * 1e-3) / 1e12)
    log(f"MFMA-only probe: {best:.0f} TFLOP/s sustained (bf16 32x32x16, normal-like operands)")
    return best


def blas_leg(torch, dev, tokens: int, reps: int = 20) -> dict:
    """The three GEMM products of each distinct 7B linear shape (fwd x W^T, dx = gy W, dW = gy^T x; bf16,
    no mask, no SLoRB) through sf_gemm and through torch.matmul (hipBLASLt), and the layer's 21 products
    weighted by how many linears share each shape."""
    from sparseforge_amd import linear as lin

    def timeit(fn):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1) / reps

    g = torch.Generator(device=dev).manual_seed(5)
    rows, tot = {}, {"sf_gemm": 0.0, "hipblaslt": 0.0}
    count = {}
    for _name, fin, fout in LINEARS:
        count[(fin, fout)] = count.get((fin, fout), 0) + 1
    flops_layer = 0.0
    for (fin, fout), k in count.items():
        x = torch.randn(tokens, fin, generator=g, device=dev).to(torch.bfloat16)
        W = (torch.randn(fout, fin, generator=g, device=dev) * 0.02).to(torch.bfloat16)
        gy = torch.randn(tokens, fout, generator=g, device=dev).to(torch.bfloat16)
        fl = 2.0 * tokens * fin * fout
        prods = {"fwd": (lambda: lin.mm_nt(x, W), lambda: x @ W.t()),
                 "dx": (lambda: lin.mm_nn(gy, W), lambda: gy @ W),
                 "dw": (lambda: lin.mm_tn(gy, x), lambda: gy.t() @ x)}
        row = {}
        for pname, (f_sf, f_bl) in prods.items():
            a, b = timeit(f_sf), timeit(f_bl)
            row[pname] = {"sf_gemm_TFLOP/s": round(fl / a / 1e9, 1), "hipblaslt_TFLOP/s": round(fl / b / 1e9, 1)}
            tot["sf_gemm"] += k * a
            tot["hipblaslt"] += k * b
            flops_layer += k * fl
        rows[f"{fout}x{fin}"] = row
        del x, W, gy
    torch.cuda.empty_cache()
    out = {"tokens": tokens, "products": rows,
           "layer_21_products_ms": {k: round(v, 3) for k, v in tot.items()},
           "layer_21_products_TFLOP/s": {k: round(flops_layer / v / 1e9, 1) for k, v in tot.items()}}
    log("GEMM vs hipBLASLt, the layer's 21 products: " + ", ".join(
        f"{k} {v:.2f} ms" for k, v in out["layer_21_products_ms"].items()))
    return out


def hbm_sustained(torch, dev, n: int = 180 * (1 << 20), reps: int = 5) -> dict:
    """GB/s of sf_hbm_probe's streams (token arithmetic) over n elements, best over grid sizes and reps:
    what this GPU's HBM sustains for the fused mask update's traffic (read W bf16, H f32, M f32, write M:
    14 B/elem), the score statistics' (read W, H: 6 B/elem) and a plain copy (8 B/elem)."""
    from sparseforge_amd import _lib as L

    W = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    H = torch.zeros(n, dtype=torch.float32, device=dev)
    M = torch.zeros(n, dtype=torch.float32, device=dev)
    st = torch.cuda.current_stream(dev)
    out = {}
    for name, pattern, nbytes in (("update_pattern", 0, 14), ("stats_pattern", 1, 6), ("copy", 2, 8)):
        best = 0.0
        for blocks in (2048, 4096, 16384):
            for r in range(reps + 2):
                e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                e0.record(st)
                L.check(L.lib().sf_hbm_probe(pattern, L.ptr(W), L.ptr(H), L.ptr(M), n, blocks, L.stream(dev)),
                        "sf_hbm_probe")
                e1.record(st)
                e1.synchronize()
                if r >= 2:
                    best = max(best, nbytes * n / (e0.elapsed_time(e1) * 1e-3) / 1e9)
        out[name] = round(best, 1)
    del W, H, M
    torch.cuda.empty_cache()
    log("HBM probe: " + ", ".join(f"{k} {v:.0f} GB/s" for k, v in out.items()))
    return out


def cpu_baseline(budget_s: float = 15.0, tokens: int = 512) -> dict:
    import numpy as np

    from oracle import linear as ol
    from oracle.masks import hard_mask_from_soft

    try:
        from threadpoolctl import threadpool_info

        cores = max([int(i.get("num_threads", 1)) for i in threadpool_info() if i.get("user_api") == "blas"] or [1])
    except Exception:
        cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    rng = np.random.default_rng(0)
    shapes = []
    for _name, fin, fout in LINEARS:
        W = (rng.standard_normal((fout, fin), dtype=np.float32) * 0.02)
        E = hard_mask_from_soft(rng.random((fout, fin), dtype=np.float32), "nm_2_4")
        k = fin // RANK
        P = np.zeros((RANK, fin), np.float32)
        P[np.arange(RANK)[:, None], np.arange(RANK)[:, None] * k + np.arange(k)] = 1.0
        S = rng.standard_normal((fout, RANK), dtype=np.float32) * 0.01
        x = rng.standard_normal((tokens, fin), dtype=np.float32)
        gy = rng.standard_normal((tokens, fout), dtype=np.float32)
        shapes.append((x, W, E, P, S, gy))
    flops_per_rep = step_flops(tokens)
    reps, t0 = 0, time.perf_counter()
    while True:
        for x, W, E, P, S, gy in shapes:
            ol.forward(x, W, E, None, 1.0, P, S)
            ol.backward(x, W, E, gy, False, P, S)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s or reps >= 50:
            break
    return {"value": round(flops_per_rep * reps / el / 1e12, 4), "unit": "TFLOP/s", "cores": cores, "kind": "port",
            "sample": f"numpy fp32 oracle (oracle/linear.py) fwd+bwd of the 7 decoder-layer linears at T={tokens} "
                      f"tokens (full shapes, SLoRB rank {RANK}), {reps} reps in {el:.1f} s"}


def cpu_pool_size() -> int:
    """Worker processes of the CPU baselines: the host cores, at most 16 (one GPU's CPU share on the box)."""
    return max(1, min(16, os.cpu_count() or 1))


def _single_thread_blas():
    try:
        from threadpoolctl import threadpool_limits

        threadpool_limits(1)
    except Exception:
        pass


def _adamw_worker(args):
    """One core: oracle AdamW steps over its own 4 M-parameter slice until the budget runs out."""
    seed, budget_s = args
    import numpy as np

    from oracle import adamw as oa

    _single_thread_blas()
    rng = np.random.default_rng(seed)
    n = 1 << 22
    p = (rng.standard_normal(n, dtype=np.float32) * 0.02)
    g = (rng.standard_normal(n, dtype=np.float32) * 1e-3)
    mask = rng.random(n, dtype=np.float32)
    m, v = np.zeros(n, np.float32), np.zeros(n, np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        p, m, v, _ = oa.step(p, g, m, v, None, mask, reps + 1, 1e-4, (0.9, 0.95), 1e-8, 0.1, decay=6e-5)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return n * reps / el


def _mask_worker(args):
    """One core: oracle mask updates (stats, tau quantile, gate, penalty, EMA, flips) of its own
    [1024, 4096] slice of a linear until the budget runs out."""
    seed, budget_s = args
    import numpy as np

    from oracle import masks as om

    _single_thread_blas()
    rng = np.random.default_rng(seed)
    rows, cols = 1024, HIDDEN
    W = om.round_bf16(rng.standard_normal((rows, cols), dtype=np.float32) * 0.02)
    H = rng.random((rows, cols), dtype=np.float32) * 1e-3 + 1e-6
    M = rng.random((rows, cols), dtype=np.float32)
    c = om.full_config(mask_type="unstructured", hard_mask_type="nm_2_4", mask_metric="hessian_ratio",
                       sparsity_warmup_steps=0, mask_update_period=1, tau_sample_size=262144)
    idx = rng.integers(0, rows * cols, 262144)
    reps, t0 = 0, time.perf_counter()
    while True:
        M = om.layer_update_mask(c, 1 + reps, W, H, M, None, idx, 0.0, w_dt="bf16")[0]
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return rows * cols * reps / el


def _hutch_worker(args):
    """One core: oracle Hutchinson accumulator updates (probe regenerated, clamp, EMA) of 4 M elements."""
    seed, budget_s = args
    import numpy as np

    from oracle import hutchinson as oh

    _single_thread_blas()
    rng = np.random.default_rng(seed)
    n = 1 << 22
    H = rng.random(n, dtype=np.float32) * 1e-3
    hvp = rng.standard_normal(n, dtype=np.float32)
    reps, t0 = 0, time.perf_counter()
    while True:
        H = oh.update(H, hvp, oh.rademacher(seed * 1000 + reps, n), 0.98)
        reps += 1
        el = time.perf_counter() - t0
        if el >= budget_s:
            return n * reps / el


def cpu_parallel_baseline(worker, bytes_per_param: int, budget_s: float, what: str) -> dict:
    """Run `worker` on every pool core at once (each on its own slice); the aggregate rate in GB/s.
    Called before the GPU is initialised: worker processes are forked from a process without a GPU context."""
    import multiprocessing as mp

    n = cpu_pool_size()
    with mp.get_context("fork").Pool(n) as pool:
        rates = pool.map(worker, [(7 + i, budget_s) for i in range(n)])
    params_per_s = float(sum(rates))
    return {"value": round(bytes_per_param * params_per_s / 1e9, 3), "unit": "GB/s", "cores": n, "kind": "port",
            "sample": f"{what}: {n} processes, one per core, each on its own slice for {budget_s:.0f} s; "
                      f"{bytes_per_param} B/param"}


# ---------------------------------------------------------------------------
def per_linear_times(torch, mods, xs, gys, reps: int = 5) -> list:
    """cfg2's per-linear figure: fwd + bwd of each linear alone (device events around each repetition)."""
    out = []
    for (name, fin, fout), lin, x, gy in zip(LINEARS, mods, xs, gys):
        for _ in range(2):
            linear_step([lin], [x], [gy])
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
        for e0, e1 in ev:
            e0.record()
            linear_step([lin], [x], [gy])
            e1.record()
        torch.cuda.synchronize()
        ms = min(e0.elapsed_time(e1) for e0, e1 in ev)
        fl = flops_fwd_bwd(x.shape[0], fin, fout, RANK)
        out.append({"linear": name, "in": fin, "out": fout, "ms": round(ms, 4),
                    "TFLOP/s": round(fl / (ms * 1e-3) / 1e12, 2)})
    return out


def hvp_layer_leg(torch, mods, xs, reps: int = 3) -> dict:
    """Hutchinson probe of one decoder layer's seven linears at T = 8192 (hard 2:4, SLoRB): the
    update_hessian_hutchinson call after a forward (first-order gradients with create_graph, the probe
    dot, the double backward, the seven accumulator updates), on a quadratic loss sum 1/2 ||y||^2."""
    from sparseforge_amd import utils as U

    model = torch.nn.ModuleList(mods)
    times = []
    for r in range(reps + 1):
        ys = [lin(x) for lin, x in zip(mods, xs)]
        loss = sum(0.5 * (y.float() ** 2).sum() for y in ys)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        U.update_hessian_hutchinson(model, loss)
        e1.record()
        torch.cuda.synchronize()
        del ys, loss
        if r:
            times.append(e0.elapsed_time(e1))
    for lin, x in zip(mods, xs):
        lin.weight.grad = lin.x_proj.grad = lin.SLoRB_Weight.grad = x.grad = None
    ms = min(times)
    log(f"hutchinson probe of one decoder layer (7 linears, T={xs[0].shape[0]}): {ms:.2f} ms")
    return {"ms_per_layer": round(ms, 3), "linears": len(mods), "tokens": xs[0].shape[0],
            "what": "update_hessian_hutchinson after a forward: create_graph gradients, probe dot, double "
                    "backward, accumulator updates; quadratic loss"}


def hutch_arena_leg(torch, arena, steps: int) -> dict:
    """The accumulator update of every linear of the 7B arena: H (f32) <- beta H + (1 - beta) clamp(hvp v, 0)
    with a bf16 Hessian-vector product and the probe regenerated from the seed: 10 B per parameter."""
    from sparseforge_amd import profiling as prof
    from sparseforge_amd import utils as U

    n = sum(W.numel() for W, _, _ in arena)
    # the whole arena in one multi-tensor call, as update_hessian_hutchinson issues it (the arena's bf16 W
    # stands in for the bf16 Hessian-vector product)
    U.hutchinson_update_multi_([(H, W, 0.98, k) for k, (W, H, _M) in enumerate(arena)])  # warmup
    torch.cuda.synchronize()
    with prof.kernel_timer() as kt:
        t0 = time.perf_counter()
        for s_ in range(steps):
            U.hutchinson_update_multi_([(H, W, 0.98, (s_ + 1) * 1000 + k) for k, (W, H, _M) in enumerate(arena)])
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    k_ = kt.summary()["sf_hutchinson_update_multi"]
    gbs = HUTCH_BYTES_PER_PARAM * n * steps / el / 1e9
    log(f"hutchinson update: {el * 1e3 / steps:.2f} ms over the arena, {gbs:.0f} GB/s; kernel {k_.rate / 1e9:.0f} GB/s")
    return {"value": round(gbs, 2), "unit": "GB/s", "params": n, "steps": steps,
            "ms_per_step": round(el * 1e3 / steps, 3), "bytes_per_param": HUTCH_BYTES_PER_PARAM,
            "roofline": {"bound": "hbm", "kernel": "sf_hutchinson_update_multi (hutch_update_multi_kernel)",
                         "achieved": round(k_.rate / 1e9, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(k_.rate / 1e9 / PEAK_HBM_GBS, 4), "launches": k_.launches,
                         "avg_launch_ms": round(k_.avg_ms, 4),
                         "traffic": profiled_traffic().get("sf_hutch_bytes_per_param"), "traffic_unit": "B/param",
                         "traffic_source": TRAFFIC_SUMMARY}}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--tokens", type=int, default=TOKENS)
    ap.add_argument("--mask-layers", type=int, default=LAYERS, help="decoder layers in the mask-update arena")
    ap.add_argument("--mask-steps", type=int, default=10)
    ap.add_argument("--adamw-steps", type=int, default=10,
                    help="steps of the AdamW leg (the first step's host-side table build is not overlapped)")
    ap.add_argument("--hutch-steps", type=int, default=10, help="updates of the Hutchinson accumulator leg")
    ap.add_argument("--bsr-steps", type=int, default=5, help="steps of the block-sparse leg (0 skips it)")
    ap.add_argument("--kl-steps", type=int, default=10, help="steps of the distillation-KL leg (0 skips it)")
    ap.add_argument("--s24-steps", type=int, default=10,
                    help="steps of the 2:4 packed inference-forward leg (0 skips it)")
    ap.add_argument("--e2e-steps", type=int, default=10,
                    help="timed steps of the end-to-end 1.1B retraining leg (0 skips it)")
    ap.add_argument("--e2e-warmup", type=int, default=2)
    ap.add_argument("--e2e-micro", type=int, default=2, help="micro-batch of the end-to-end leg (divides 8)")
    ap.add_argument("--e2e-layers", type=int, default=22)
    ap.add_argument("--e2e-only", action="store_true", help="run only the end-to-end leg")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline legs")
    ap.add_argument("--legs", default=",".join(ALL_LEGS),
                    help=f"comma-separated GPU legs to run (default all: {','.join(ALL_LEGS)}); profiling runs pick one")
    ap.add_argument("--calib", action="store_true",
                    help="first run one plain 256 MiB device copy (a known-size reference for HBM byte counters)")
    a = ap.parse_args(argv)

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if a.gpus != 1 or world != 1:
        print("bench.py: this build measures one MI355X only (no multi-GPU path); run with --gpus 1", file=sys.stderr)
        return 2

    legs = set(a.legs.split(","))
    unknown = legs - set(ALL_LEGS)
    if unknown:
        print(f"bench.py: unknown legs {sorted(unknown)}", file=sys.stderr)
        return 2
    # CPU baselines first: their worker processes are forked before anything touches the GPU
    cpu = {}
    if not a.no_cpu and not a.e2e_only and "linear" in legs:
        log(f"timing CPU baselines (numpy oracle, {cpu_pool_size()} worker processes for the HBM legs)")
        cpu["linear"] = cpu_baseline()
        cpu["mask"] = cpu_parallel_baseline(_mask_worker, MASK_BYTES_PER_PARAM, 8.0,
                                            "oracle/masks.py layer_update_mask on [1024, 4096] slices")
        cpu["adamw"] = cpu_parallel_baseline(_adamw_worker, ADAMW_BYTES_PER_PARAM, 6.0,
                                             "oracle/adamw.py step on 4 M-parameter slices")
        cpu["hutch"] = cpu_parallel_baseline(_hutch_worker, HUTCH_BYTES_PER_PARAM, 4.0,
                                             "oracle/hutchinson.py update (probe regenerated) on 4 M-element slices")

    import torch

    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        return 1
    from sparseforge_amd import _lib as L
    from sparseforge_amd import kernels as K
    from sparseforge_amd import profiling as prof
    from sparseforge_amd import sparse_modeling as sm

    L.load()
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if a.e2e_only:
        print(json.dumps({"e2e_1p1b": e2e_leg(torch, dev, a.e2e_steps, a.e2e_warmup, a.e2e_micro, a.e2e_layers)}),
              flush=True)
        return 0
    if a.calib:
        src = torch.ones(64 << 20, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)  # reads 256 MiB, writes 256 MiB
        torch.cuda.synchronize()
        del src, dst

    # ---- SparseLinear leg ---------------------------------------------------
    out = {"metric": "SparseLinear fwd+bwd TFLOP/s @7B shapes; 2:4 mask-update HBM GB/s"}
    if "linear" in legs:
        out.update(linear_leg(torch, sm, prof, dev, a))
    if "blas" in legs:
        out["gemm_vs_hipblaslt"] = blas_leg(torch, dev, a.tokens)
    if legs & {"mask", "hutch", "adamw"}:
        arena_legs(torch, L, K, prof, dev, a, legs, out)
    # ---- block-sparse-16 leg (gate/up shape, block densities 0.5 and 0.25) ----
    if "bsr" in legs and a.bsr_steps > 0:
        out["block_sparse"] = [bsr_leg(torch, dev, a.tokens, d, a.bsr_steps, 2) for d in (0.5, 0.25)]
        torch.cuda.empty_cache()
    if "kl" in legs and a.kl_steps > 0:
        out["distill_kl"] = kl_leg(torch, dev, a.kl_steps)
    if "s24" in legs and a.s24_steps > 0:
        out["sparse24_forward"] = sparse24_leg(torch, dev, a.tokens, a.s24_steps)
    torch.cuda.empty_cache()
    if "e2e" in legs and a.e2e_steps > 0:
        out["e2e_1p1b"] = e2e_leg(torch, dev, a.e2e_steps, a.e2e_warmup, a.e2e_micro, a.e2e_layers)
    torch.cuda.empty_cache()
    if "linear" in legs:
        sustained = mfma_sustained(torch, dev)
        out["roofline"]["mfma_sustained"] = round(sustained, 1)
        out["roofline"]["frac_of_sustained"] = round(out["roofline"]["achieved"] / sustained, 4)
    if cpu:
        out["cpu_baseline"] = cpu["linear"]
        if "mask_update" in out:
            out["mask_update"]["cpu_baseline"] = cpu["mask"]
        if "adamw" in out:
            out["adamw"]["cpu_baseline"] = cpu["adamw"]
        if "hutchinson" in out:
            out["hutchinson"]["cpu_baseline"] = cpu["hutch"]
    print(json.dumps(out), flush=True)
    return 0


def linear_leg(torch, sm, prof, dev, a) -> dict:
    """The headline leg: fwd + bwd of the seven 7B-layer linears; the fields of the bench line."""
    log(f"building decoder layer (T={a.tokens}, bf16, SLoRB rank {RANK})")
    mods, xs, gys = build_layer(torch, sm, dev, a.tokens)
    for _ in range(a.warmup):
        linear_step(mods, xs, gys)
    torch.cuda.synchronize()
    log(f"warmup done; timing {a.steps} steps")
    with prof.kernel_timer() as kt:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(a.steps):
            linear_step(mods, xs, gys)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    ks = kt.summary()
    flops = step_flops(a.tokens)
    ms_per_step = el * 1e3 / a.steps
    tflops = flops * a.steps / el / 1e12
    # sf_gemm: the dense products (input and weight gradients, the SLoRB products); its own FLOPs over
    # its own device time.  The hardening_x = 0 forward runs on the 2:4 sparse MFMA (sf_gemm_2to4),
    # reported against the sparse peak in dense-equivalent FLOPs.
    g = ks["sf_gemm"]
    gemm_tflops = g.rate / 1e12
    s24 = ks.get("sf_gemm_2to4")
    log(f"linear: {ms_per_step:.2f} ms/step, {tflops:.1f} TFLOP/s; sf_gemm {g.launches} launches, "
        f"avg {g.avg_ms:.3f} ms, {gemm_tflops:.1f} TFLOP/s" +
        (f"; sf_gemm_2to4 {s24.launches} launches, {s24.rate / 1e12:.1f} TFLOP/s dense-equivalent" if s24 else ""))
    other = {n: {"launches": s.launches, "avg_ms": round(s.avg_ms, 4), "total_ms": round(s.total_ms, 3)}
             for n, s in ks.items()}
    per_linear = per_linear_times(torch, mods, xs, gys)
    log("per linear: " + ", ".join(f"{r['linear']} {r['ms']:.3f} ms" for r in per_linear))
    mixed = mixed_phase_leg(torch, prof, mods, xs, gys, a.steps, flops)
    hvp = hvp_layer_leg(torch, mods, xs)
    del mods, xs, gys
    torch.cuda.empty_cache()
    traffic = profiled_traffic()
    return {
        "value": round(tflops, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (random-init W ~ N(0, 0.02), x ~ N(0, 1), Hessian accumulator ~ U(1e-6, 1e-3))",
        "config": {"workload": "LLaMA-2-7B decoder-layer SparseLinear fwd+bwd (q/k/v/o 4096x4096, gate/up "
                               "11008x4096, down 4096x11008), hard 2:4 mask (hardening_x=0), SLoRB rank 64",
                   "tokens": a.tokens, "linears": len(LINEARS), "flops_per_step": flops},
        "roofline": {"bound": "mfma", "achieved": round(gemm_tflops, 3), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(gemm_tflops / PEAK_BF16_TFLOPS, 4),
                     "traffic": traffic.get("sf_gemm_bytes_per_launch"), "traffic_unit": "B/launch",
                     "traffic_source": TRAFFIC_SUMMARY,
                     "kernel": "sf_gemm (gemm_bf16_kernel, skinny_kernel)", "launches": g.launches,
                     "avg_launch_ms": round(g.avg_ms, 4)},
        "sparse_forward": None if s24 is None else {
            "kernel": "sf_gemm_2to4 (gemm24_kernel, v_smfmac_f32_32x32x32_bf16)", "launches": s24.launches,
            "avg_launch_ms": round(s24.avg_ms, 4), "achieved": round(s24.rate / 1e12, 3),
            "unit": "TFLOP/s dense-equivalent", "peak": PEAK_BF16_SPARSE_TFLOPS,
            "frac": round(s24.rate / 1e12 / PEAK_BF16_SPARSE_TFLOPS, 4)},
        "per_linear": per_linear,
        "mixed_phase": mixed,
        "hutchinson_probe_layer": hvp,
        "kernels": other,
    }


def mixed_phase_leg(torch, prof, mods, xs, gys, steps: int, flops: float) -> dict:
    """The same layer step in the hardening phase (0 < hardening_x < 1, most of a training run: the
    paper's schedule spends steps 2000..17000 there): E = hx * soft + (1 - hx) * hard(soft) in bf16, the
    forward on the dense kernel over the masked weight one elementwise pass writes."""
    hx0 = [m.hardening_x for m in mods]
    for m in mods:
        m.hardening_x = 0.5
    for _ in range(2):
        linear_step(mods, xs, gys)
    with prof.kernel_timer() as kt:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            linear_step(mods, xs, gys)
        torch.cuda.synchronize()
        el = time.perf_counter() - t0
    for m, h in zip(mods, hx0):
        m.hardening_x = h
    ks = kt.summary()
    g = ks["sf_gemm"]
    res = {"hardening_x": 0.5, "ms_per_step": round(el * 1e3 / steps, 4),
           "TFLOP/s": round(flops * steps / el / 1e12, 3),
           "sf_gemm": {"launches": g.launches, "avg_ms": round(g.avg_ms, 4), "TFLOP/s": round(g.rate / 1e12, 3),
                       "frac": round(g.rate / 1e12 / PEAK_BF16_TFLOPS, 4)},
           "kernels": {n: {"launches": k.launches, "avg_ms": round(k.avg_ms, 4), "total_ms": round(k.total_ms, 3)}
                       for n, k in ks.items()}}
    log(f"mixed phase (hardening_x = 0.5): {res['ms_per_step']:.2f} ms/step, {res['TFLOP/s']:.1f} TFLOP/s; "
        f"sf_gemm {g.rate / 1e12:.1f} TFLOP/s")
    return res


def arena_legs(torch, L, K, prof, dev, a, legs, out) -> None:
    """The 7B-arena HBM legs: mask update (+ mask statistics), Hutchinson accumulator, AdamW."""
    log(f"building mask arena ({a.mask_layers} layers x 7 linears)")
    arena = build_arena(torch, dev, a.mask_layers)
    n_params = sum(W.numel() for W, _, _ in arena)
    traffic = profiled_traffic()
    if "mask" in legs:
        # the tau samples: sorted draws (sf_sample_indices_sorted, what update_mask and calculate_model_mask
        # draw), one per layer shape, reused by every layer and update as a fixed input
        sample_idx = {}
        for W, _, _ in arena:
            key = tuple(W.shape)
            if key not in sample_idx:
                sample_idx[key] = K.sample_indices_sorted(262144, [W.numel()], [1234 + len(sample_idx)], dev)[0]
        # what drawing a fresh sample for every layer costs (calculate_model_mask's draws: one call per sample
        # size, the layers' lists in launches of 64)
        numels = [W.numel() for W, _, _ in arena]
        K.sample_indices_sorted(262144, numels, list(range(len(numels))), dev)
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        K.sample_indices_sorted(262144, numels, list(range(len(numels))), dev)
        e1.record()
        torch.cuda.synchronize()
        sampler_ms = e0.elapsed_time(e1)
        log(f"sorted tau samples for all {len(numels)} layers: {sampler_ms:.3f} ms")
        jobs, mws = mask_jobs(torch, K, arena, sample_idx)
        mask_step(L, K, jobs, mws, 0)  # warmup
        torch.cuda.synchronize()
        log(f"mask arena: {n_params / 1e9:.3f} G params; timing {a.mask_steps} updates")
        t0 = time.perf_counter()
        for s in range(a.mask_steps):
            mask_step(L, K, jobs, mws, s)
        torch.cuda.synchronize()
        mel = time.perf_counter() - t0
        # each stage alone over the arena (HIP events around each batched call): the statistics pass
        # (6 B/param), the tau selection, the fused update (14 B/param)
        stage_ms = {}
        for name, stg in (("stats", L.MULTI_STATS), ("tau", L.MULTI_TAU), ("update", L.MULTI_UPDATE)):
            with prof.kernel_timer() as mt:
                mask_step(L, K, jobs, mws, a.mask_steps, stg)
            stage_ms[name] = mt.summary()["sf_update_mask_multi"]
        mask_gbs = MASK_BYTES_PER_PARAM * n_params * a.mask_steps / mel / 1e9
        sustained = hbm_sustained(torch, dev)
        up = stage_ms["update"]
        up_gbs = up.rate / 1e9
        st_gbs = stage_ms["stats"].rate / 1e9
        log(f"mask update: {mel * 1e3 / a.mask_steps:.2f} ms/update of the arena, {mask_gbs:.0f} GB/s; "
            f"update stage {up_gbs:.0f} GB/s, stats stage {st_gbs:.0f} GB/s, tau {stage_ms['tau'].total_ms:.2f} ms")
        # mask statistics / penalties of the whole model: one fused sf_mask_stats pass per soft mask (4 B/param)
        srows = torch.empty((len(arena), L.MSTAT_COUNT), dtype=torch.float64, device=dev)
        sws = K.mask_stats_workspace(dev)
        for i, (_W, _H, M) in enumerate(arena):
            K.mask_stats(M, srows[i], 0, 1e-8, sws)
        torch.cuda.synchronize()
        with prof.kernel_timer() as mst:
            for i, (_W, _H, M) in enumerate(arena):
                K.mask_stats(M, srows[i], 0, 1e-8, sws)
            torch.cuda.synchronize()
        msk = mst.summary()["sf_mask_stats"]
        mstats_gbs = msk.rate / 1e9
        log(f"mask statistics: sf_mask_stats {mstats_gbs:.0f} GB/s over {len(arena)} masks")
        out["mask_update"] = {
            "value": round(mask_gbs, 2), "unit": "GB/s", "params": n_params, "updates": a.mask_steps,
            "ms_per_update": round(mel * 1e3 / a.mask_steps, 3), "bytes_per_param": MASK_BYTES_PER_PARAM,
            "roofline": {"bound": "hbm", "kernel": "sf_update_mask_multi (update stage, update_mask_multi_kernel)",
                         "achieved": round(up_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": round(up_gbs / PEAK_HBM_GBS, 4),
                         "traffic": traffic.get("sf_update_mask_bytes_per_param"), "traffic_unit": "B/param",
                         "bytes_per_param": 14, "avg_launch_ms": round(up.avg_ms, 4),
                         "frac_of_sustained": round(up_gbs / sustained["update_pattern"], 4)},
            "arena_frac": round(mask_gbs / PEAK_HBM_GBS, 4),
            "hbm_sustained": sustained,
            # the arena's best time at the sustained rates of its two streams (update 14 B, statistics 6 B per
            # param, the tau select free) against the measured update
            "arena_frac_of_sustained": round(
                (14 / sustained["update_pattern"] + 6 / sustained["stats_pattern"]) * mask_gbs / 20, 4),
            "score_stats_gbs": round(st_gbs, 2),
            "sampler_ms_all_layers": round(sampler_ms, 3),
            "stage_ms": {k: round(v.total_ms, 3) for k, v in stage_ms.items()},
            # sixteen statistics per element: bound by VALU issue (about 58 instructions per element)
            "mask_stats": {"kernel": "sf_mask_stats", "GB/s": round(mstats_gbs, 2), "bytes_per_param": 4,
                           "bound": "valu", "frac_of_hbm": round(mstats_gbs / PEAK_HBM_GBS, 4),
                           "launches": msk.launches,
                           "avg_launch_ms": round(msk.avg_ms, 4)},
        }
    if "hutch" in legs and a.hutch_steps > 0:
        out["hutchinson"] = hutch_arena_leg(torch, arena, a.hutch_steps)
    if "adamw" not in legs:
        del arena
        torch.cuda.empty_cache()
        return
    # ---- mask-aware AdamW leg (same arena: W is the bf16 copy, M the mask) ---
    from sparseforge_amd.adamw import TensorStep, adamw_step_multi_

    log("building AdamW state (f32 master, bf16 grad, f32 m / v)")
    gen = torch.Generator(device=dev).manual_seed(2)
    opt_state = []
    arena = [(W, M) for W, _H, M in arena]  # the Hutchinson accumulator is not an AdamW operand: free it
    for W, M in arena:
        master = W.float()
        grad = (torch.randn(W.shape, generator=gen, device=dev) * 1e-3).to(torch.bfloat16)
        opt_state.append((master, grad, torch.zeros_like(master), torch.zeros_like(master), M, W))
    torch.cuda.synchronize()
    items = [TensorStep(master, grad, m, v, None, M, W) for master, grad, m, v, M, W in opt_state]

    def adamw_leg_step(k):
        # the whole arena in one sf_adamw_step_multi call (a launch per 40 tensors)
        adamw_step_multi_(items, k, 1e-4, (0.9, 0.95), 1e-8, 0.1, decay=6e-5)

    adamw_leg_step(1)  # warmup
    torch.cuda.synchronize()
    with prof.kernel_timer() as at:
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(a.adamw_steps):
            adamw_leg_step(k + 2)
        torch.cuda.synchronize()
        ael = time.perf_counter() - t0
    as_ = at.summary()["sf_adamw_step_multi"]
    adamw_gbs = ADAMW_BYTES_PER_PARAM * n_params * a.adamw_steps / ael / 1e9
    log(f"adamw: {ael * 1e3 / a.adamw_steps:.2f} ms/step of the arena, {adamw_gbs:.0f} GB/s; "
        f"sf_adamw_step_multi {as_.rate / 1e9:.0f} GB/s over kernel time")
    out["adamw"] = {
        "value": round(adamw_gbs, 2), "unit": "GB/s", "params": n_params, "steps": a.adamw_steps,
        "ms_per_step": round(ael * 1e3 / a.adamw_steps, 3), "bytes_per_param": ADAMW_BYTES_PER_PARAM,
        "roofline": {"bound": "hbm", "kernel": "sf_adamw_step_multi (adamw_multi_kernel)",
                     "achieved": round(as_.rate / 1e9, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(as_.rate / 1e9 / PEAK_HBM_GBS, 4),
                     "traffic": traffic.get("sf_adamw_bytes_per_param"), "traffic_unit": "B/param",
                     "launches": as_.launches, "avg_launch_ms": round(as_.avg_ms, 4)},
    }
    del arena, opt_state, items
    torch.cuda.empty_cache()


if __name__ == "__main__":
    sys.exit(main())
