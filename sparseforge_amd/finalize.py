"""Finalization of a trained sparse model and the 2:4 packed inference forward.

  finalize_sparse_model               legacy/main_llama.py:2499-2568 (the
                                      single-process branch): hard masks,
                                      weights multiplied by them, masks frozen
  optimize_sparse_model_for_inference legacy/eval_wiki_ppl.py:548-651
  pack_2to4 / unpack_2to4             the packed 2:4 layout of a hardened
                                      weight (sf_pack_2to4): kept values +
                                      2-bit column indices, half the bytes
  SparseLinear24 / convert_model_to_2to4
                                      forward-only layers that run the packed
                                      weight through gfx950's sparse MFMA
                                      (sf_gemm_2to4); same result as the
                                      finalized dense_forward F.linear

The reference's finalized model keeps the dense [out, in] weight with zeros;
the packed layer is the MI355X inference form of the same weights.
"""
from __future__ import annotations

from dataclasses import dataclass

import ctypes

import torch

from . import _lib as L
from . import linear as LIN
from . import profiling as _prof
from .sparse_modeling import SparseLinear


@dataclass
class Packed2to4:
    vals: torch.Tensor   # [out, in / 2] bf16
    idx: torch.Tensor    # uint8 [out * in / 8]: u32 words [out / 32][in / 64][2][32]
    out_features: int
    in_features: int


@torch.no_grad()
def pack_2to4(weight: torch.Tensor, mask: torch.Tensor) -> Packed2to4:
    """Pack weight * mask (kept where mask != 0) into the 2:4 layout; ValueError when some group of 4
    keeps more than two columns (one host read of the count)."""
    dev = L.require_device(weight, mask)
    if weight.dim() != 2 or weight.shape != mask.shape:
        raise ValueError("pack_2to4 expects a 2-D weight and a mask of the same shape")
    out_f, in_f = weight.shape
    if out_f % 32 or in_f % 64:
        raise ValueError(f"2:4 packing needs out % 32 == 0 and in % 64 == 0 (got {out_f} x {in_f})")
    ib = ctypes.c_size_t(0)
    vb = L.lib().sf_pack_2to4_sizes(out_f, in_f, ctypes.byref(ib))
    vals = torch.empty(vb // 2, dtype=torch.bfloat16, device=dev).view(out_f, in_f // 2)
    idx = torch.empty(ib.value, dtype=torch.uint8, device=dev)
    bad = torch.zeros(1, dtype=torch.int64, device=dev)
    L.check(L.lib().sf_pack_2to4(L.ptr(weight), L.dtype_code(weight), L.ptr(mask), L.dtype_code(mask), out_f, in_f,
                                 L.ptr(vals), L.ptr(idx), L.ptr(bad), L.stream(dev)), "sf_pack_2to4")
    nbad = int(bad.item())
    if nbad:
        raise ValueError(f"pack_2to4: {nbad} groups of 4 keep more than two columns; the mask is not 2:4")
    return Packed2to4(vals, idx, out_f, in_f)


@torch.no_grad()
def unpack_2to4(p: Packed2to4, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """The dense [out, in] weight (zeros at the pruned columns)."""
    dev = L.require_device(p.vals, p.idx)
    W = torch.empty(p.out_features, p.in_features, dtype=dtype, device=dev)
    L.check(L.lib().sf_unpack_2to4(L.ptr(p.vals), L.ptr(p.idx), p.out_features, p.in_features, L.ptr(W),
                                   L.dtype_code(W), L.stream(dev)), "sf_unpack_2to4")
    return W


def gemm_2to4(x: torch.Tensor, p: Packed2to4, bias: torch.Tensor | None = None,
              out_dtype: torch.dtype | None = None) -> torch.Tensor:
    """y [tokens, out] = x [tokens, in] (bf16) . W^T (+ bias) with W packed."""
    dev = L.require_device(x, p.vals, p.idx, bias)
    if x.dim() != 2 or x.shape[1] != p.in_features or x.dtype != torch.bfloat16:
        raise ValueError(f"gemm_2to4: x must be bf16 [tokens, {p.in_features}]")
    if bias is not None and bias.shape != (p.out_features,):
        raise ValueError("gemm_2to4: bias must be [out_features]")
    y = torch.empty(x.shape[0], p.out_features, dtype=out_dtype or x.dtype, device=dev)
    with _prof.region("sf_gemm_2to4", 2.0 * x.shape[0] * p.in_features * p.out_features, "FLOP", dev):
        L.check(L.lib().sf_gemm_2to4(L.ptr(x), x.shape[1], x.shape[0], L.ptr(p.vals), L.ptr(p.idx), p.out_features,
                                     p.in_features, L.ptr(bias), L.dtype_code(bias) if bias is not None else L.DT_F32,
                                     L.ptr(y), L.dtype_code(y), p.out_features, L.stream(dev)), "sf_gemm_2to4")
    return y


def _sparse_layers(model):
    return [(n, m) for n, m in model.named_modules() if isinstance(m, SparseLinear)]


@torch.no_grad()
def finalize_sparse_model(model) -> int:
    """Harden every SparseLinear at the end of training (legacy/main_llama.py:2499-2568): mask <- hard
    projection of the soft mask, frozen flags <- max(frozen, hard), weight <- weight * mask, mask
    updates off, forward switched to the finalized (hard) mask.  Returns the number of layers."""
    from .utils import get_raw_model

    n = 0
    for name, module in _sparse_layers(get_raw_model(model)):
        try:
            hard = module._hard_mask_from_soft(module.mask).detach()
            ff = hard.to(dtype=torch.uint8).to(dtype=module.frozen_mask_flags.dtype)
            module.mask.copy_(hard)
            module.frozen_mask_flags.data = torch.maximum(module.frozen_mask_flags.data, ff)
            module.weight.data.copy_(LIN.apply_mask(module.weight.data.contiguous(), module.mask.contiguous()))
            module.change_mask = False
            module._hardening_finalized = True
            n += 1
        except Exception as e:  # the reference warns and goes on with the next layer
            print(f"[Finalization] WARNING: failed to finalize module {name}: {e}")
    return n


@torch.no_grad()
def optimize_sparse_model_for_inference(model, use_slorb: bool = False):
    """Fold the hard mask into the weights and switch to dense_forward (legacy/eval_wiki_ppl.py:548-651);
    with SLoRB the layers stay in sparse_forward with the mask made hard."""
    can_dense = not use_slorb
    optimized = total = 0
    for _, module in _sparse_layers(model):
        total += 1
        if getattr(module, "mask", None) is None:
            optimized += 1
            continue
        soft = module.mask
        binary = bool(torch.all((soft == 0) | (soft == 1)).item())
        hard = soft.to(dtype=module.weight.dtype) if binary else \
            module._hard_mask_from_soft(soft).to(dtype=module.weight.dtype)
        already = False
        if can_dense and getattr(module, "_hardening_finalized", False):
            w0 = (module.weight.data == 0).float().mean().item()
            m0 = (hard == 0).float().mean().item()
            if w0 >= m0 - 1e-4:
                already = True
                module.mode = "dense_forward"
                module._inference_optimized = True
        if not already:
            if can_dense:
                module.weight.data.copy_(LIN.apply_mask(module.weight.data.contiguous(), hard.contiguous()))
                module.mode = "dense_forward"
            else:
                module.mask.detach().copy_(hard)  # (bumps the mask's version: a cached projection is rebuilt)
            module._inference_optimized = True
        optimized += 1
    if total:
        print(f"[INFO] Optimized {optimized}/{total} SparseLinear layers for inference")
    return model


class SparseLinear24(torch.nn.Module):
    """Forward-only layer over a packed 2:4 weight: y = x . W_hard^T + b (+ SLoRB (x P^T) S^T)."""

    def __init__(self, packed: Packed2to4, bias: torch.Tensor | None = None, x_proj: torch.Tensor | None = None,
                 slorb_weight: torch.Tensor | None = None):
        super().__init__()
        self.in_features, self.out_features = packed.in_features, packed.out_features
        self.register_buffer("vals", packed.vals)
        self.register_buffer("idx", packed.idx)
        self.bias = None if bias is None else torch.nn.Parameter(bias.detach().clone(), requires_grad=False)
        self.x_proj = None if x_proj is None else x_proj.detach().clone()
        self.slorb_weight = None if slorb_weight is None else slorb_weight.detach().clone()

    @property
    def packed(self) -> Packed2to4:
        return Packed2to4(self.vals, self.idx, self.out_features, self.in_features)

    @classmethod
    @torch.no_grad()
    def from_sparse_linear(cls, module: SparseLinear) -> "SparseLinear24":
        """Pack a finalized (or any 2:4-hard) SparseLinear: W * hard(mask), plus its SLoRB factors."""
        hard = module._hard_mask_from_soft(module.mask).contiguous()
        W = module.weight.detach().to(torch.bfloat16).contiguous()
        slorb = bool(getattr(module, "SLoRB", False)) and hasattr(module, "x_proj")
        return cls(pack_2to4(W, hard), module.bias, module.x_proj if slorb else None,
                   module.SLoRB_Weight if slorb else None)

    @torch.no_grad()
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).to(torch.bfloat16).contiguous()
        b = None if self.bias is None else self.bias.detach().contiguous()
        if self.x_proj is None:
            y = gemm_2to4(x2, self.packed, b)
        else:
            # the SLoRB term as the product's second (dense) K segment: x W^T + z S^T + b rounded once,
            # as the masked layer rounds it; the rank is zero-padded to the segment's multiple of 8
            P = self.x_proj.to(device=x2.device, dtype=torch.bfloat16).contiguous()
            S = self.slorb_weight.to(device=x2.device, dtype=torch.bfloat16).contiguous()
            z = LIN.mm_nt(x2, P)
            pad = -z.shape[1] % 8
            if pad:
                z = torch.nn.functional.pad(z, (0, pad))
                S = torch.nn.functional.pad(S, (0, pad))
            y = LIN.gemm_2to4(x2, self.vals, self.idx, self.out_features, z=z, S=S, bias=b)
        return y.reshape(*shape[:-1], self.out_features)


@torch.no_grad()
def convert_model_to_2to4(model, strict: bool = False) -> int:
    """Replace every SparseLinear whose hard mask is 2:4 (nm_2_4 or structured N=2, M=4) and whose shape
    packs (out % 32 == 0, in % 64 == 0) by a SparseLinear24.  strict: raise on a layer that does not
    pack instead of leaving it.  Returns the number of layers replaced."""
    replaced = 0
    for name, module in list(_sparse_layers(model)):
        t = module._effective_hard_type()
        two_four = t == "nm_2_4" or (t == "structured" and int(module.N) == 2 and int(module.M) == 4)
        fits = module.out_features % 32 == 0 and module.in_features % 64 == 0
        if not (two_four and fits):
            if strict:
                raise ValueError(f"{name}: hard type {t} / shape {module.out_features} x {module.in_features} "
                                 "does not pack as 2:4")
            continue
        new = SparseLinear24.from_sparse_linear(module)
        parent = model
        *path, leaf = name.split(".")
        for p in path:
            parent = getattr(parent, p)
        setattr(parent, leaf, new)
        replaced += 1
    return replaced
