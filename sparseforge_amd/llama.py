"""A LLaMA-architecture decoder for the end-to-end sparse retraining step.

The reference retrains HuggingFace's LlamaForCausalLM with every nn.Linear
inside the decoder stack (`model.model`) swapped for SparseLinear, keeping
the embedding, the final norm and lm_head dense (legacy/model_llama.py:18-57),
and it needs eager attention so that Hutchinson's double backward works
(legacy/model_llama.py:108-123, legacy/utils.py:796-801).  This module builds
that architecture directly, with the drop-in SparseLinear for the student's
projections and plain nn.Linear for the dense teacher:

    h = embed(tokens)
    per layer:  h = h + o(attn(rope(q(n1(h))), rope(k(n1(h))), v(n1(h))))
                h = h + down(silu(gate(n2(h))) * up(n2(h)))
    logits = lm_head(norm(h))

* RMSNorm: x * rsqrt(mean(x^2) + eps) in float32, scaled by a learned
  weight after the cast back to the input dtype.
* Rotary embedding: the half-split form (pairs (i, i + d/2) rotate by
  position * theta^(-2i/d)); the tables are computed in float32 and cast to
  the activations' dtype, as HuggingFace's LlamaRotaryEmbedding does.
* Attention: causal softmax attention written with differentiable torch ops
  (the Hessian-vector product differentiates it twice).  bf16 activations
  follow HuggingFace's eager attention operation for operation: rotation in
  bf16, bf16 products q k^T and p v (float32 accumulation), the 1/sqrt(D)
  scale, the causal mask, the softmax in float32 cast back to bf16.  float32
  activations run the same sequence in float32.  Every batched product goes
  through _BMM, whose operands (in the forward and in every derivative) are
  made contiguous first: no batched bf16 product sees a transposed view.
* forward(idx, targets) returns (logits, loss, None) like the reference's
  LlamaSparse.forward (legacy/model_llama.py:59-85): loss is the
  cross-entropy of the logits against already shifted targets,
  ignore_index=-1.
"""
from __future__ import annotations

import dataclasses
import math
from dataclasses import dataclass

import torch
import torch.nn as nn
from torch.nn import functional as F

from . import _lib as L
from . import profiling as _prof
from .sparse_modeling import SparseLinear, SparseLinearConfig


@dataclass
class LlamaShape:
    """Architecture of the decoder (the fields of a LLaMA config this build uses)."""

    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 22
    num_attention_heads: int = 32
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    output_hidden_state: bool = False  # set by Distill_Model

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    """HuggingFace's LlamaRMSNorm: weight * (x32 * rsqrt(mean(x32^2) + eps)).to(x dtype).  On the GPU (x and
    weight of one dtype, bf16 or f32, rows of at most 4096 columns, a multiple of 8) each pass is one device
    kernel (sf_rmsnorm_*): forward, backward and the backward's own backward that the Hutchinson probe takes;
    elsewhere torch's ops."""

    def __init__(self, dim: int, eps: float, device=None, dtype=None):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim, device=device, dtype=dtype))
        self.eps = eps

    def forward(self, x):
        if _norm_on_device(x, self.weight):
            x2 = x.reshape(-1, x.shape[-1]).contiguous()
            if x2.data_ptr() % 16 == 0:  # the kernels' vector accesses
                return _RMSNorm.apply(x2, self.weight, self.eps).view(x.shape)
        return rms_norm_torch(x, self.weight, self.eps)


def rms_norm_torch(x, weight, eps):
    """The torch form (the CPU path; on the GPU the form the device passes are checked against)."""
    xf = x.float()
    xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
    return weight * xf.to(x.dtype)


def _norm_on_device(x: torch.Tensor, w: torch.Tensor) -> bool:
    D = x.shape[-1]
    return (x.is_cuda and x.dtype in (torch.bfloat16, torch.float32) and w.dtype == x.dtype and w.dim() == 1
            and w.shape[0] == D and D % 8 == 0 and D <= 4096 and w.is_contiguous() and w.data_ptr() % 16 == 0)


def _norm_ws(rows: int, cols: int, dev) -> torch.Tensor:
    return torch.empty(max(int(L.lib().sf_rmsnorm_workspace_size(rows, cols)), 16), dtype=torch.uint8, device=dev)


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """A gradient made contiguous at a 16-byte aligned address (a fresh copy when a view starts elsewhere)."""
    t = t.contiguous()
    return t if t.data_ptr() % 16 == 0 else t.clone()


class _RMSNorm(torch.autograd.Function):
    """RMSNorm over the rows of x2 [rows, D] (sf_rmsnorm_forward); its backward is _RMSNormGrad, whose backward
    (sf_rmsnorm_double_backward) is what the Hutchinson Hessian-vector product differentiates."""

    @staticmethod
    def forward(ctx, x2, w, eps):  # x2: contiguous, 16-byte aligned (saved as the graph's own input)
        dev = L.require_device(x2, w)
        rows, D = x2.shape
        y = torch.empty_like(x2)
        rstd = torch.empty(rows, dtype=torch.float32, device=dev)
        with _prof.region("sf_rmsnorm_forward", 2 * x2.numel() * x2.element_size(), "B", dev):
            L.check(L.lib().sf_rmsnorm_forward(L.ptr(x2), L.ptr(w), L.dtype_code(x2), rows, D, float(eps), L.ptr(y),
                                               L.ptr(rstd), L.stream(dev)), "sf_rmsnorm_forward")
        ctx.save_for_backward(x2, w, rstd)
        return y

    @staticmethod
    def backward(ctx, gy):
        x2, w, rstd = ctx.saved_tensors
        gx, gw = _RMSNormGrad.apply(gy.to(x2.dtype), x2, w, rstd)
        return gx, gw, None


class _RMSNormGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gy, x2, w, rstd):
        dev = L.require_device(gy, x2, w, rstd)
        gy = _aligned(gy)
        rows, D = x2.shape
        gx, gw = torch.empty_like(x2), torch.empty_like(w)
        ws = _norm_ws(rows, D, dev)
        with _prof.region("sf_rmsnorm_backward", 3 * x2.numel() * x2.element_size(), "B", dev):
            L.check(L.lib().sf_rmsnorm_backward(L.ptr(x2), L.ptr(w), L.ptr(gy), L.ptr(rstd), L.dtype_code(x2), rows,
                                                D, L.ptr(gx), L.ptr(gw), L.ptr(ws), ws.numel(), L.stream(dev)),
                    "sf_rmsnorm_backward")
        ctx.save_for_backward(gy, x2, w, rstd)
        return gx, gw

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx, ggw):
        gy, x2, w, rstd = ctx.saved_tensors
        dev = x2.device
        rows, D = x2.shape
        ggx = _aligned(ggx.to(x2.dtype)) if ggx is not None else torch.zeros_like(x2)
        ggw = _aligned(ggw.to(w.dtype)) if ggw is not None else None
        ggy, gx2, gw2 = torch.empty_like(x2), torch.empty_like(x2), torch.empty_like(w)
        ws = _norm_ws(rows, D, dev)
        with _prof.region("sf_rmsnorm_double_backward", 5 * x2.numel() * x2.element_size(), "B", dev):
            L.check(L.lib().sf_rmsnorm_double_backward(L.ptr(x2), L.ptr(w), L.ptr(gy), L.ptr(rstd), L.ptr(ggx),
                                                       L.ptr(ggw) if ggw is not None else None, L.dtype_code(x2),
                                                       rows, D, L.ptr(ggy), L.ptr(gx2), L.ptr(gw2), L.ptr(ws),
                                                       ws.numel(), L.stream(dev)), "sf_rmsnorm_double_backward")
        return ggy, gx2, gw2, None


def rotary_tables(seq: int, head_dim: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """cos, sin [seq, head_dim] (float32) of the half-split rotary embedding."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    ang = torch.arange(seq, device=device, dtype=torch.float32)[:, None] * inv[None, :]
    ang = torch.cat([ang, ang], dim=-1)
    return ang.cos(), ang.sin()


def _rotate(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x * cos + rotate_half(x) * sin with rotate_half(x) = cat(-x2, x1) (the half-split rotation), written as
    roll(x, half) * cat(-sin1, sin2): (-a) * s and a * (-s) round to the same value, so the result is bit for bit
    the cat form's, and the derivatives are a roll and products instead of zero-filled slice gradients."""
    half = x.shape[-1] // 2
    signed_sin = torch.cat([-sin[..., :half], sin[..., half:]], dim=-1)
    return x * cos + torch.roll(x, shifts=half, dims=-1) * signed_sin


def _contig3(t: torch.Tensor) -> torch.Tensor:
    """A [batch, m, n] operand made contiguous; the transposed view of a contiguous tensor (what the products'
    derivatives pass) is transposed by one tiled pass on the GPU (sf_transpose_batched) instead of torch's
    strided copy."""
    if t.is_contiguous():
        return t
    src = t.transpose(1, 2)
    if t.is_cuda and t.dim() == 3 and src.is_contiguous() and t.element_size() in (2, 4) \
            and src.data_ptr() % 16 == 0:
        out = torch.empty(t.shape, dtype=t.dtype, device=t.device)
        dev = t.device
        with _prof.region("sf_transpose_batched", 2 * t.numel() * t.element_size(), "B", dev):
            L.check(L.lib().sf_transpose_batched(L.ptr(src), t.element_size(), src.shape[0], src.shape[1],
                                                 src.shape[2], L.ptr(out), L.stream(dev)), "sf_transpose_batched")
        return out
    return t.contiguous()


class _BMM(torch.autograd.Function):
    """torch.bmm(a, b) (+ a constant bias, broadcast over the batch) differentiable any number of times,
    with contiguous operands in every product.

    The derivatives are products of the same kind, so the forward, the backward and the Hutchinson
    double backward all multiply contiguous tensors.  Each derivative takes the form whose transposed
    copies are smaller: grad_a = g b^T copies b^T, (b g^T)^T copies g^T and the result; grad_b = a^T g
    copies a^T, (g^T a)^T copies g^T and the result.  For p v (p [S, S], v [S, D]) that keeps the
    value gradient from transposing the S x S probabilities."""

    @staticmethod
    def forward(ctx, a, b, bias=None):
        ctx.save_for_backward(a, b)
        if bias is not None:
            return torch.baddbmm(bias, _contig3(a), _contig3(b))
        return torch.bmm(_contig3(a), _contig3(b))

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        g = g.to(a.dtype)
        n = lambda t: t.shape[1] * t.shape[2]  # noqa: E731
        ga = gb = None
        if ctx.needs_input_grad[0]:
            if n(b) <= n(g) + n(a):
                ga = _BMM.apply(g, b.transpose(1, 2))
            else:
                ga = _BMM.apply(b, g.transpose(1, 2)).transpose(1, 2)
        if ctx.needs_input_grad[1]:
            if n(a) <= n(g) + n(b):
                gb = _BMM.apply(a.transpose(1, 2), g)
            else:
                gb = _BMM.apply(g.transpose(1, 2), a).transpose(1, 2)
        return ga, gb, None


# Causal structure of the attention's S x S operands: OUT_LOWER (only the product's lower triangle is ever read:
# the scores, the gradient of p), A_LOWER / B_LOWER (that operand is zero above its diagonal: p, the scores'
# gradient).  Products of these kinds skip the blocks the triangle leaves out.
OUT_LOWER, A_LOWER, B_LOWER = 1, 2, 3
CAUSAL_BLOCKS = 4  # row (or column) blocks of a causal product; S below 512 runs as one full product


def _causal_blocks(S: int):
    nb = CAUSAL_BLOCKS if S >= 512 else 1
    step = (S + nb - 1) // nb
    return [(i, min(i + step, S)) for i in range(0, S, step)]


def _causal_product(a: torch.Tensor, b: torch.Tensor, mode: int) -> torch.Tensor:
    """a @ b ([BH, M, K] x [BH, K, N]) with one S x S side lower-triangular, as row / column blocks of
    torch.bmm on views (each block's product covers the triangle up to the block's end):
    OUT_LOWER: c[r0:r1, :r1] = a[r0:r1] b[:, :r1]  (c's entries above the blocks stay unwritten: never read)
    A_LOWER:   c[r0:r1] = a[r0:r1, :r1] b[:r1]      (a is zero past column r1 in those rows)
    B_LOWER:   c[:, c0:c1] = a[:, c0:] b[c0:, c0:c1] (b is zero above row c0 in those columns)."""
    a, b = _contig3(a), _contig3(b)
    BH, M, K = a.shape
    N = b.shape[2]
    c = torch.empty(BH, M, N, dtype=a.dtype, device=a.device)
    if mode == OUT_LOWER:
        for r0, r1 in _causal_blocks(M):
            torch.bmm(a[:, r0:r1], b[:, :, :r1], out=c[:, r0:r1, :r1])
    elif mode == A_LOWER:
        for r0, r1 in _causal_blocks(M):
            torch.bmm(a[:, r0:r1, :r1], b[:, :r1], out=c[:, r0:r1])
    else:
        for c0, c1 in _causal_blocks(N):
            torch.bmm(a[:, :, c0:], b[:, c0:, c0:c1], out=c[:, :, c0:c1])
    return c


class _CBMM(torch.autograd.Function):
    """A causal product (_causal_product) differentiable any number of times: the derivatives of each kind
    are products of the kinds again (the S x S operand always untransposed), e.g. for OUT_LOWER the gradient
    g is zero above its diagonal (it comes from the causal softmax passes), so grad_a = g b^T is A_LOWER and
    grad_b = a^T g is B_LOWER."""

    @staticmethod
    def forward(ctx, a, b, mode: int):
        ctx.save_for_backward(a, b)
        ctx.mode = mode
        return _causal_product(a, b, mode)

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        mode = ctx.mode
        g = g.to(a.dtype)
        ga = gb = None
        if mode == OUT_LOWER:
            if ctx.needs_input_grad[0]:
                ga = _CBMM.apply(g, b.transpose(1, 2), A_LOWER)
            if ctx.needs_input_grad[1]:
                gb = _CBMM.apply(a.transpose(1, 2), g, B_LOWER)
        elif mode == A_LOWER:
            if ctx.needs_input_grad[0]:
                ga = _CBMM.apply(g, b.transpose(1, 2), OUT_LOWER)
            if ctx.needs_input_grad[1]:
                gb = _CBMM.apply(g.transpose(1, 2), a, B_LOWER).transpose(1, 2)
        else:
            if ctx.needs_input_grad[0]:
                ga = _CBMM.apply(b, g.transpose(1, 2), A_LOWER).transpose(1, 2)
            if ctx.needs_input_grad[1]:
                gb = _CBMM.apply(a.transpose(1, 2), g, OUT_LOWER)
        return ga, gb, None


def _softmax_launch(name: str, fn, nbytes: int, dev, *args) -> None:
    with _prof.region(name, nbytes, "B", dev):
        L.check(fn(*args, L.stream(dev)), name)


class _CausalSoftmax(torch.autograd.Function):
    """p = softmax(scores, dim=-1, dtype=float32).to(scores.dtype) of causal [B H, S, S] scores (the masked
    entries -inf, their probability 0) on the device (sf_softmax_rows).  Its backward is a Function of its
    own (_CausalSoftmaxGrad), so the Hutchinson Hessian-vector product differentiates it once more, as it
    differentiates the reference's torch ops.  Only the scores are kept: each pass recomputes y from them."""

    @staticmethod
    def forward(ctx, x):
        dev = L.require_device(x)
        rows, cols = x.numel() // x.shape[-1], x.shape[-1]
        p = torch.empty_like(x)
        _softmax_launch("sf_softmax_rows", L.lib().sf_softmax_rows, x.numel() * x.element_size(), dev,
                        L.ptr(x), L.dtype_code(x), rows, cols, 1, L.ptr(p))
        ctx.save_for_backward(x)
        return p

    @staticmethod
    def backward(ctx, gp):
        x, = ctx.saved_tensors
        return _CausalSoftmaxGrad.apply(gp.to(x.dtype).contiguous(), x)


class _CausalSoftmaxGrad(torch.autograd.Function):
    """grad_x = (y (g - sum(g y))).to(x dtype), g = grad_p in float32 (sf_softmax_rows_backward), and its
    backward with respect to grad_p and the scores (sf_softmax_rows_double_backward)."""

    @staticmethod
    def forward(ctx, gp, x):
        dev = L.require_device(gp, x)
        rows, cols = x.numel() // x.shape[-1], x.shape[-1]
        gx = torch.empty_like(x)
        _softmax_launch("sf_softmax_rows_backward", L.lib().sf_softmax_rows_backward,
                        x.numel() * x.element_size(), dev, L.ptr(x), L.ptr(gp), L.dtype_code(x), rows, cols, 1,
                        L.ptr(gx))
        ctx.save_for_backward(gp, x)
        return gx

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggx):
        gp, x = ctx.saved_tensors
        dev = x.device
        ggx = ggx.to(x.dtype).contiguous()
        rows, cols = x.numel() // x.shape[-1], x.shape[-1]
        ggp, gx2 = torch.empty_like(x), torch.empty_like(x)
        _softmax_launch("sf_softmax_rows_double_backward", L.lib().sf_softmax_rows_double_backward,
                        x.numel() * x.element_size(), dev, L.ptr(x), L.ptr(gp), L.ptr(ggx), L.dtype_code(x), rows,
                        cols, 1, L.ptr(ggp), L.ptr(gx2))
        return ggp, gx2


def causal_softmax(scores: torch.Tensor) -> torch.Tensor:
    """softmax(scores, dim=-1, dtype=float32).to(scores.dtype) of causal scores [.., S, S] whose masked entries
    are -inf: the device kernels on a GPU (S <= 4096), torch's ops on the CPU."""
    if scores.is_cuda:
        return _CausalSoftmax.apply(scores.contiguous())
    return torch.softmax(scores, dim=-1, dtype=torch.float32).to(scores.dtype)


def _heads_launch(name: str, fn, src: torch.Tensor, dst: torch.Tensor, B: int, S: int, H: int, D: int,
                  cos: torch.Tensor, sin: torch.Tensor, rotate: bool, transposed: bool, scale: float) -> None:
    dev = L.require_device(src, dst)
    with _prof.region(name, 2 * src.numel() * src.element_size(), "B", dev):
        L.check(fn(L.ptr(src), L.dtype_code(src), B, S, H, D, L.ptr(cos), L.ptr(sin), int(rotate), int(transposed),
                   float(scale), L.ptr(dst), L.stream(dev)), name)


def _head_major(g: torch.Tensor, transposed: bool) -> tuple[torch.Tensor, bool]:
    """A head-major gradient as the kernels read it: contiguous in the expected layout, or the transposed view of
    a contiguous tensor of the other layout (the flag flips, no copy); otherwise a contiguous copy."""
    if g.is_contiguous():
        return g, transposed
    if g.transpose(1, 2).is_contiguous():
        return g.transpose(1, 2), not transposed
    return g.contiguous(), transposed


class _ToHeads(torch.autograd.Function):
    """x [B, S, H, D] (a projection's rows) -> scale * rot(x) (or scale * x) as [B H, S, D], or [B H, D, S] when
    transposed (sf_to_heads): the transpose to per-head operands and the rotary embedding of HuggingFace's eager
    attention in one pass.  Its backward is _FromHeads (the adjoint), whose backward is this map again."""

    @staticmethod
    def forward(ctx, x, cos, sin, rotate: bool, transposed: bool, scale: float):
        B, S, H, D = x.shape
        x = x.contiguous()
        y = torch.empty((B * H, D, S) if transposed else (B * H, S, D), dtype=x.dtype, device=x.device)
        _heads_launch("sf_to_heads", L.lib().sf_to_heads, x, y, B, S, H, D, cos, sin, rotate, transposed, scale)
        ctx.cfg = (B, S, H, D, rotate, transposed, scale)
        ctx.save_for_backward(cos, sin)
        return y

    @staticmethod
    def backward(ctx, g):
        cos, sin = ctx.saved_tensors
        B, S, H, D, rotate, transposed, scale = ctx.cfg
        return _FromHeads.apply(g, cos, sin, (B, S, H, D), rotate, transposed, scale), None, None, None, None, None


class _FromHeads(torch.autograd.Function):
    """The adjoint of _ToHeads (sf_from_heads): g [B H, S, D] (or [B H, D, S] when transposed) ->
    rot^T(scale * g) as [B, S, H, D]; without rotation and scale it is the per-head output's way back to rows."""

    @staticmethod
    def forward(ctx, g, cos, sin, shape, rotate: bool, transposed: bool, scale: float):
        B, S, H, D = shape
        src, tr = _head_major(g, transposed)
        x = torch.empty((B, S, H, D), dtype=g.dtype, device=g.device)
        _heads_launch("sf_from_heads", L.lib().sf_from_heads, src, x, B, S, H, D, cos, sin, rotate, tr, scale)
        ctx.cfg = (rotate, transposed, scale)
        ctx.save_for_backward(cos, sin)
        return x

    @staticmethod
    def backward(ctx, gx):
        cos, sin = ctx.saved_tensors
        rotate, transposed, scale = ctx.cfg
        return _ToHeads.apply(gx, cos, sin, rotate, transposed, scale), None, None, None, None, None, None


_CAUSAL_BIAS: dict = {}


def causal_bias(S: int, device, dtype=torch.float32) -> torch.Tensor:
    """[1, S, S]: 0 on and below the diagonal, -inf above (cached per size, device and dtype)."""
    key = (S, str(device), dtype)
    if key not in _CAUSAL_BIAS:
        _CAUSAL_BIAS[key] = torch.full((S, S), float("-inf"), device=device, dtype=dtype).triu_(1)[None]
    return _CAUSAL_BIAS[key]


def causal_attention(q, k, v, cos, sin) -> torch.Tensor:
    """q, k, v [B, S, H, D] -> [B, S, H * D] in q's dtype, causal.

    The operation sequence of HuggingFace's eager attention, which the reference retrains with
    (legacy/model_llama.py:39-55, eager_attention_forward): rotary tables cast to q's dtype and the
    rotation in it; s = (q k^T) * D^-0.5; s + causal mask; softmax in float32, cast to q's dtype;
    p v.  When D^-0.5 is a power of two (D = 64, 256, ...) the scale goes into q before the product,
    which gives the same bits ((2^e q) k^T = 2^e (q k^T) exactly); otherwise the scores are scaled after
    it.  The masked positions get -inf where the reference adds the dtype's lowest value: either way
    their probability is exactly 0."""
    if q.is_cuda:
        return _causal_attention_device(q, k, v, cos, sin)
    return _causal_attention_torch(q, k, v, cos, sin)


def _causal_attention_torch(q, k, v, cos, sin) -> torch.Tensor:
    """causal_attention with torch's layout ops (the CPU path; on the GPU the reference form the device path is
    checked against)."""
    B, S, H, D = q.shape
    dt = q.dtype
    with torch.autocast(q.device.type, enabled=False):
        c, s_ = cos.to(dt), sin.to(dt)
        qh = _rotate(q.transpose(1, 2), c, s_)                                   # [B, H, S, D]
        kh = _rotate(k.transpose(1, 2), c, s_)
        scale = D ** -0.5
        exact = math.frexp(scale)[0] == 0.5                                       # a power of two
        if exact:
            qh = qh * scale
        qh = qh.reshape(B * H, S, D)
        kt = kh.transpose(-2, -1).reshape(B * H, D, S)
        if exact:
            # the mask rides in the product: rnd(qk + 0) = rnd(qk) and qk + -inf = -inf, the bits of the
            # product followed by the masked add
            scores = _BMM.apply(qh, kt, causal_bias(S, q.device, dt))              # [B H, S, S]
        else:
            scores = _BMM.apply(qh, kt) * scale + causal_bias(S, q.device, dt)
        p = causal_softmax(scores)
        out = _BMM.apply(p, v.transpose(1, 2).reshape(B * H, S, D))              # [B H, S, D]
    return out.view(B, H, S, D).transpose(1, 2).reshape(B, S, H * D)


def _causal_attention_device(q, k, v, cos, sin) -> torch.Tensor:
    """causal_attention on the GPU: the same operations, with the transposes to per-head operands, the rotary
    embedding and the way back to rows in sf_to_heads / sf_from_heads passes (no strided copies)."""
    B, S, H, D = q.shape
    with torch.autocast(q.device.type, enabled=False):
        scale = D ** -0.5
        exact = math.frexp(scale)[0] == 0.5  # a power of two: it rides in q, bit for bit the scaled product
        cos, sin = cos.float().contiguous(), sin.float().contiguous()
        qh = _ToHeads.apply(q, cos, sin, True, False, scale if exact else 1.0)   # [B H, S, D]
        kt = _ToHeads.apply(k, cos, sin, True, True, 1.0)                        # [B H, D, S]
        # No mask tensor: the causal softmax kernels read only columns 0..i of row i and give the rest
        # probability 0 (zero gradient), which is what adding -inf there does; on the kept entries the
        # mask adds 0, so the scores' bits there are the product's either way.
        scores = _CBMM.apply(qh, kt, OUT_LOWER)
        if not exact:
            scores = scores * scale
        p = causal_softmax(scores)
        vh = _ToHeads.apply(v, cos, sin, False, False, 1.0)                      # [B H, S, D]
        out = _CBMM.apply(p, vh, A_LOWER)                                        # [B H, S, D]
        return _FromHeads.apply(out, cos, sin, (B, S, H, D), False, False, 1.0).view(B, S, H * D)


def swiglu(g: torch.Tensor, u: torch.Tensor) -> torch.Tensor:
    """silu(g) * u, HuggingFace LlamaMLP's gate: one device pass each way on the GPU (g and u of one dtype, bf16 or
    f32, same shape, contiguous, 16-byte aligned, a multiple of 8 elements), torch's ops elsewhere."""
    if (g.is_cuda and g.dtype in (torch.bfloat16, torch.float32) and u.dtype == g.dtype and u.shape == g.shape
            and g.is_contiguous() and u.is_contiguous() and g.numel() % 8 == 0 and g.data_ptr() % 16 == 0
            and u.data_ptr() % 16 == 0):
        return _SwiGLU.apply(g, u)
    return F.silu(g) * u


def _sg_launch(name: str, nbytes: int, dev, *args) -> None:
    with _prof.region(name, nbytes, "B", dev):
        L.check(getattr(L.lib(), name)(*args, L.stream(dev)), name)


class _SwiGLU(torch.autograd.Function):
    """silu(g) * u (sf_swiglu_forward); its backward is _SwiGLUGrad, whose backward (sf_swiglu_double_backward)
    the Hutchinson Hessian-vector product takes."""

    @staticmethod
    def forward(ctx, g, u):
        dev = L.require_device(g, u)
        y = torch.empty_like(g)
        _sg_launch("sf_swiglu_forward", 3 * g.numel() * g.element_size(), dev, L.ptr(g), L.ptr(u), L.dtype_code(g),
                   g.numel(), L.ptr(y))
        ctx.save_for_backward(g, u)
        return y

    @staticmethod
    def backward(ctx, gy):
        g, u = ctx.saved_tensors
        return _SwiGLUGrad.apply(_aligned(gy.to(g.dtype)), g, u)


class _SwiGLUGrad(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gy, g, u):
        dev = L.require_device(gy, g, u)
        gg, gu = torch.empty_like(g), torch.empty_like(g)
        _sg_launch("sf_swiglu_backward", 5 * g.numel() * g.element_size(), dev, L.ptr(g), L.ptr(u), L.ptr(gy),
                   L.dtype_code(g), g.numel(), L.ptr(gg), L.ptr(gu))
        ctx.save_for_backward(gy, g, u)
        return gg, gu

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, ggg, ggu):
        gy, g, u = ctx.saved_tensors
        dev = g.device
        ggg = _aligned(ggg.to(g.dtype)) if ggg is not None else None
        ggu = _aligned(ggu.to(g.dtype)) if ggu is not None else None
        dgy, dg, du = torch.empty_like(g), torch.empty_like(g), torch.empty_like(g)
        _sg_launch("sf_swiglu_double_backward", 8 * g.numel() * g.element_size(), dev, L.ptr(g), L.ptr(u),
                   L.ptr(gy), L.ptr(ggg), L.ptr(ggu), L.dtype_code(g), g.numel(), L.ptr(dgy), L.ptr(dg), L.ptr(du))
        return dgy, dg, du


class DecoderLayer(nn.Module):
    def __init__(self, shape: LlamaShape, make_linear, device=None, dtype=None):
        super().__init__()
        h, f = shape.hidden_size, shape.intermediate_size
        self.input_layernorm = RMSNorm(h, shape.rms_norm_eps, device=device, dtype=dtype)
        self.post_attention_layernorm = RMSNorm(h, shape.rms_norm_eps, device=device, dtype=dtype)
        self.self_attn = nn.Module()
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self.self_attn, name, make_linear(h, h))
        self.mlp = nn.Module()
        self.mlp.gate_proj = make_linear(h, f)
        self.mlp.up_proj = make_linear(h, f)
        self.mlp.down_proj = make_linear(f, h)
        self.heads = shape.num_attention_heads

    def forward(self, x, cos, sin):
        B, S, Hd = x.shape
        a = self.self_attn
        n = self.input_layernorm(x)
        q = a.q_proj(n).view(B, S, self.heads, -1)
        k = a.k_proj(n).view(B, S, self.heads, -1)
        v = a.v_proj(n).view(B, S, self.heads, -1)
        x = x + a.o_proj(causal_attention(q, k, v, cos, sin))
        n = self.post_attention_layernorm(x)
        m = self.mlp
        return x + m.down_proj(swiglu(m.gate_proj(n), m.up_proj(n)))


class LlamaDecoder(nn.Module):
    """Student (SparseLinear projections, `sparse_config` given) or dense teacher (nn.Linear)."""

    def __init__(self, shape: LlamaShape, sparse_config: SparseLinearConfig | None = None, slorb_rank: int = 64,
                 device=None, dtype=torch.bfloat16):
        super().__init__()
        self.config = dataclasses.replace(shape)

        def make_linear(fin, fout):
            if sparse_config is None:
                return nn.Linear(fin, fout, bias=False, device=device, dtype=dtype)
            cfg = sparse_config
            if cfg.SLoRB:
                if fin % slorb_rank:
                    raise ValueError(f"in_features {fin} is not a multiple of the SLoRB rank {slorb_rank}")
                cfg = dataclasses.replace(cfg, SLoRB_k=fin // slorb_rank)  # rank = in / k
            for key, val in vars(sparse_config).items():  # attributes set outside the dataclass fields
                if not hasattr(cfg, key):
                    setattr(cfg, key, val)
            return SparseLinear(fin, fout, sparselinear_config=cfg, bias=False, device=device, dtype=dtype)

        self.embed_tokens = nn.Embedding(shape.vocab_size, shape.hidden_size, device=device, dtype=dtype)
        self.layers = nn.ModuleList(DecoderLayer(shape, make_linear, device, dtype)
                                    for _ in range(shape.num_hidden_layers))
        self.norm = RMSNorm(shape.hidden_size, shape.rms_norm_eps, device=device, dtype=dtype)
        self.lm_head = nn.Linear(shape.hidden_size, shape.vocab_size, bias=False, device=device, dtype=dtype)
        self._rope = {}

    @torch.no_grad()
    def init_random(self, generator: torch.Generator, std: float = 0.02, slorb_std: float = 0.01) -> None:
        """Random init: N(0, std) projections / embedding / lm_head, unit norms; SparseLinear masks at
        one (initialize), SLoRB projection the block-sum matrix (init_SLoRB), SLoRB weights N(0, slorb_std)."""
        def normal_(t, s):
            t.copy_(torch.randn(t.shape, generator=generator, device=t.device, dtype=torch.float32) * s)

        normal_(self.embed_tokens.weight, std)
        normal_(self.lm_head.weight, std)
        for mod in self.modules():
            if isinstance(mod, SparseLinear):
                normal_(mod.weight, std)
                mod.initialize()
                if mod.SLoRB:
                    mod.init_SLoRB()
                    normal_(mod.SLoRB_Weight, slorb_std)
            elif isinstance(mod, nn.Linear) and mod is not self.lm_head:
                normal_(mod.weight, std)

    def _tables(self, seq: int, device):
        key = (seq, str(device))
        if key not in self._rope:
            self._rope[key] = rotary_tables(seq, self.config.head_dim, self.config.rope_theta, device)
        return self._rope[key]

    def forward(self, idx: torch.Tensor, targets: torch.Tensor | None = None):
        cos, sin = self._tables(idx.shape[1], idx.device)
        h = self.embed_tokens(idx)
        for layer in self.layers:
            h = layer(h, cos, sin)
        logits = self.lm_head(self.norm(h))
        loss = None
        if targets is not None:
            loss = F.cross_entropy(logits.view(-1, logits.size(-1)), targets.view(-1), ignore_index=-1)
        return logits, loss, None
