"""Masked linear + SLoRB as autograd functions over the sf_gemm MFMA engine.

Reference: legacy/sparse_modeling.py:56-132 (FusedMaskedLinearSTE) and
:737-796 (SparseLinear.forward with the SLoRB pair of F.linear).

    z  = x P^T                                    (SLoRB projection, [T, r])
    y  = x (W.E.s)^T + z S^T + b                  (one GEMM: the z S^T term is a second K segment)
    dz = dy S
    dx = dy (W.E) + dz P                          (one GEMM, two K segments; no s, as in :113-115)
    dW = dy^T x  (+ decay W [E < 0.5])            (STE: the mask does not enter dW, :120-125)
    db = sum_t dy,  dS = dy^T z,  dP = dz^T x

The backward is itself an autograd Function whose backward is written with
the same kernels, so torch.autograd.grad(..., create_graph=True) and the
Hutchinson Hessian-vector product (legacy/utils.py:772-795) work through it.
SLoRB ranks that are not a multiple of the 16-byte vector width are padded
with zero rows/columns of P and S, which leaves every product unchanged.
"""
from __future__ import annotations

import torch

from . import _lib as L
from . import kernels as K
from . import profiling as _prof


# ---------------------------------------------------------------------------
# GEMM front end
# ---------------------------------------------------------------------------
def _vec(dtype: torch.dtype) -> int:
    return 8 if dtype == torch.bfloat16 else 4


def gemm(M, N, A1, B1, K1, a_layout, b_layout, *, A2=None, B2=None, K2=0, bmask=None, bscale=1.0, bias=None,
         emask=None, dw=None, decay=0.0, out=None, out_dtype=None, accumulate=False, bmask_t=None,
         max_splits=None) -> torch.Tensor:
    """C[M, N] = A1 . B1'^T (+ A2 . B2^T) on the device.

    a_layout: L.LAYOUT_K (A1 is [M, K]) or L.LAYOUT_MN (A1 is [K, M]);
    b_layout: L.LAYOUT_K (B1 is [N, K]) or L.LAYOUT_MN (B1 is [K, N]).
    bmask: effective mask of B1 in B1's dtype (multiplied in), or a uint8
    and-mask (0x00 / 0xFF per element) for a 0/1 mask.
    bmask_t: optional K-major copy [N, K] of a uint8 bmask of an N-contiguous
    B1 (transpose_u8(bmask)); the bf16 kernel then copies the mask with the
    weight tile instead of staging both through registers.
    """
    dev = L.require_device(A1, B1, A2, B2, bmask, bias, emask, dw, out, bmask_t)
    dt = A1.dtype

    def _shape(t, want, name):
        if t is not None and tuple(t.shape) != tuple(want):
            raise ValueError(f"gemm: {name} has shape {tuple(t.shape)}, expected {tuple(want)}")

    def _op_shape(rows, k, layout):
        return (rows, k) if layout == L.LAYOUT_K else (k, rows)

    _shape(A1, _op_shape(M, K1, a_layout), "A1")
    _shape(B1, _op_shape(N, K1, b_layout), "B1")
    _shape(bmask, _op_shape(N, K1, b_layout), "bmask")
    if K2:
        if A2 is None or B2 is None:
            raise ValueError("gemm: K2 > 0 needs A2 and B2")
        _shape(A2, _op_shape(M, K2, a_layout), "A2")
        _shape(B2, _op_shape(N, K2, b_layout), "B2")
    _shape(bias, (N,), "bias")
    _shape(emask, (M, N), "emask")
    _shape(dw, (M, N), "dw")
    _shape(out, (M, N), "out")
    bmask_bytes = bmask is not None and bmask.dtype == torch.uint8
    for t in (B1, A2, B2, None if bmask_bytes else bmask, emask, dw):
        if t is not None and t.dtype != dt:
            raise TypeError(f"gemm: operand dtype {t.dtype} != {dt}")
    if bmask_bytes and bscale != 1.0:
        raise ValueError("gemm: a byte and-mask cannot carry a weight-scaling factor")
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype or dt, device=dev)
    d = L.GemmDesc()
    d.dtype = L.dtype_code(A1)
    d.a_layout, d.b_layout = a_layout, b_layout
    d.M, d.N, d.K1, d.K2 = M, N, K1, K2
    d.A1, d.B1 = L.ptr(A1), L.ptr(B1)
    d.lda1 = A1.shape[1]
    d.ldb1 = B1.shape[1]
    if K2:
        d.A2, d.B2 = L.ptr(A2), L.ptr(B2)
        d.lda2, d.ldb2 = A2.shape[1], B2.shape[1]
    d.bmask = L.ptr(bmask)
    d.bmask_bytes = int(bmask_bytes)
    if (bmask_t is not None and bmask_bytes and b_layout == L.LAYOUT_MN and dt == torch.bfloat16
            and K1 % 16 == 0 and bmask_t.data_ptr() % 16 == 0):
        _shape(bmask_t, (N, K1), "bmask_t")
        if bmask_t.dtype != torch.uint8:
            raise TypeError("gemm: bmask_t must be a uint8 and-mask")
        d.bmask, d.bmask_kmajor, d.ldbm = L.ptr(bmask_t), 1, K1
    d.bscale = float(bscale)
    d.C, d.ldc, d.c_dtype = L.ptr(out), out.shape[1], L.dtype_code(out)
    if bias is not None:
        d.bias, d.bias_dtype = L.ptr(bias), L.dtype_code(bias)
    d.emask, d.dw, d.decay = L.ptr(emask), L.ptr(dw), float(decay)
    d.accumulate = int(bool(accumulate))
    ws_bytes = L.lib().sf_gemm_workspace_size(L.byref(d))
    if max_splits is not None and ws_bytes > max_splits * M * N * 4:  # fewer K splits (the big products only)
        ws_bytes = max_splits * M * N * 4 if max_splits > 1 else 0
    ws = None
    if ws_bytes:  # split-K scratch from torch's caching allocator; the library never allocates
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev)
        d.workspace, d.workspace_bytes = ws.data_ptr(), ws_bytes
    with _prof.region("sf_gemm", 2.0 * M * N * (K1 + K2), "FLOP", dev):
        L.check(L.lib().sf_gemm(L.byref(d), L.stream(dev)), "sf_gemm")
    return out


def mm_nt(A, B, **kw):
    """A [M, K] . B [N, K]^T"""
    return gemm(A.shape[0], B.shape[0], A, B, A.shape[1], L.LAYOUT_K, L.LAYOUT_K, **kw)


def mm_nn(A, B, **kw):
    """A [M, K] . B [K, N]"""
    return gemm(A.shape[0], B.shape[1], A, B, A.shape[1], L.LAYOUT_K, L.LAYOUT_MN, **kw)


def mm_tn(A, B, **kw):
    """A [K, M]^T . B [K, N]"""
    return gemm(A.shape[1], B.shape[1], A, B, A.shape[0], L.LAYOUT_MN, L.LAYOUT_MN, **kw)


def column_sum(A: torch.Tensor, out_dtype: torch.dtype) -> torch.Tensor:
    dev = L.require_device(A)
    out = torch.empty(A.shape[1], dtype=out_dtype, device=dev)
    L.check(L.lib().sf_column_sum(L.ptr(A), L.dtype_code(A), A.shape[0], A.shape[1], L.ptr(out),
                                  L.dtype_code(out), L.stream(dev)), "sf_column_sum")
    return out


def effective_mask(mask: torch.Tensor, dtype: torch.dtype, mode: str, hx: float, hard_kind: int, hard_n: int,
                   hard_m: int = 4) -> torch.Tensor:
    """E = mask.to(dtype) ('soft'), (hx*mask + (1-hx)*hard(mask)).to(dtype) ('mix') or hard(mask) ('hard').

    With mode 'hard' and dtype torch.uint8 the result is a byte and-mask
    (0xFF kept, 0x00 pruned) that the GEMMs apply while staging W.
    """
    dev = L.require_device(mask)
    eff = torch.empty(mask.shape, dtype=dtype, device=dev)
    m = {"mix": L.EFF_MIX, "hard": L.EFF_HARD}.get(mode, L.EFF_SOFT)
    code = L.DT_U8 if dtype == torch.uint8 else L.dtype_code(eff)
    nbytes = mask.numel() * (mask.element_size() + eff.element_size())
    with _prof.region("sf_effective_mask", nbytes, "B", dev):
        L.check(L.lib().sf_effective_mask(L.ptr(mask), L.dtype_code(mask), L.ptr(eff), code,
                                          mask.shape[0], mask.shape[1], m, float(hx), hard_kind, hard_n, hard_m,
                                          L.stream(dev)), "sf_effective_mask")
    return eff


def effective_mask_given(mask: torch.Tensor, hard: torch.Tensor, dtype: torch.dtype, mode: str,
                         hx: float) -> torch.Tensor:
    """effective_mask with the hard projection passed in (the block hard types)."""
    dev = L.require_device(mask, hard)
    if hard.shape != mask.shape:
        raise ValueError("hard mask shape differs from the soft mask")
    eff = torch.empty(mask.shape, dtype=dtype, device=dev)
    m = {"mix": L.EFF_MIX, "hard": L.EFF_HARD}.get(mode, L.EFF_SOFT)
    code = L.DT_U8 if dtype == torch.uint8 else L.dtype_code(eff)
    nbytes = mask.numel() * (mask.element_size() + hard.element_size() + eff.element_size())
    with _prof.region("sf_effective_mask", nbytes, "B", dev):
        L.check(L.lib().sf_effective_mask_given(L.ptr(mask), L.dtype_code(mask), L.ptr(hard), L.dtype_code(hard),
                                                L.ptr(eff), code, mask.shape[0], mask.shape[1], m, float(hx),
                                                L.stream(dev)), "sf_effective_mask_given")
    return eff


def apply_mask(W: torch.Tensor, E: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """(W * E).to(W dtype) [* scale, rounded again]: the masked weight the unmasked GEMMs read."""
    dev = L.require_device(W, E)
    if E.shape != W.shape:
        raise ValueError(f"mask shape {tuple(E.shape)} != weight shape {tuple(W.shape)}")
    out = torch.empty_like(W)
    code = L.DT_U8 if E.dtype == torch.uint8 else L.dtype_code(E)
    with _prof.region("sf_apply_mask", W.numel() * (2 * W.element_size() + E.element_size()), "B", dev):
        L.check(L.lib().sf_apply_mask(L.ptr(W), L.dtype_code(W), L.ptr(E), code, float(scale), L.ptr(out),
                                      W.shape[0], W.shape[1], L.stream(dev)), "sf_apply_mask")
    return out


_BAD24: dict = {}


def apply_mask_2to4(W: torch.Tensor, E: torch.Tensor):
    """Wm = W * E for a bf16 W and a byte and-mask E that keeps two of every four columns, plus
    the packed 2:4 form of Wm (values, index words), in one pass (sf_apply_mask_2to4).  Groups
    keeping more than two columns are only counted in a per-device device counter, never read
    here: the N:M hard projection with N = 2, M = 4 produces none."""
    dev = L.require_device(W, E)
    out_f, in_f = W.shape
    Wm = torch.empty_like(W)
    vals = torch.empty(out_f, in_f // 2, dtype=torch.bfloat16, device=dev)
    idx = torch.empty(out_f * in_f // 8, dtype=torch.uint8, device=dev)
    key = dev.index if dev.index is not None else torch.cuda.current_device()
    bad = _BAD24.get(key)
    if bad is None:
        bad = _BAD24[key] = torch.zeros(1, dtype=torch.int64, device=dev)
    with _prof.region("sf_apply_mask_2to4", W.numel() * 5 + vals.numel() * 2 + idx.numel(), "B", dev):
        L.check(L.lib().sf_apply_mask_2to4(L.ptr(W), L.ptr(E), out_f, in_f, L.ptr(Wm), L.ptr(vals), L.ptr(idx),
                                           L.ptr(bad), L.stream(dev)), "sf_apply_mask_2to4")
    return Wm, vals, idx


def gemm_2to4(x2: torch.Tensor, vals: torch.Tensor, idx: torch.Tensor, out_features: int, z=None, S=None,
              bias=None) -> torch.Tensor:
    """y [T, out] bf16 = x2 Wm^T (+ z S^T) (+ bias) with Wm packed 2:4 (sf_gemm_2to4_lowrank)."""
    dev = L.require_device(x2, vals, idx, z, S, bias)
    T, in_f = x2.shape
    y = torch.empty(T, out_features, dtype=torch.bfloat16, device=dev)
    r = 0 if z is None else z.shape[1]
    flops = 2.0 * T * out_features * (in_f + r)
    with _prof.region("sf_gemm_2to4", flops, "FLOP", dev):
        L.check(L.lib().sf_gemm_2to4_lowrank(L.ptr(x2), x2.stride(0), T, L.ptr(vals), L.ptr(idx), out_features,
                                             in_f, L.ptr(z), 0 if z is None else z.stride(0), L.ptr(S),
                                             0 if S is None else S.stride(0), r, L.ptr(bias),
                                             L.dtype_code(bias) if bias is not None else 0, L.ptr(y),
                                             L.dtype_code(y), y.stride(0), L.stream(dev)), "sf_gemm_2to4_lowrank")
    return y


def transpose_u8(E: torch.Tensor) -> torch.Tensor:
    """[rows, cols] uint8 -> its transpose [cols, rows] (sf_transpose_u8)."""
    dev = L.require_device(E)
    if E.dtype != torch.uint8 or E.dim() != 2:
        raise TypeError("transpose_u8 expects a 2-D uint8 tensor")
    out = torch.empty(E.shape[1], E.shape[0], dtype=torch.uint8, device=dev)
    with _prof.region("sf_transpose_u8", 2 * E.numel(), "B", dev):
        L.check(L.lib().sf_transpose_u8(L.ptr(E), E.shape[0], E.shape[1], L.ptr(out), L.stream(dev)),
                "sf_transpose_u8")
    return out


def decay_term(G: torch.Tensor, E: torch.Tensor | None, decay: float, out: torch.Tensor | None = None) -> torch.Tensor:
    """out (+)= decay * G * [E < 0.5] in G's dtype (E = None: nothing is pruned and the term is 0).

    The derivative along G of the SR-STE term decay * W * [E < 0.5] of the weight
    gradient (legacy/sparse_modeling.py:123-125), which is elementwise in W.  Off
    the paper's path (its decay is 0), so it is two device elementwise ops.
    """
    L.require_device(G, E, out)
    if out is None:
        out = torch.zeros_like(G)
    if E is None:
        return out
    if E.shape != G.shape or out.shape != G.shape:
        raise ValueError("decay_term: G, E and out must have one shape")
    pruned = (E == 0) if E.dtype == torch.uint8 else (E < 0.5)
    out.add_(G * pruned.to(G.dtype), alpha=float(decay))
    return out


def _as_values(E: torch.Tensor | None, dt: torch.dtype) -> torch.Tensor | None:
    """A byte and-mask as 0/1 values of dtype dt (for epilogue products); other masks unchanged."""
    if E is not None and E.dtype == torch.uint8:
        return (E != 0).to(dt)
    return E


def _cat_k(parts, dim: int):
    """The operands of one K segment side by side (None when there are none)."""
    if not parts:
        return None
    return parts[0] if len(parts) == 1 else torch.cat(parts, dim).contiguous()


def _pad_rank(P: torch.Tensor, S: torch.Tensor):
    """Zero-pad the SLoRB rank to a multiple of the vector width."""
    r = P.shape[0]
    v = _vec(P.dtype)
    rp = (r + v - 1) // v * v
    if rp == r:
        return P.contiguous(), S.contiguous(), r
    Pp = torch.zeros(rp, P.shape[1], dtype=P.dtype, device=P.device)
    Pp[:r] = P
    Sp = torch.zeros(S.shape[0], rp, dtype=S.dtype, device=S.device)
    Sp[:, :r] = S
    return Pp, Sp, r


def _opt(t):
    return t.contiguous() if t is not None else None


_SIDE: dict = {}
_CUS: dict = {}


def _side_stream(t: torch.Tensor):
    """A second stream for the weight-gradient products when the two big backward products (dx [T, in] and
    dW [out, in], 256 x 256 tiles) would each leave compute units idle: running dW beside dx fills them.
    None when both fill the GPU by themselves (the LLaMA-7B layer shapes) or off the GPU."""
    if not t.is_cuda:
        return None
    dev = t.device.index if t.device.index is not None else torch.cuda.current_device()
    if dev not in _SIDE:
        _SIDE[dev] = torch.cuda.Stream(device=dev)  # default priority
        _CUS[dev] = torch.cuda.get_device_properties(dev).multi_processor_count
    return _SIDE[dev]


def _fills(rows: int, cols: int, dev: int) -> bool:
    return ((rows + 255) // 256) * ((cols + 255) // 256) >= _CUS[dev]


# ---------------------------------------------------------------------------
# autograd
# ---------------------------------------------------------------------------
class _MaskedLinearBackward(torch.autograd.Function):
    """(gy, x, W, P, S, b?) -> (dx, dW, db, dP, dS); differentiable for the HVP."""

    @staticmethod
    def forward(ctx, gy, x, W, P, S, E, decay, has_bias, z_fwd=None, wm_fwd=None):
        has_slorb = P is not None
        # z = x P^T is kept from the forward; its dependence on x and P is
        # written out explicitly in backward(), so the cached copy is detached.
        z = (z_fwd if z_fwd is not None else mm_nt(x, P)) if has_slorb else None
        dz = mm_nn(gy, S) if has_slorb else None
        # dx = gy (W.E): the forward's masked weight when it kept one (no weight-scaling factor),
        # else rebuilt with one elementwise pass
        Wm = wm_fwd if wm_fwd is not None else (apply_mask(W, E) if E is not None else W)
        T, out, inn = gy.shape[0], gy.shape[1], x.shape[1]
        side = _side_stream(gy)
        if side is not None:
            di = gy.device.index if gy.device.index is not None else torch.cuda.current_device()
            if _fills(T, inn, di) and _fills(out, inn, di):
                side = None
        dW = torch.empty(out, inn, dtype=gy.dtype, device=gy.device)  # allocated on the calling stream
        dS = torch.empty(out, P.shape[0], dtype=gy.dtype, device=gy.device) if has_slorb else None
        main = torch.cuda.current_stream(gy.device) if side is not None else None

        # beside dx a product needs fewer K splits to fill the compute units dx leaves idle
        ms = 2 if side is not None else None

        def weight_grads():
            if decay != 0.0:
                mm_tn(gy, x, emask=_as_values(E, W.dtype), dw=W, decay=decay, out=dW, max_splits=ms)
            else:
                mm_tn(gy, x, out=dW, max_splits=ms)
            if has_slorb:
                mm_tn(gy, z, out=dS)

        if side is not None:  # dW and dS beside dz, dx and dP; joined before returning
            side.wait_stream(main)
            with torch.cuda.stream(side):
                weight_grads()
        if has_slorb:
            dx = mm_nn(gy, Wm, A2=dz, B2=P, K2=P.shape[0])
        else:
            dx = mm_nn(gy, Wm)
        if side is None:
            weight_grads()
        db = column_sum(gy, W.dtype) if has_bias else None
        dP = mm_tn(dz, x) if has_slorb else None
        if side is not None:
            main.wait_stream(side)
        # W.E stays for the double backward's d/d gy (gdx (W.E)^T), so that product runs unmasked
        ctx.save_for_backward(gy, x, W, P, S, E, z, dz, Wm if E is not None else None)
        del Wm
        ctx.decay = decay
        ctx.has_slorb = has_slorb
        return dx, dW, db, dP, dS

    @staticmethod
    def backward(ctx, g_dx, g_dW, g_db, g_dP, g_dS):
        gy, x, W, P, S, E, z, dz, Wm = ctx.saved_tensors
        T, out = gy.shape
        dt = gy.dtype
        g_dx, g_dW, g_db, g_dP, g_dS = (_opt(t) for t in (g_dx, g_dW, g_db, g_dP, g_dS))
        if not ctx.has_slorb:
            g_dP = g_dS = None
        # d/d gy = gdx (W.E)^T + x gdW^T + u S^T + z gdS^T + gdb with u = gdx P^T + x gdP^T: the
        # low-rank terms ride as one second K segment [u | z] . [S | gdS]^T of the first full-size
        # product; the second full-size product accumulates into its output in the output dtype
        # (as autograd sums gradient contributions)
        u = None
        if ctx.has_slorb:
            if g_dx is not None:
                u = mm_nt(g_dx, P)
                if g_dP is not None:
                    mm_nt(x, g_dP, out=u, accumulate=True)
            elif g_dP is not None:
                u = mm_nt(x, g_dP)
        la = _cat_k([t for t in (u, z if g_dS is not None else None) if t is not None], 1)
        lb = _cat_k([t for t, a in ((S, u), (g_dS, g_dS)) if a is not None], 1)
        seg = {"A2": la, "B2": lb, "K2": la.shape[1]} if la is not None else {}
        # d/dW = (gy^T gdx) . E  (+ decay gdW [E < 0.5]: the SR-STE term decay W [E < 0.5] of dW is
        # elementwise in W, legacy/sparse_modeling.py:123-125), beside the two products below when
        # they leave compute units idle (as in forward())
        gW = None
        side = _side_stream(gy) if g_dx is not None else None
        if side is not None:
            di = gy.device.index if gy.device.index is not None else torch.cuda.current_device()
            if _fills(T, x.shape[1], di) and _fills(out, x.shape[1], di):
                side = None
        if g_dx is not None:
            gW = torch.empty(out, x.shape[1], dtype=gy.dtype, device=gy.device)
        main = torch.cuda.current_stream(gy.device) if side is not None else None

        def weight_grad():
            if g_dx is not None:
                mm_tn(gy, g_dx, emask=_as_values(E, W.dtype), out=gW, max_splits=2 if side is not None else None)
            return decay_term(g_dW, E, ctx.decay, out=gW) if ctx.decay != 0.0 and g_dW is not None else gW

        if side is not None:
            side.wait_stream(main)
            with torch.cuda.stream(side):
                weight_grad()
        ggy = None
        if g_dx is not None:
            ggy = mm_nt(g_dx, Wm if Wm is not None else W, bias=g_db, **seg)
            if g_dW is not None:
                mm_nt(x, g_dW, out=ggy, accumulate=True)
        elif g_dW is not None:
            ggy = mm_nt(x, g_dW, bias=g_db, **seg)
        elif la is not None:
            ggy = mm_nt(la, lb, bias=g_db)
        if ggy is None and g_db is not None:
            ggy = g_db.expand(T, out).to(dt).contiguous()
        # d/dx = gy gdW + [w | dz] . [P ; gdP] with w = gy gdS (one GEMM, the low-rank part its
        # second K segment)
        w = mm_nn(gy, g_dS) if ctx.has_slorb and g_dS is not None else None
        ra = _cat_k([t for t in (w, dz if g_dP is not None else None) if t is not None], 1)
        rb = _cat_k([t for t, a in ((P, w), (g_dP, g_dP)) if a is not None], 0)
        gx = None
        if g_dW is not None:
            gx = mm_nn(gy, g_dW, **({"A2": ra, "B2": rb, "K2": ra.shape[1]} if ra is not None else {}))
        elif ra is not None:
            gx = mm_nn(ra, rb)
        if side is None:
            gW = weight_grad()
        else:
            main.wait_stream(side)
        # d/dP = dz^T gdx + (gy gdS)^T x ;  d/dS = gy^T (gdx P^T + x gdP^T)
        gP = gS = None
        if ctx.has_slorb:
            if g_dx is not None and w is not None:  # two skinny products (K = tokens each)
                gP = mm_tn(dz, g_dx)
                mm_tn(w, x, out=gP, accumulate=True)
            elif g_dx is not None:
                gP = mm_tn(dz, g_dx)
            elif w is not None:
                gP = mm_tn(w, x)
            if u is not None:
                gS = mm_tn(gy, u)
        return ggy, gx, gW, gP, gS, None, None, None, None, None


class _MaskedLinear(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x2, W, bias, P, S, E, scale, decay, nm24=False):
        z = None
        if nm24:
            # E is a 2:4 hard mask: the pass that writes W.E also packs it, and the product runs on
            # the sparse MFMA (the SLoRB term as a dense second segment of the same kernel)
            Wm, vals, idx = apply_mask_2to4(W, E)
            if P is not None:
                z = mm_nt(x2, P)
            y = gemm_2to4(x2, vals, idx, W.shape[0], z=z, S=S, bias=bias)
            del vals, idx
        else:
            # y = x (W.E.s)^T: one elementwise pass writes the masked weight, the GEMM runs unmasked
            Wm, s = (apply_mask(W, E, scale), 1.0) if E is not None else (W, scale)
            if P is not None:
                z = mm_nt(x2, P)
                y = mm_nt(x2, Wm, bscale=s, A2=z, B2=S, K2=P.shape[0], bias=bias)
            else:
                y = mm_nt(x2, Wm, bscale=s, bias=bias)
        # Without a weight-scaling factor the input gradient needs the same W.E: it is saved for the
        # backward (2 B/param of bf16 weight) instead of being rebuilt there by another pass.  It goes
        # through save_for_backward, so the version counters of W and E guard it like the rest.
        keep = E is not None and scale == 1.0
        ctx.save_for_backward(x2, W, P, S, E, z, Wm if keep else None)
        del Wm
        ctx.decay = decay
        ctx.has_bias = bias is not None
        return y

    @staticmethod
    def backward(ctx, gy):
        x2, W, P, S, E, z, wm = ctx.saved_tensors
        gy = gy.contiguous().to(W.dtype)
        dx, dW, db, dP, dS = _MaskedLinearBackward.apply(gy, x2, W, P, S, E, ctx.decay, ctx.has_bias, z, wm)
        del wm
        return dx, dW, db, dP, dS, None, None, None, None


def _compute_dtype(x: torch.Tensor, W: torch.Tensor) -> torch.dtype:
    if torch.is_autocast_enabled("cuda"):
        return torch.get_autocast_dtype("cuda")
    return W.dtype


def masked_linear(x, weight, bias, mask, mask_mode, hx, hard_kind, hard_n, scale, P=None, S=None, decay=0.0,
                  eff=None, hard=None, hard_m=4, cache=None):
    """y = x (W.E.s)^T + (x P^T) S^T + b with STE gradients.

    mask_mode: 'none' (E = 1), 'soft' (E = mask) or 'mix' (E = hx*mask + (1-hx)*hard(mask)).
    eff: a precomputed E in the compute dtype (skips the mask pass).
    hard: a precomputed hard(mask) (block hard types); else hard_kind / hard_n / hard_m project
    per group of hard_m along the input dimension.
    cache: a dict owned by the caller (one per layer) that keeps the mixed-mode E between calls.
    The soft mask changes only when the mask update writes it, while the reference rebuilds
    hard(mask) on every forward (legacy/sparse_modeling.py:759-771); E is reused while the mask's
    storage, its version counter (bumped by every in-place write: torch ops, and the library's mask
    kernels explicitly) and the projection parameters are unchanged.
    Strided inputs are accepted (made contiguous before the kernels, as F.linear accepts them).
    """
    L.require_device_only(x, weight, bias, mask, P, S, eff, hard)
    dt = _compute_dtype(x, weight)
    if dt not in (torch.float32, torch.bfloat16):
        raise TypeError(f"sparseforge_amd: unsupported compute dtype {dt}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, x.shape[-1])
    if x2.dtype != dt:
        x2 = x2.to(dt)
    x2 = x2.contiguous()
    W = (weight if weight.dtype == dt else weight.to(dt)).contiguous()
    b = None if bias is None else (bias if bias.dtype == dt else bias.to(dt)).contiguous()
    mask = _opt(mask)
    hard = _opt(hard)
    own_hard_bytes = eff is None and hard is None and mask_mode == "mix" and hx <= 0.0 and scale == 1.0
    key = None
    if eff is None and cache is not None and mask_mode == "mix" and hard is None:
        key = (mask.data_ptr(), mask._version, tuple(mask.shape), mask.dtype, float(hx), float(scale), hard_kind,
               hard_n, hard_m, dt)
        if cache.get("key") == key:
            eff = cache["eff"]
        else:
            cache.clear()
    if eff is None and mask_mode != "none":
        if mask_mode == "mix" and hx <= 0.0 and scale == 1.0:
            # E = hard(mask) exactly: staged as a byte and-mask (W * 1 = W, W * 0 = 0)
            eff = (effective_mask_given(mask, hard, torch.uint8, "hard", 0.0) if hard is not None
                   else effective_mask(mask, torch.uint8, "hard", 0.0, hard_kind, hard_n, hard_m))
        elif hard is not None and mask_mode == "mix":
            eff = effective_mask_given(mask, hard, dt, mask_mode, hx)
        else:
            eff = effective_mask(mask, dt, mask_mode, hx, hard_kind, hard_n, hard_m)
        if key is not None:
            cache["key"], cache["eff"] = key, eff
    if mask_mode == "none":
        eff = None
    eff = _opt(eff)
    Pp = Sp = None
    r = 0
    if P is not None:
        Pp, Sp, r = (P, S, P.shape[0]) if P.dtype == dt else (P.to(dt), S.to(dt), P.shape[0])
        Pp, Sp = Pp.contiguous(), Sp.contiguous()
        if Pp.shape[0] % _vec(dt):
            Pp, Sp, r = _PadRank.apply(Pp, Sp)
    # A 2:4 hard mask along the input dimension (both N:M kinds keep exactly two of every four
    # columns when in % 4 == 0) runs the forward product on the sparse MFMA.
    nm24 = (own_hard_bytes and eff is not None and hard_kind in (L.HARD_NM_TAIL_KEEP, L.HARD_NM_STRICT)
            and hard_n == 2 and hard_m == 4 and dt == torch.bfloat16 and W.shape[0] % 32 == 0
            and W.shape[1] % 64 == 0 and x2.shape[0] * W.shape[1] * 2 < 2 ** 31
            and W.shape[0] * W.shape[1] < 2 ** 31)
    y = _MaskedLinear.apply(x2, W, b, Pp, Sp, eff, float(scale), float(decay), nm24)
    return y.view(*lead, y.shape[-1])


class _PadRank(torch.autograd.Function):
    """Zero-pad P [r, in] and S [out, r] to a rank multiple of the vector width (differentiable)."""

    @staticmethod
    def forward(ctx, P, S):
        Pp, Sp, r = _pad_rank(P, S)
        ctx.r = r
        return Pp, Sp, r

    @staticmethod
    def backward(ctx, gPp, gSp, _):
        r = ctx.r
        gP = gPp[:r] if gPp is not None else None
        gS = gSp[:, :r] if gSp is not None else None
        return gP, gS


class FusedMaskedLinearSTE(torch.autograd.Function):
    """Drop-in of legacy/sparse_modeling.py:56-132: apply(x, weight, bias, mask, decay, scale_factor).

    `mask` is the effective mask (any [out, in] float tensor); it is cast to the
    weight dtype as the reference's `mask_cast` and applied inside the GEMMs.
    """

    @staticmethod
    def apply(x, weight, bias, mask, decay: float, scale_factor: float = 1.0):  # noqa: D102
        m = mask.detach().contiguous()
        return masked_linear(x, weight, bias, m, "soft", 1.0, L.HARD_NONE, 2, scale_factor, decay=float(decay))
