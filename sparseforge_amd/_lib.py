"""ctypes binding of include/sparseforge_amd.h.

The HIP library is loaded from the package directory (built in-tree by
``sparseforge_amd.build``).  torch is imported first so that the library's
``libamdhip64.so.7`` dependency resolves to the HIP runtime torch already
loaded: device pointers and streams are then shared between the two.

There is no fallback: if the library is missing, or a tensor handed to an
op is not a contiguous tensor on a ROCm device, the call raises.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libsparseforge_amd.so")

SF_OK = 0
SF_ERR_INVALID = -1
SF_ERR_UNSUPPORTED = -2
SF_ERR_HIP = -3

DT_F32 = 0
DT_BF16 = 1
DT_U8 = 2

HARD_NONE = 0
HARD_THRESHOLD = 1
HARD_NM_TAIL_KEEP = 2
HARD_NM_STRICT = 3

METRIC = {
    "magnitude": 0,
    "hessian_obd": 1,
    "hessian_ratio": 2,
    "hessian": 3,
    "wanda": 4,
    "movement": 5,
    "weight_squared": 6,  # hessian_obd's score when hessian_diag is a placeholder: W * W
}

GATE_UNSTRUCTURED = 0
GATE_STRUCTURED = 1
GATE_STRUCTURED_EXACT = 2
GATE_ZSCORE = 3

PENALTY_NONE = 0
PENALTY_MID = 1
PENALTY_NM_2_4 = 2
PENALTY_STRUCTURED_TOPN = 3
PENALTY_TARGET = 4

BLOCK_MEAN = 0
BLOCK_RMS = 1

# stages of sf_update_mask_multi
MULTI_STATS, MULTI_TAU, MULTI_UPDATE = 1, 2, 4
MULTI_ALL = 7

# sums of sf_mask_stats (one row of MSTAT_COUNT doubles per mask)
MSTAT_SUM, MSTAT_SUM2, MSTAT_ENTROPY = 0, 1, 2
MSTAT_LT05, MSTAT_LT01, MSTAT_LT001, MSTAT_GT90, MSTAT_GT99, MSTAT_GT05 = 3, 4, 5, 6, 7, 8
MSTAT_SUM_LT05, MSTAT_SUM_GT05, MSTAT_MID, MSTAT_NONFINITE = 9, 10, 11, 12
MSTAT_TOP2, MSTAT_BOT2, MSTAT_TAIL_LT05 = 13, 14, 15
MSTAT_COUNT = 16

EFF_SOFT = 0
EFF_MIX = 1
EFF_HARD = 2

LAYOUT_K = 0
LAYOUT_MN = 1

TAU_NOALLOC_MAX_SAMPLE = 1 << 20  # SF_TAU_NOALLOC_MAX_SAMPLE

BFMT_DENSE = 0
BFMT_BSR16 = 1


class MaskParams(ctypes.Structure):
    """Mirror of ``sf_mask_params``."""

    _fields_ = [
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("metric", ctypes.c_int),
        ("gate", ctypes.c_int),
        ("n_keep", ctypes.c_int),
        ("m_group", ctypes.c_int),
        ("hard_kind", ctypes.c_int),
        ("hard_n", ctypes.c_int),
        ("hard_m", ctypes.c_int),
        ("penalty", ctypes.c_int),
        ("has_frozen", ctypes.c_int),
        ("snap_high", ctypes.c_int),
        ("score_dtype", ctypes.c_int),
        ("temperature", ctypes.c_float),
        ("eps_metric", ctypes.c_float),
        ("movement_temp", ctypes.c_float),
        ("beta_struct", ctypes.c_float),
        ("mask_lr", ctypes.c_float),
        ("penalty_coef", ctypes.c_float),
        ("binarize", ctypes.c_float),
        ("freeze_low", ctypes.c_float),
        ("freeze_high", ctypes.c_float),
        ("apply_freeze", ctypes.c_int),
    ]


class GemmDesc(ctypes.Structure):
    """Mirror of ``sf_gemm_desc``."""

    _fields_ = [
        ("dtype", ctypes.c_int),
        ("a_layout", ctypes.c_int),
        ("b_layout", ctypes.c_int),
        ("M", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("K1", ctypes.c_int64),
        ("K2", ctypes.c_int64),
        ("A1", ctypes.c_void_p),
        ("lda1", ctypes.c_int64),
        ("B1", ctypes.c_void_p),
        ("ldb1", ctypes.c_int64),
        ("A2", ctypes.c_void_p),
        ("lda2", ctypes.c_int64),
        ("B2", ctypes.c_void_p),
        ("ldb2", ctypes.c_int64),
        ("bmask", ctypes.c_void_p),
        ("bscale", ctypes.c_float),
        ("C", ctypes.c_void_p),
        ("ldc", ctypes.c_int64),
        ("c_dtype", ctypes.c_int),
        ("bias", ctypes.c_void_p),
        ("bias_dtype", ctypes.c_int),
        ("emask", ctypes.c_void_p),
        ("dw", ctypes.c_void_p),
        ("decay", ctypes.c_float),
        ("accumulate", ctypes.c_int),
        ("bmask_bytes", ctypes.c_int),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("b_format", ctypes.c_int),
        ("b_map", ctypes.c_void_p),
        ("b_map_rows", ctypes.c_int64),
        ("b_map_cols", ctypes.c_int64),
        ("c_blocks", ctypes.c_void_p),
        ("c_map", ctypes.c_void_p),
        ("c_map_rows", ctypes.c_int64),
        ("c_map_cols", ctypes.c_int64),
        ("bmask_kmajor", ctypes.c_int),
        ("ldbm", ctypes.c_int64),
    ]


class AdamwTensor(ctypes.Structure):
    """Mirror of ``sf_adamw_tensor``."""

    _fields_ = [
        ("param", ctypes.c_void_p),
        ("grad", ctypes.c_void_p),
        ("exp_avg", ctypes.c_void_p),
        ("exp_avg_sq", ctypes.c_void_p),
        ("max_exp_avg_sq", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("param_bf16_copy", ctypes.c_void_p),
        ("n", ctypes.c_int64),
        ("grad_dtype", ctypes.c_int),
        ("mask_dtype", ctypes.c_int),
        ("apply_l1", ctypes.c_int),
        ("reserved", ctypes.c_int),
    ]


class MaskLayer(ctypes.Structure):
    """Mirror of ``sf_mask_layer`` (one layer of sf_update_mask_multi)."""

    _fields_ = [
        ("rows", ctypes.c_int64),
        ("cols", ctypes.c_int64),
        ("W", ctypes.c_void_p),
        ("H", ctypes.c_void_p),
        ("aux", ctypes.c_void_p),
        ("mask", ctypes.c_void_p),
        ("frozen", ctypes.c_void_p),
        ("sample_idx", ctypes.c_void_p),
        ("sample_size", ctypes.c_int64),
        ("stats", ctypes.c_void_p),
        ("tau", ctypes.c_void_p),
        ("flips", ctypes.c_void_p),
    ]


class HutchTensor(ctypes.Structure):
    """Mirror of ``sf_hutch_tensor``."""

    _fields_ = [
        ("H", ctypes.c_void_p),
        ("hvp", ctypes.c_void_p),
        ("n", ctypes.c_int64),
        ("seed", ctypes.c_uint64),
        ("beta", ctypes.c_double),
    ]


class AdamwParams(ctypes.Structure):
    """Mirror of ``sf_adamw_params``."""

    _fields_ = [
        ("lr", ctypes.c_double),
        ("weight_decay", ctypes.c_double),
        ("beta1", ctypes.c_double),
        ("beta2", ctypes.c_double),
        ("eps", ctypes.c_double),
        ("decay", ctypes.c_double),
        ("l1", ctypes.c_double),
        ("amsgrad", ctypes.c_int),
        ("apply_l1", ctypes.c_int),
        ("step", ctypes.c_int64),
    ]


byref = ctypes.byref

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I = ctypes.c_int
_F = ctypes.c_float
_SZ = ctypes.c_size_t
_MP = ctypes.POINTER(MaskParams)

# name -> (restype, argtypes); one row per declaration of include/sparseforge_amd.h
SIGNATURES = {
    "sf_last_error": (ctypes.c_char_p, []),
    "sf_version": (_I, []),
    "sf_hard_mask": (_I, [_P, _I, _P, _I, _I64, _I64, _I, _I, _I, _P]),
    "sf_mask_workspace_size": (_SZ, [_I64, _I64, _I64]),
    "sf_score_stats": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _P, _SZ, _P]),
    "sf_tau_quantile": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _P, _I64, _F, _P, _P, _SZ, _P]),
    "sf_tau_quantile_noalloc": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _P, _I64, _F, _P, _P]),
    "sf_sample_indices": (_I, [_P, _I64, _I64, ctypes.c_uint64, _P]),
    "sf_sample_indices_sorted_workspace_size": (_SZ, [_I64, _I]),
    "sf_sample_indices_sorted": (_I, [_P, _I64, _P, _P, _I, _P, _SZ, _P]),
    "sf_gate_target": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _I, _P, _I, _P, _P, _P, _I, _P]),
    "sf_update_mask": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _I, _P, _I, _P, _P, _P, _P]),
    "sf_update_mask_multi_workspace_size": (_SZ, [ctypes.POINTER(MaskLayer), _I]),
    "sf_update_mask_multi": (_I, [_MP, _F, ctypes.POINTER(MaskLayer), _I, _I, _I, _I, _I, _I, _I, _P, _SZ, _P]),
    "sf_hard_flip_count": (_I, [_P, _P, _I, _I64, _I64, _I, _I, _I, _P, _P]),
    "sf_importance_scores": (_I, [_MP, _P, _I, _P, _I, _P, _I, _P, _I, _P]),
    "sf_joint_scores": (_I, [_MP, _P, _P, _P, _MP, _P, _P, _P, _I, _I, _I, _P, _I, _P]),
    "sf_glu_update_masks": (_I, [_MP, _P, _I, _P, _P, _I, _P, _I, _P, _P, _I, _I, _P, _P, _P]),
    "sf_effective_mask": (_I, [_P, _I, _P, _I, _I64, _I64, _I, _F, _I, _I, _I, _P]),
    "sf_effective_mask_given": (_I, [_P, _I, _P, _I, _P, _I, _I64, _I64, _I, _F, _P]),
    "sf_block_stat": (_I, [_P, _I, _I64, _I64, _I, _I, _P, _P]),
    "sf_topk_keep_workspace_size": (_SZ, [_I64]),
    "sf_topk_keep": (_I, [_P, _I64, _I64, _P, _P, _SZ, _P]),
    "sf_tile_topk": (_I, [_P, _I, _I64, _I64, _I, _I64, _P, _I, _P]),
    "sf_block_fill": (_I, [_P, _I64, _I64, _I, _P, _F, _P, _I, _I, _F, _P, _I, _P, _I, _P]),
    "sf_apply_gate": (_I, [_MP, _P, _P, _I, _P, _I, _P, _I, _I, _P]),
    "sf_freeze_mask": (_I, [_MP, _P, _I, _P, _I, _P]),
    "sf_apply_mask": (_I, [_P, _I, _P, _I, _F, _P, _I64, _I64, _P]),
    "sf_kl_chunk_rows": (_I64, [_I64]),
    "sf_kl_workspace_size": (ctypes.c_size_t, [_I64]),
    "sf_kl_forward": (_I, [_P, _P, _I, _I64, _I64, _F, _I64, _P, _I, _P, _P, _P, ctypes.c_size_t, _P]),
    "sf_kl_backward": (_I, [_P, _P, _I, _I64, _I64, _F, _P, _P, _P, _I, _P, _P]),
    "sf_to_heads": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _I, _I, _F, _P, _P]),
    "sf_from_heads": (_I, [_P, _I, _I64, _I64, _I64, _I64, _P, _P, _I, _I, _F, _P, _P]),
    "sf_transpose_batched": (_I, [_P, _I, _I64, _I64, _I64, _P, _P]),
    "sf_softmax_rows": (_I, [_P, _I, _I64, _I64, _I, _P, _P]),
    "sf_softmax_rows_backward": (_I, [_P, _P, _I, _I64, _I64, _I, _P, _P]),
    "sf_softmax_rows_double_backward": (_I, [_P, _P, _P, _I, _I64, _I64, _I, _P, _P, _P]),
    "sf_swiglu_forward": (_I, [_P, _P, _I, _I64, _P, _P]),
    "sf_swiglu_backward": (_I, [_P, _P, _P, _I, _I64, _P, _P, _P]),
    "sf_swiglu_double_backward": (_I, [_P, _P, _P, _P, _P, _I, _I64, _P, _P, _P, _P]),
    "sf_rmsnorm_workspace_size": (_SZ, [_I64, _I64]),
    "sf_rmsnorm_forward": (_I, [_P, _P, _I, _I64, _I64, _F, _P, _P, _P]),
    "sf_rmsnorm_backward": (_I, [_P, _P, _P, _P, _I, _I64, _I64, _P, _P, _P, _SZ, _P]),
    "sf_rmsnorm_double_backward": (_I, [_P, _P, _P, _P, _P, _P, _I, _I64, _I64, _P, _P, _P, _P, _SZ, _P]),
    "sf_transpose_u8": (_I, [_P, _I64, _I64, _P, _P]),
    "sf_gemm": (_I, [ctypes.POINTER(GemmDesc), _P]),
    "sf_gemm_workspace_size": (_SZ, [ctypes.POINTER(GemmDesc)]),
    "sf_column_sum": (_I, [_P, _I, _I64, _I64, _P, _I, _P]),
    "sf_adamw_step": (_I, [_P, _I, _P, _I, _P, _P, _P, _I, _P, _I, _P, _I64, ctypes.POINTER(AdamwParams), _P]),
    "sf_adamw_step_multi": (_I, [ctypes.POINTER(AdamwTensor), _I, _I, _I, ctypes.POINTER(AdamwParams), _P]),
    "sf_bsr_count": (_I, [_P, _I, _P, _I, _I64, _I64, _I, _P, _P, _P]),
    "sf_bsr_scan": (_I, [_P, _I64, _P, _P]),
    "sf_bsr_fill": (_I, [_P, _I, _P, _I, _I64, _I64, _I, _P, _P, _P, _P, _I, _P, _P]),
    "sf_bsr_block_map": (_I, [_P, _P, _I64, _I64, _P, _P]),
    "sf_bsr_transpose": (_I, [_P, _I, _I64, _P, _I64, _I64, _P, _P, _P]),
    "sf_rademacher": (_I, [_P, _I, _I64, ctypes.c_uint64, _P]),
    "sf_rademacher_dot_workspace_size": (_SZ, []),
    "sf_rademacher_dot": (_I, [_P, _I, _P, _I, _I64, ctypes.c_uint64, _P, _P, _SZ, _P]),
    "sf_hutchinson_update_multi": (_I, [ctypes.POINTER(HutchTensor), _I, _I, _I, _P]),
    "sf_hutchinson_update": (_I, [_P, _I, _P, _I, _P, _I, _I64, ctypes.c_uint64, ctypes.c_double, _P]),
    "sf_mask_stats_workspace_size": (_SZ, []),
    "sf_mask_stats": (_I, [_P, _I, _I64, _I64, _I64, _F, _P, _P, _SZ, _P]),
    "sf_mask_hist": (_I, [_P, _I, _I64, _P, _I64, _I, _F, _F, _P, _P]),
    "sf_keep_split_sum": (_I, [_P, _P, _I64, _P, _P]),
    "sf_pack_2to4_sizes": (_SZ, [_I64, _I64, ctypes.POINTER(ctypes.c_size_t)]),
    "sf_pack_2to4": (_I, [_P, _I, _P, _I, _I64, _I64, _P, _P, _P, _P]),
    "sf_unpack_2to4": (_I, [_P, _P, _I64, _I64, _P, _I, _P]),
    "sf_gemm_2to4": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _I, _P, _I, _I64, _P]),
    "sf_apply_mask_2to4": (_I, [_P, _P, _I64, _I64, _P, _P, _P, _P, _P]),
    "sf_gemm_2to4_lowrank": (_I, [_P, _I64, _I64, _P, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I, _P, _I,
                                  _I64, _P]),
    "sf_mfma_probe": (_I, [_I, _I, _P, _P]),
    "sf_hbm_probe": (_I, [_I, _P, _P, _P, _I64, _I, _P]),
}

_lock = threading.Lock()
_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the HIP library and bind every declared entry point (no GPU needed)."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"sparseforge_amd: HIP library not found at {path}; build it with "
                "`python -m sparseforge_amd.build` (there is no CPU fallback)"
            )
        lib = ctypes.CDLL(path)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
        return lib


def lib() -> ctypes.CDLL:
    return _lib if _lib is not None else load()


def last_error() -> str:
    msg = lib().sf_last_error()
    return msg.decode(errors="replace") if msg else ""


def check(rc: int, what: str) -> None:
    """Raise the exception type the reference raises for the same condition."""
    if rc == SF_OK:
        return
    msg = f"{what}: {last_error()}"
    if rc == SF_ERR_INVALID:
        raise ValueError(msg)
    if rc == SF_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return DT_F32
    if t.dtype == torch.bfloat16:
        return DT_BF16
    raise TypeError(f"sparseforge_amd: unsupported dtype {t.dtype} (float32 / bfloat16 only)")


def require_device(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must be contiguous ROCm tensors on one device."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"sparseforge_amd runs on the GPU only; got a tensor on {t.device} (no CPU path exists)"
            )
        if not t.is_contiguous():
            raise ValueError("sparseforge_amd: tensors must be contiguous")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"sparseforge_amd: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise ValueError("sparseforge_amd: no tensor given")
    return dev


def require_device_only(*tensors: torch.Tensor | None) -> torch.device:
    """All given tensors must be ROCm tensors on one device (any strides)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError(
                f"sparseforge_amd runs on the GPU only; got a tensor on {t.device} (no CPU path exists)"
            )
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"sparseforge_amd: tensors on different devices ({dev} vs {t.device})")
    if dev is None:
        raise ValueError("sparseforge_amd: no tensor given")
    return dev


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
