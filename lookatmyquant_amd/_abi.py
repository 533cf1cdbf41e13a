"""ctypes binding of liblamq_hip.so, the gfx950 HIP library (include/lamq.h), and thin wrappers that take torch
device tensors. Statuses become exceptions: LAMQ_EINVAL -> ValueError, LAMQ_EUNSUP -> NotImplementedError, a
hipError_t -> RuntimeError. There is no other implementation of these operations: if the library or a GPU is
missing, every call raises."""

from __future__ import annotations

import ctypes
from pathlib import Path

import torch  # loaded first: the library then binds to the HIP runtime torch already mapped (same SONAME)

PKG = Path(__file__).resolve().parent
SO = PKG / "liblamq_hip.so"

_c_i64, _c_int, _c_dbl, _c_flt, _c_size, _p = ctypes.c_int64, ctypes.c_int, ctypes.c_double, ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p

# name -> (restype, argtypes), exactly the declarations of include/lamq.h
SIGNATURES = {
    "lamq_abi_version": (_c_int, []),
    "lamq_viterbi_workspace_size": (_c_size, [_c_i64, _c_int, _c_int, _c_int]),
    "lamq_viterbi_rows": (_c_int, [_p, _c_i64, _c_int, _c_i64, _p, _c_int, _c_int, _p, _p, _c_i64, _p, _c_size, _p]),
    "lamq_ldlq_trellis_block": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _p, _p, _c_int, _c_int, _c_i64, _c_i64,
                                         _c_int, _c_int, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p]),
    "lamq_ldlq_scalar_block": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _p, _c_int, _c_int, _c_i64, _c_i64, _p,
                                        _c_i64, _p, _c_i64, _p]),
    "lamq_ldlq_multirate_block": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _c_int, _c_int, _p, _c_i64, _c_i64,
                                           _p, _c_i64, _p, _c_i64, _p]),
    "lamq_viterbi16_workspace_size": (_c_size, [_c_i64, _c_int, _c_int, _c_int]),
    "lamq_viterbi16_rows": (_c_int, [_p, _c_i64, _c_int, _c_i64, _p, _c_int, _c_int, _p, _p, _c_i64, _p, _c_size, _p]),
    "lamq_ldlq_trellis16_block": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _p, _p, _c_int, _c_int, _c_i64,
                                           _c_i64, _c_int, _c_int, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p]),
    "lamq_ldlq_trellis16_block_workspace_size": (ctypes.c_size_t, [_c_i64, _c_int, _c_int]),
    "lamq_ldlq_trellis16_block_ws": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _p, _p, _c_int, _c_int, _c_i64,
                                              _c_i64, _c_int, _c_int, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p,
                                              ctypes.c_size_t, _p]),
    "lamq_ldlq_trellis16_block_groups": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _c_int, _p, _c_int,
                                                  _c_i64, _c_i64, _c_int, _c_int, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p]),
    "lamq_ldlq_trellis_block_groups": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _c_int, _p, _c_int, _c_i64,
                                                _c_i64, _c_int, _c_int, _p, _p, _c_i64, _p, _c_i64, _c_i64, _p]),
    "lamq_trailing_update_f64": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _c_i64, _c_i64, _c_i64, _p]),
    "lamq_gemm_sub_f64": (_c_int, [_p, _c_i64, _p, _c_i64, _p, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _p]),
    "lamq_refit_step": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _c_i64, _c_i64, _c_int, _c_i64, _c_i64, _p,
                                 _c_i64, _p]),
    "lamq_zero_columns": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _p]),
    "lamq_chol_inv_upper_workspace_size": (_c_size, [_c_i64]),
    "lamq_chol_inv_upper": (_c_int, [_p, _c_i64, _c_i64, _c_dbl, _p, _c_i64, _p, _c_i64, _p, _p, _p, _c_size, _p]),
    "lamq_chol_inv_upper_ex": (_c_int, [_p, _c_i64, _c_i64, _c_dbl, _c_int, _p, _c_i64, _p, _c_i64, _p, _p, _p, _c_size,
                                        _p, _p]),
    "lamq_rht_rows": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p, _p, _c_int, _p, _c_int, _c_int, _p, _p]),
    "lamq_transpose_f64": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_i64, _p]),
    "lamq_row_rms": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _p]),
    "lamq_gram_workspace_size": (_c_size, [_c_i64, _c_i64, _c_int]),
    "lamq_hessian_accum": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _c_flt, _p, _c_i64, _p, _c_size, _p]),
    "lamq_hessian_finalize": (_c_int, [_p, _c_i64, _c_i64, _c_flt, _p, _c_i64, _p]),
    "lamq_cross_gram": (_c_int, [_p, _p, _c_i64, _c_i64, _c_i64, _p, _c_flt, _p, _c_i64, _p, _c_size, _p]),
    "lamq_hessian_accum_rows": (_c_int, [_p, _p, _c_i64, _c_i64, _c_i64, _c_flt, _p, _c_i64, _p, _c_size, _p]),
    "lamq_cross_gram_rows": (_c_int, [_p, _p, _p, _c_i64, _c_i64, _c_i64, _c_flt, _p, _c_i64, _p, _c_size, _p]),
    "lamq_kl_workspace_size": (_c_size, [_c_i64]),
    "lamq_kl_rows": (_c_int, [_p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _p, _p, _p, _c_size, _p]),
    "lamq_kl_rows_f32": (_c_int, [_p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _p, _p, _p, _c_size, _p]),
    "lamq_kl_rows_noalloc": (_c_int, [_p, _p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _p, _p, _p]),
    "lamq_pack_trellis": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _c_int, _c_int, _p, _c_i64, _p, _p]),
    "lamq_pack_codes": (_c_int, [_p, _c_i64, _c_i64, _p, _c_i64, _c_i64, _c_int, _c_int, _c_int, _c_int, _p, _c_i64, _p, _p]),
    "lamq_pack_codes_groups": (_c_int, [_p, _c_int, _c_i64, _c_int, _c_int, _p, _p]),
    "lamq_shaping_feedback_size": (_c_size, [_c_i64, _c_int]),
    "lamq_shaping_feedback": (_c_int, [_p, _c_i64, _c_i64, _c_int, _p, _p]),
    "lamq_ldlq_shaped_column": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _c_i64, _p, _c_int, _p, _c_int, _p, _c_i64, _p,
                                         _p]),
    "lamq_causal_softmax_bf16": (_c_int, [_p, _p, _c_i64, _c_int, _c_i64, _c_i64, _c_flt, _p]),
    "lamq_swiglu_bf16": (_c_int, [_p, _p, _p, _c_i64, _p]),
    "lamq_rms_norm_bf16": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _p, _c_i64, _c_flt, _p]),
    "lamq_rms_norm_rope_bf16": (_c_int, [_p, _c_i64, _c_i64, _c_i64, _p, _p, _p, _c_i64, _c_i64, _c_i64, _p, _c_i64,
                                         _c_flt, _p]),
    "lamq_attention_causal_bf16": (_c_int, [_p] + [_c_i64] * 3 + [_p] + [_c_i64] * 3 + [_p] + [_c_i64] * 3 + [_p]
                                   + [_c_i64] * 3 + [_c_i64] * 5 + [_c_flt, _p]),
    "lamq_probe_l2_delivery": (_c_int, [_p, _c_i64, _c_int, _c_int, _p]),
}


class TrellisGroup(ctypes.Structure):
    """lamq_trellis_group of include/lamq.h: one row group of lamq_ldlq_trellis16_block_groups."""

    _fields_ = [("r0", _c_i64), ("rows", _c_i64), ("k", _c_int), ("table64", _p), ("table16", _p), ("workspace", _p),
                ("workspace_bytes", _c_size)]


class TrellisGroup32(ctypes.Structure):
    """lamq_trellis_group32 of include/lamq.h: one row group of lamq_ldlq_trellis_block_groups (L = 12)."""

    _fields_ = [("r0", _c_i64), ("rows", _c_i64), ("k", _c_int), ("table64", _p), ("table32", _p)]


class PackGroup(ctypes.Structure):
    """lamq_pack_group of include/lamq.h: one row group of lamq_pack_codes_groups."""

    _fields_ = [("src", _p), ("ld", _c_i64), ("src_rows", _c_i64), ("rows", _p), ("m", _c_i64), ("base", ctypes.c_int32),
                ("k", _c_int), ("codes", _p), ("ldc", _c_i64)]


_LIB = None


def lib():
    """The loaded library; raises if it was not built (python -m lookatmyquant_amd.build)."""
    global _LIB
    if _LIB is None:
        if not SO.exists():
            raise RuntimeError(f"{SO} is missing: build it with `python -m lookatmyquant_amd.build` (hipcc, gfx950)")
        L = ctypes.CDLL(str(SO))
        for name, (res, args) in SIGNATURES.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _LIB = L
    return _LIB


def check(rc: int, what: str):
    if rc == 0:
        return
    if rc == -1:
        raise ValueError(f"{what}: invalid argument")
    if rc == -2:
        raise NotImplementedError(f"{what}: shape or parameter not supported by the gfx950 kernels")
    raise RuntimeError(f"{what}: HIP error {rc}")


def device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("no ROCm GPU is visible: the lookatmyquant_amd kernels run only on an MI355X (gfx950)")
    return torch.device("cuda", torch.cuda.current_device())


def stream(dev: torch.device | None = None) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def need(t: torch.Tensor, dtype: torch.dtype, name: str, dims: int | None = None):
    if not isinstance(t, torch.Tensor) or t.dtype != dtype or not t.is_cuda:
        raise ValueError(f"{name} must be a {dtype} tensor on the GPU")
    if dims is not None and t.dim() != dims:
        raise ValueError(f"{name} must have {dims} dimensions")
    if t.dim() >= 1 and t.stride(-1) != 1:
        raise ValueError(f"{name} must have unit stride in its last dimension")
    if t.dim() == 2 and t.shape[0] > 1 and t.stride(0) < t.shape[1]:
        raise ValueError(f"{name}: overlapping rows")


def ld(t: torch.Tensor) -> int:
    return t.stride(0) if t.dim() == 2 else t.shape[-1]


def workspace(nbytes: int, dev: torch.device) -> torch.Tensor | None:
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=dev) if nbytes else None
