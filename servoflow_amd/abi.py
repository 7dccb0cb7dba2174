"""ctypes bindings for libsf_hip_kernels.so (the C-ABI declared in include/sf_hip.h).

The library is the product: these bindings only describe its entry points.
Loading raises if the shared object is missing; nothing here computes on the
CPU or falls back to another implementation.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libsf_hip_kernels.so")

SF_OK = 0
SF_EINVAL = -1
SF_ENOTSUP = -2
SF_EWORKSPACE = -3
SF_ELAUNCH = -4
SF_EDEVICE = -5
SF_ESCRATCH = -6
SF_ATTN_NOALLOC_SCRATCH_BYTES = 8 << 20

SF_F32 = 0
SF_F16 = 1
SF_BF16 = 2
SF_I8 = 3
SF_I32 = 5


class AttnDesc(ctypes.Structure):
    """Mirror of `sf_attn_desc`."""

    _fields_ = [
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("Sq", ctypes.c_int32),
        ("Sk", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("in_dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("is_causal", ctypes.c_int32),
        ("num_splits", ctypes.c_int32),
        ("kv_valid_len", ctypes.c_void_p),
        ("q_stride", ctypes.c_int64 * 3),
        ("k_stride", ctypes.c_int64 * 3),
        ("v_stride", ctypes.c_int64 * 3),
        ("o_stride", ctypes.c_int64 * 3),
        ("kv_mask", ctypes.c_void_p),
        ("kv_mask_stride", ctypes.c_int64),
        ("exact_pv", ctypes.c_int32),
        ("q_partials", ctypes.c_void_p),
        ("q_splits", ctypes.c_int32),
        ("q_bias", ctypes.c_void_p),
        ("q_scale", ctypes.c_void_p),
        ("q_gamma", ctypes.c_void_p),
        ("q_eps", ctypes.c_float),
        ("k_gamma", ctypes.c_void_p),
        ("q_f16", ctypes.c_int32),
        ("q_row_ss", ctypes.c_void_p),
        ("q_row_tiles", ctypes.c_int32),
        ("q_row_n", ctypes.c_int32),
        ("q_row_eps", ctypes.c_float),
        ("v_f16", ctypes.c_int32),
    ]


SF_ACT_NONE = 0
SF_ACT_GELU_TANH = 1
SF_ACT_SILU = 2
SF_EPI_PLAIN = 0
SF_EPI_HEADS = 1
SF_EPI_ADD_NORM = 2
SF_EPI_PARTIALS = 3


class GemmDesc(ctypes.Structure):
    """Mirror of `sf_gemm_desc`."""

    _fields_ = [
        ("M", ctypes.c_int32), ("N", ctypes.c_int32), ("K", ctypes.c_int32),
        ("A", ctypes.c_void_p), ("lda", ctypes.c_int64), ("a_dtype", ctypes.c_int32),
        ("W", ctypes.c_void_p), ("ldw", ctypes.c_int64), ("w_dtype", ctypes.c_int32),
        ("w_scale", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("act", ctypes.c_int32),
        ("epilogue", ctypes.c_int32),
        ("C", ctypes.c_void_p), ("ldc", ctypes.c_int64), ("c_dtype", ctypes.c_int32),
        ("accumulate", ctypes.c_int32),
        ("H", ctypes.c_int32), ("S", ctypes.c_int32), ("eps", ctypes.c_float),
        ("head_gamma", ctypes.c_void_p * 3),
        ("head_out", ctypes.c_void_p * 3),
        ("head_stride", (ctypes.c_int64 * 3) * 3),
        ("norm_gamma", ctypes.c_void_p), ("norm_out", ctypes.c_void_p),
        ("norm_ldo", ctypes.c_int64), ("norm_dtype", ctypes.c_int32),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("round_product", ctypes.c_int32),
        ("w_codes16", ctypes.c_void_p),
        ("w16_f16", ctypes.c_int32),
        ("norm_ss", ctypes.c_void_p),
        ("a_row_ss", ctypes.c_void_p),
        ("a_row_tiles", ctypes.c_int32),
        ("a_row_n", ctypes.c_int32),
        ("a_row_eps", ctypes.c_float),
    ]


class CodesJob(ctypes.Structure):
    """Mirror of `sf_codes_job`."""

    _fields_ = [("q", ctypes.c_void_p), ("ldq", ctypes.c_int64), ("out", ctypes.c_void_p),
                ("N", ctypes.c_int32), ("K", ctypes.c_int32)]


SF_CODES_MAX_JOBS = 8


class W16Job(ctypes.Structure):
    """Mirror of `sf_w16_job`."""

    _fields_ = [("w", ctypes.c_void_p), ("w_dtype", ctypes.c_int32), ("ldw", ctypes.c_int64),
                ("out", ctypes.c_void_p), ("N", ctypes.c_int32), ("K", ctypes.c_int32)]


class AbsmaxJob(ctypes.Structure):
    """Mirror of `sf_absmax_job`."""

    _fields_ = [("p", ctypes.c_void_p), ("n", ctypes.c_int64), ("out", ctypes.c_void_p)]


SF_ABSMAX_MAX_JOBS = 64


class SfError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {strerror(status)} (status {status})")
        self.status = status


_lib = None


def lib() -> ctypes.CDLL:
    """Loads libsf_hip_kernels.so once; raises FileNotFoundError if unbuilt."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(
            f"{LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
        )
    L = ctypes.CDLL(LIB_PATH)
    P = ctypes.POINTER(AttnDesc)
    L.sf_attn_desc_init_bhsd.argtypes = [P] + [ctypes.c_int32] * 7
    L.sf_attn_desc_init_bhsd.restype = None
    L.sf_attn_workspace_bytes.argtypes = [P]
    L.sf_attn_workspace_bytes.restype = ctypes.c_size_t
    L.sf_attn_num_splits.argtypes = [P]
    L.sf_attn_num_splits.restype = ctypes.c_int32
    L.sf_attn_fwd.argtypes = [P, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                              ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    L.sf_attn_fwd.restype = ctypes.c_int
    L.sf_attn_fwd_noalloc.argtypes = [P, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                      ctypes.c_void_p, ctypes.c_void_p]
    L.sf_attn_fwd_noalloc.restype = ctypes.c_int
    L.sf_gemm.argtypes = [ctypes.POINTER(GemmDesc), ctypes.c_void_p]
    L.sf_gemm.restype = ctypes.c_int
    L.sf_gemm_workspace_bytes.argtypes = [ctypes.POINTER(GemmDesc)]
    L.sf_gemm_workspace_bytes.restype = ctypes.c_size_t
    L.sf_gemm_prepare.argtypes = [ctypes.POINTER(GemmDesc)]
    L.sf_gemm_prepare.restype = ctypes.c_int
    L.sf_gemm_algo_pick.argtypes = [ctypes.POINTER(GemmDesc), ctypes.POINTER(ctypes.c_int32),
                                    ctypes.POINTER(ctypes.c_int32), ctypes.POINTER(ctypes.c_int32)]
    L.sf_gemm_algo_pick.restype = ctypes.c_int
    vp, i32, i64 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64
    L.sf_rmsnorm.argtypes = [vp, i32, i64, vp, vp, i32, i64, i32, i32, ctypes.c_float, vp]
    L.sf_rmsnorm.restype = ctypes.c_int
    L.sf_rmsnorm_deferred.argtypes = [vp, i64, vp, vp, i32, i64, vp, i32, i32, vp]
    L.sf_rmsnorm_deferred.restype = ctypes.c_int
    L.sf_add_rmsnorm.argtypes = [vp, i32, vp, vp, vp, i32, i32, i32, ctypes.c_float, vp]
    L.sf_add_rmsnorm.restype = ctypes.c_int
    L.sf_dequant_int8.argtypes = [vp, vp, i32, vp, i32, i64, i64, vp]
    L.sf_dequant_int8.restype = ctypes.c_int
    L.sf_int8_codes_to_bf16.argtypes = [ctypes.POINTER(CodesJob), i32, vp]
    L.sf_int8_codes_to_bf16.restype = ctypes.c_int
    L.sf_weights_to_f16.argtypes = [ctypes.POINTER(W16Job), i32, vp]
    L.sf_weights_to_f16.restype = ctypes.c_int
    L.sf_gemm_num_splits.argtypes = [ctypes.POINTER(GemmDesc)]
    L.sf_gemm_num_splits.restype = ctypes.c_int32
    L.sf_gemm_int8_direct.argtypes = [ctypes.POINTER(GemmDesc)]
    L.sf_gemm_int8_direct.restype = ctypes.c_int32
    L.sf_heads_bf16.argtypes = [ctypes.POINTER(GemmDesc), vp, i64, vp]
    L.sf_heads_bf16.restype = ctypes.c_int
    L.sf_absmax_bf16_batched.argtypes = [ctypes.POINTER(AbsmaxJob), i32, vp]
    L.sf_absmax_bf16_batched.restype = ctypes.c_int
    L.sf_bf16_to_f16_below.argtypes = [ctypes.POINTER(AbsmaxJob), i32, ctypes.c_float, vp]
    L.sf_bf16_to_f16_below.restype = ctypes.c_int
    L.sf_gemm_set_algo_timing.argtypes = [i32]
    L.sf_gemm_set_algo_timing.restype = ctypes.c_int
    L.sf_strerror.argtypes = [ctypes.c_int]
    L.sf_strerror.restype = ctypes.c_char_p
    _lib = L
    return L


def strerror(status: int) -> str:
    return lib().sf_strerror(status).decode()


def check(status: int, what: str) -> None:
    if status != SF_OK:
        raise SfError(status, what)


def attn_desc_bhsd(B, H, Sq, Sk, D=64, in_dtype=SF_BF16, out_dtype=SF_BF16) -> AttnDesc:
    d = AttnDesc()
    lib().sf_attn_desc_init_bhsd(ctypes.byref(d), B, H, Sq, Sk, D, in_dtype, out_dtype)
    return d
