"""numpy front end for oracle/_build/libsf_oracle.so.

TEST INFRASTRUCTURE ONLY: the CPU checker for the MI355X kernels.  Only
tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import it.
Each wrapper names the reference file:line its C function restates.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "libsf_oracle.so")

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} missing: run `make -C oracle`")
    L = ctypes.CDLL(LIB_PATH)
    i32, i64, f32 = ctypes.c_int, ctypes.c_int64, ctypes.c_float
    L.sfo_randn.argtypes = [ctypes.c_uint64, i64, f32, _f32p]
    L.sfo_bf16_round.argtypes = [f32]
    L.sfo_bf16_round.restype = f32
    L.sfo_bf16_round_array.argtypes = [_f32p, i64]
    L.sfo_attention_f32.argtypes = [_f32p, _f32p, _f32p, _f32p] + [i32] * 5 + [f32, i32, _vp]
    L.sfo_attention_f64.argtypes = [_f32p, _f32p, _f32p, _f64p] + [i32] * 5 + [ctypes.c_double, i32, _vp]
    L.sfo_rms_norm.argtypes = [_f32p, _f32p, _f32p, i64, i64, f32]
    L.sfo_fused_add_rms_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, i64, i64, f32]
    L.sfo_gelu_tanh.argtypes = [f32]
    L.sfo_gelu_tanh.restype = f32
    L.sfo_silu.argtypes = [f32]
    L.sfo_silu.restype = f32
    L.sfo_linear.argtypes = [_f32p, _f32p, _vp, _f32p, i64, i64, i64, i32]
    L.sfo_split_qkv.argtypes = [_f32p] * 4 + [i32] * 4
    L.sfo_split_kv.argtypes = [_f32p] * 3 + [i32] * 4
    L.sfo_seq_to_head.argtypes = [_f32p, _f32p] + [i32] * 4
    L.sfo_head_to_seq.argtypes = [_f32p, _f32p] + [i32] * 4
    L.sfo_dequant_int8.argtypes = [_i8p, _f32p, _f32p, i64, i64, i32]
    L.sfo_quantize_int8_rows.argtypes = [_f32p, i64, i64, _i8p, _f32p]
    L.sfo_linspace.argtypes = [i32, f32, f32, _f32p]
    L.sfo_sincos_table.argtypes = [i32, i32, _f32p]
    L.sfo_timestep_index.argtypes = [f32, i32]
    L.sfo_timestep_index.restype = i32
    _lib = L
    return L


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def randn(seed: int, shape, std: float = 1.0) -> np.ndarray:
    """SplitMix64 -> Box-Muller N(0, std^2) (the build's deterministic inputs)."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().sfo_randn(seed & 0xFFFFFFFFFFFFFFFF, n, std, out)
    return out.reshape(shape)


def bf16_round(a: np.ndarray) -> np.ndarray:
    out = _c32(a).copy()
    lib().sfo_bf16_round_array(out, out.size)
    return out


def attention_f32(q, k, v, scale=0.0, causal=False, valid_len=None):
    """naive_attention_kernel, src/backend/cuda/ops/attention.cu:90-139."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    out = np.empty((B, H, Sq, D), dtype=np.float32)
    vl = None
    if valid_len is not None:
        vl_arr = np.ascontiguousarray(valid_len, dtype=np.int32)
        vl = vl_arr.ctypes.data
    lib().sfo_attention_f32(q, k, v, out, B, H, Sq, Sk, D, float(scale), int(causal), vl)
    return out


def attention_f64(q, k, v, scale=0.0, causal=False, valid_len=None):
    """Two-pass fp64 softmax(QK^T*scale)V (independent order, pins attention_f32)."""
    q, k, v = _c32(q), _c32(k), _c32(v)
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    out = np.empty((B, H, Sq, D), dtype=np.float64)
    vl = None
    if valid_len is not None:
        vl_arr = np.ascontiguousarray(valid_len, dtype=np.int32)
        vl = vl_arr.ctypes.data
    lib().sfo_attention_f64(q, k, v, out, B, H, Sq, Sk, D, float(scale), int(causal), vl)
    return out


def rms_norm(x, gamma, eps=1e-6):
    """rms_norm_kernel_impl, src/backend/cuda/ops/norm.cuh:89-122 (last dim)."""
    x = _c32(x)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().sfo_rms_norm(x, _c32(gamma), out, x.size // cols, cols, eps)
    return out


def fused_add_rms_norm(inp, residual, gamma, eps=1e-6):
    """fused_add_rms_norm_kernel, norm.cuh:130-171; returns (out, new residual)."""
    inp = _c32(inp)
    res = _c32(residual).copy()
    cols = inp.shape[-1]
    out = np.empty_like(inp)
    lib().sfo_fused_add_rms_norm(inp, res, _c32(gamma), out, inp.size // cols, cols, eps)
    return out, res


def gelu_tanh(x: float) -> float:
    return lib().sfo_gelu_tanh(x)


def silu(x: float) -> float:
    return lib().sfo_silu(x)


def linear(x, W, bias=None, act=0):
    """y = act(x W^T + b): gemm_bias_act, cuda_backend.cu:246-285,337-467."""
    x = _c32(x)
    W = _c32(W)
    K = x.shape[-1]
    M = x.size // K
    N = W.shape[0]
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    b = _c32(bias) if bias is not None else None
    lib().sfo_linear(x, W, b.ctypes.data if b is not None else None, y, M, N, K, act)
    return y


def split_qkv(qkv, H, D):
    qkv = _c32(qkv)
    B, S, _ = qkv.shape
    Q, K, V = (np.empty((B, H, S, D), np.float32) for _ in range(3))
    lib().sfo_split_qkv(qkv, Q, K, V, B, S, H, D)
    return Q, K, V


def split_kv(kv, H, D):
    kv = _c32(kv)
    B, S, _ = kv.shape
    K, V = (np.empty((B, H, S, D), np.float32) for _ in range(2))
    lib().sfo_split_kv(kv, K, V, B, S, H, D)
    return K, V


def seq_to_head(x, H, D):
    x = _c32(x)
    B, S, _ = x.shape
    out = np.empty((B, H, S, D), np.float32)
    lib().sfo_seq_to_head(x, out, B, S, H, D)
    return out


def head_to_seq(x):
    x = _c32(x)
    B, H, S, D = x.shape
    out = np.empty((B, S, H * D), np.float32)
    lib().sfo_head_to_seq(x, out, B, H, S, D)
    return out


def dequant_int8(q, scale, per_channel=True):
    """dequantize_int8_fp16_kernel index math, quantization.cu:18-51."""
    q = np.ascontiguousarray(q, dtype=np.int8)
    N = q.shape[0]
    K = q.size // N
    out = np.empty(q.shape, np.float32)
    lib().sfo_dequant_int8(q, _c32(scale), out, N, K, int(per_channel))
    return out


def quantize_int8_rows(W):
    W = _c32(W)
    N, K = W.shape
    q = np.empty((N, K), np.int8)
    s = np.empty(N, np.float32)
    lib().sfo_quantize_int8_rows(W, N, K, q, s)
    return q, s


def linspace(num_steps, t_start=1.0, t_end=0.0):
    """Schedule::linspace, src/sampling/flow_matching.cpp:10-17."""
    out = np.empty(num_steps + 1, np.float32)
    lib().sfo_linspace(num_steps, t_start, t_end, out)
    return out


def sincos_table(max_steps=1000, freq_dim=256):
    """TimestepEmbedding::build_sincos_table, src/models/rdt1b/dit_block.cu:58-72."""
    out = np.empty((max_steps, freq_dim), np.float32)
    lib().sfo_sincos_table(max_steps, freq_dim, out)
    return out


def timestep_index(t, num_train_timesteps=1000):
    """round(t * (T - 1)) clamped, src/models/rdt1b/rdt1b.cpp:312-313."""
    return int(lib().sfo_timestep_index(float(t), num_train_timesteps))
