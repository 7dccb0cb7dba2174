"""Torch-tensor front end for `sf_attn_fwd` (tests and bench plumbing).

torch supplies device memory and the current HIP stream; the arithmetic runs
in libsf_hip_kernels.so.  Mirrors IBackend::attention
(include/servoflow/backend/backend.h:105-110): Q [B,H,Sq,D], K/V [B,H,Sk,D],
out [B,H,Sq,D] (or any strided view with a contiguous head dim), mask
semantics as documented on `sf_attn_desc`.
"""
from __future__ import annotations

import ctypes

import torch

from . import abi

_DT = {torch.bfloat16: abi.SF_BF16, torch.float32: abi.SF_F32, torch.float16: abi.SF_F16}


def _strides3(t: torch.Tensor):
    if t.dim() != 4 or t.stride(3) != 1:
        raise ValueError("expected a 4-D tensor [B,H,S,D] with a contiguous last dim")
    return (t.stride(0), t.stride(1), t.stride(2))


def make_desc(q, k, v, out, scale=0.0, is_causal=False, valid_len=None, num_splits=0, kv_mask=None,
              exact_pv=False, q_gamma=None, k_gamma=None, qk_eps=1e-6):
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    if k.shape != (B, H, Sk, D) or v.shape != (B, H, Sk, D) or out.shape != (B, H, Sq, D):
        raise ValueError(f"shape mismatch q{tuple(q.shape)} k{tuple(k.shape)} "
                         f"v{tuple(v.shape)} out{tuple(out.shape)}")
    d = abi.AttnDesc()
    d.B, d.H, d.Sq, d.Sk, d.D = B, H, Sq, Sk, D
    d.scale = float(scale)
    d.in_dtype = _DT[k.dtype]
    if q.dtype == torch.float16 and k.dtype == torch.bfloat16:   # fp16 Q rows against bf16 K
        d.q_f16 = 1
    elif q.dtype != k.dtype:
        raise ValueError(f"dtypes q {q.dtype} k {k.dtype}: K must match Q (or Q fp16 with bf16 K)")
    if v.dtype == torch.float16 and k.dtype == torch.bfloat16:   # fp16 V against bf16 K (fp16 P.V form)
        d.v_f16 = 1
    elif v.dtype != k.dtype:
        raise ValueError(f"dtypes k {k.dtype} v {v.dtype}: V must match K (or V fp16 with bf16 K)")
    d.out_dtype = _DT[out.dtype]
    d.is_causal = 1 if is_causal else 0
    d.num_splits = int(num_splits)
    if valid_len is not None:
        if valid_len.dtype != torch.int32 or valid_len.numel() != B or not valid_len.is_cuda:
            raise ValueError("valid_len must be a device int32 tensor of B elements")
        d.kv_valid_len = valid_len.data_ptr()
    if kv_mask is not None:
        if kv_mask.dtype not in (torch.bool, torch.uint8) or kv_mask.dim() != 2 or \
                kv_mask.shape[0] != B or kv_mask.shape[1] != Sk or kv_mask.stride(1) != 1 or not kv_mask.is_cuda:
            raise ValueError("kv_mask must be a device bool/uint8 tensor [B, Sk] with contiguous rows")
        d.kv_mask = kv_mask.data_ptr()
        d.kv_mask_stride = kv_mask.stride(0)
    d.exact_pv = 1 if exact_pv else 0
    for name, gm in (("q_gamma", q_gamma), ("k_gamma", k_gamma)):
        if gm is not None:
            if gm.dtype != torch.float32 or gm.numel() != D or not gm.is_cuda or not gm.is_contiguous():
                raise ValueError(f"{name} must be a contiguous device float32 tensor of D elements")
            setattr(d, name, gm.data_ptr())
    d.q_eps = float(qk_eps)
    for name, t in (("q_stride", q), ("k_stride", k), ("v_stride", v), ("o_stride", out)):
        getattr(d, name)[:] = _strides3(t)
    return d


def workspace_bytes(desc) -> int:
    return int(abi.lib().sf_attn_workspace_bytes(ctypes.byref(desc)))


def attention(q, k, v, out=None, scale=0.0, is_causal=False, valid_len=None, num_splits=0,
              out_dtype=None, workspace=None, stream=None, kv_mask=None, exact_pv=False,
              q_gamma=None, k_gamma=None, qk_eps=1e-6):
    """Runs sf_attn_fwd on torch's current stream (or `stream`) and returns `out`.
    kv_mask: optional device bool [B, Sk] key-padding mask (True = attend);
    its rows must be readable for Sk rounded up to 4 bytes.
    exact_pv: bf16 V and P as a bf16 (hi, lo) pair instead of the fp16 P.V
    contraction (which converts V exactly for 2^-14 <= |V| < 2^16, to within
    2^-25 below; a larger element makes its output column inf/NaN; see
    sf_attn_desc).
    q_gamma / k_gamma: optional float32 [D] weights of a per-head RMSNorm
    (epsilon qk_eps) applied to each Q / K row as it is loaded (bf16 or fp16
    inputs; K only for key sets of at most 128).  An fp16 q with bf16 k and
    v runs the bf16 contraction on Q rounded to bf16 after its norm
    (sf_attn_desc.q_f16).  An fp16 v with bf16 q / k runs the fp16 P.V
    form on V as given (sf_attn_desc.v_f16)."""
    if out is None:
        od = out_dtype or q.dtype
        out = torch.empty(q.shape, dtype=od, device=q.device)
    desc = make_desc(q, k, v, out, scale, is_causal, valid_len, num_splits, kv_mask, exact_pv,
                     q_gamma, k_gamma, qk_eps)
    need = workspace_bytes(desc)
    if need and workspace is None:
        workspace = torch.empty(need, dtype=torch.uint8, device=q.device)   # needs no init
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_n = workspace.numel() * workspace.element_size() if workspace is not None else 0
    s = stream if stream is not None else torch.cuda.current_stream(q.device)
    st = abi.lib().sf_attn_fwd(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                               out.data_ptr(), ws_ptr, ws_n, s.cuda_stream)
    abi.check(st, "sf_attn_fwd")
    return out
