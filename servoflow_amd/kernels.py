"""Torch-tensor front ends for sf_gemm, sf_rmsnorm, sf_add_rmsnorm and
sf_dequant_int8 (test and bench plumbing: torch supplies device memory and
the stream; the arithmetic runs in libsf_hip_kernels.so)."""
from __future__ import annotations

import ctypes

import torch

from . import abi

_DT = {torch.bfloat16: abi.SF_BF16, torch.float32: abi.SF_F32, torch.float16: abi.SF_F16, torch.int8: abi.SF_I8}


def _stream(t):
    return torch.cuda.current_stream(t.device).cuda_stream


def _p(t):
    return None if t is None else t.data_ptr()


def _desc(a, w, bias, act, w_scale):
    M, K = a.shape
    d = abi.GemmDesc()
    d.M, d.N, d.K = M, w.shape[0], K
    d.A, d.lda, d.a_dtype = a.data_ptr(), a.stride(0), _DT[a.dtype]
    d.W, d.ldw, d.w_dtype = w.data_ptr(), w.stride(0), _DT[w.dtype]
    d.w_scale = _p(w_scale)
    d.bias = _p(bias)
    d.act = act
    return d


def _run(d, a, workspace):
    """workspace: "auto" allocates what the split-K path needs, None runs the
    single-pass path, a tensor is used as given."""
    if isinstance(workspace, str):
        nbytes = abi.lib().sf_gemm_workspace_bytes(ctypes.byref(d))
        workspace = torch.empty(max(nbytes, 16), dtype=torch.uint8, device=a.device) if nbytes else None
    if workspace is not None:
        d.workspace, d.workspace_bytes = workspace.data_ptr(), workspace.numel() * workspace.element_size()
    abi.check(abi.lib().sf_gemm(ctypes.byref(d), _stream(a)), "sf_gemm")


def workspace_bytes(a, w):
    d = _desc(a, w, None, 0, None)
    return abi.lib().sf_gemm_workspace_bytes(ctypes.byref(d))


def _row_scale(d, row_ss, row_n, row_eps):
    """The activation rows are x * gamma of a deferred RMSNorm with tile sums
    row_ss ([row_n / 64, M] fp32)."""
    if row_ss is not None:
        d.a_row_ss, d.a_row_tiles, d.a_row_n, d.a_row_eps = row_ss.data_ptr(), row_ss.shape[0], row_n, row_eps


def _w16(d, w16):
    """An fp16 copy of the weights (weights_to_f16) for the library path."""
    if w16 is not None:
        d.w_codes16, d.w16_f16 = w16.data_ptr(), 1


def gemm(a, w, bias=None, act=abi.SF_ACT_NONE, out=None, out_dtype=torch.bfloat16,
         accumulate=False, w_scale=None, workspace="auto", w_codes16=None, w16=None, row_ss=None, row_n=0,
         row_eps=1e-6):
    """out[M,N] = act(a[M,K] w[N,K]^T + bias) (bf16 a; bf16 or int8 w with
    per-row fp32 w_scale).  accumulate adds into an fp32 `out`.  w_codes16:
    int8 w's codes as bf16 (int8_codes_to_bf16), read by the library path
    instead of widening them.  w16: an fp16 copy of w (weights_to_f16) for
    fp16 `a`: the library path then multiplies in fp16.  int8 w without a
    copy above 160 rows is read directly when the call fits
    (sf_gemm_int8_direct: K = 2048, N % 256 == 0, fp16 a and out)."""
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty(M, N, dtype=out_dtype, device=a.device)
    d = _desc(a, w, bias, act, w_scale)
    d.w_codes16 = _p(w_codes16)
    _w16(d, w16)
    _row_scale(d, row_ss, row_n, row_eps)
    d.epilogue = abi.SF_EPI_PLAIN
    d.C, d.ldc, d.c_dtype = out.data_ptr(), out.stride(0), _DT[out.dtype]
    d.accumulate = 1 if accumulate else 0
    _run(d, a, workspace)
    return out


def gemm_add_norm(a, w, bias, residual, gamma, eps=1e-6, act=abi.SF_ACT_NONE, w_scale=None,
                  norm_dtype=torch.bfloat16, workspace="auto", round_product=False, w16=None, norm_ss=None):
    """residual (fp32 [M,N]) += act(a w^T + bias); returns
    rmsnorm(residual) * gamma in norm_dtype.  round_product: above 160 rows
    the branch output is stored in 16 bits before the add (bf16, or fp16
    with w16)."""
    M = a.shape[0]
    N = w.shape[0]
    out = torch.empty(M, N, dtype=norm_dtype, device=a.device)
    d = _desc(a, w, bias, act, w_scale)
    _w16(d, w16)
    d.epilogue = abi.SF_EPI_ADD_NORM
    d.C, d.ldc, d.c_dtype = residual.data_ptr(), residual.stride(0), abi.SF_F32
    d.eps = eps
    d.norm_gamma, d.norm_out = gamma.data_ptr(), out.data_ptr()
    d.norm_ldo, d.norm_dtype = out.stride(0), _DT[norm_dtype]
    d.round_product = 1 if round_product else 0
    if norm_ss is not None:   # deferred form: out = residual * gamma, tile sums of squares to norm_ss
        d.norm_ss = norm_ss.data_ptr()
    _run(d, a, workspace)
    return out


def gemm_heads(a, w, bias, S, H, outs, gammas=(None, None, None), eps=1e-6, w_scale=None,
               workspace="auto", round_product=False, w16=None, row_ss=None, row_n=0, row_eps=1e-6):
    """Projection whose N columns are sections of H*64, written per head to
    outs[j] ([B,H,S,64] bf16 views) with optional per-head RMSNorm.
    round_product: above 160 rows the projection is stored in 16 bits
    before the norm (bf16, or fp16 with w16 or with int8 w multiplied
    directly, sf_gemm_int8_direct)."""
    d = _desc(a, w, bias, abi.SF_ACT_NONE, w_scale)
    _w16(d, w16)
    _row_scale(d, row_ss, row_n, row_eps)
    d.epilogue = abi.SF_EPI_HEADS
    d.H, d.S, d.eps = H, S, eps
    d.round_product = 1 if round_product else 0
    for j, o in enumerate(outs):
        d.head_out[j] = o.data_ptr()
        d.head_gamma[j] = _p(gammas[j])
        d.head_stride[j][:] = (o.stride(0), o.stride(1), o.stride(2))
    _run(d, a, workspace)
    return outs


def int8_codes_to_bf16(qs):
    """bf16 copies [N][K] of the codes of int8 matrices (row-strided views
    allowed), all in one launch (at most abi.SF_CODES_MAX_JOBS)."""
    outs = [torch.empty(q.shape[0], q.shape[1], dtype=torch.bfloat16, device=q.device) for q in qs]
    jobs = (abi.CodesJob * max(1, len(qs)))()
    for j, (q, o) in enumerate(zip(qs, outs)):
        jobs[j].q, jobs[j].ldq, jobs[j].out = q.data_ptr(), q.stride(0), o.data_ptr()
        jobs[j].N, jobs[j].K = q.shape[0], q.shape[1]
    st = abi.lib().sf_int8_codes_to_bf16(jobs, len(qs), _stream(qs[0]) if qs else None)
    abi.check(st, "sf_int8_codes_to_bf16")
    return outs


def weights_to_f16(ws):
    """fp16 copies [N][K] of bf16 or int8 (codes) matrices, one launch (at
    most abi.SF_CODES_MAX_JOBS)."""
    outs = [torch.empty(w.shape[0], w.shape[1], dtype=torch.float16, device=w.device) for w in ws]
    jobs = (abi.W16Job * max(1, len(ws)))()
    for j, (w, o) in enumerate(zip(ws, outs)):
        jobs[j].w, jobs[j].w_dtype, jobs[j].ldw = w.data_ptr(), _DT[w.dtype], w.stride(0)
        jobs[j].out, jobs[j].N, jobs[j].K = o.data_ptr(), w.shape[0], w.shape[1]
    abi.check(abi.lib().sf_weights_to_f16(jobs, len(ws), _stream(ws[0]) if ws else None), "sf_weights_to_f16")
    return outs


def rmsnorm_deferred(x, gamma, out_dtype=torch.bfloat16):
    """sf_rmsnorm_deferred on fp32 rows x [rows, cols]: (x * gamma in
    out_dtype, tile sums of squares [cols / 64, rows] fp32)."""
    rows, cols = x.shape
    out = torch.empty(rows, cols, dtype=out_dtype, device=x.device)
    ss = torch.empty(cols // 64, rows, dtype=torch.float32, device=x.device)
    st = abi.lib().sf_rmsnorm_deferred(x.data_ptr(), x.stride(0), gamma.data_ptr(), out.data_ptr(), _DT[out_dtype],
                                       out.stride(0), ss.data_ptr(), rows, cols, _stream(x))
    abi.check(st, "sf_rmsnorm_deferred")
    return out, ss


def rmsnorm(x, gamma, eps=1e-6, out_dtype=torch.bfloat16, out=None):
    rows, cols = x.shape
    if out is None:
        out = torch.empty(rows, cols, dtype=out_dtype, device=x.device)
    st = abi.lib().sf_rmsnorm(x.data_ptr(), _DT[x.dtype], x.stride(0), gamma.data_ptr(),
                              out.data_ptr(), _DT[out.dtype], out.stride(0), rows, cols, eps,
                              _stream(x))
    abi.check(st, "sf_rmsnorm")
    return out


def add_rmsnorm(delta, residual, gamma, eps=1e-6, out_dtype=torch.bfloat16):
    rows, cols = residual.shape
    out = torch.empty(rows, cols, dtype=out_dtype, device=residual.device)
    st = abi.lib().sf_add_rmsnorm(delta.data_ptr(), _DT[delta.dtype], residual.data_ptr(),
                                  gamma.data_ptr(), out.data_ptr(), _DT[out.dtype], rows, cols,
                                  eps, _stream(residual))
    abi.check(st, "sf_add_rmsnorm")
    return out


def dequant_int8(q, scale, per_channel=True, out_dtype=torch.float32):
    N = q.shape[0]
    K = q.numel() // max(N, 1)
    out = torch.empty(q.shape, dtype=out_dtype, device=q.device)
    st = abi.lib().sf_dequant_int8(q.data_ptr(), scale.data_ptr(), 1 if per_channel else 0,
                                   out.data_ptr(), _DT[out_dtype], N, K, _stream(q))
    abi.check(st, "sf_dequant_int8")
    return out
