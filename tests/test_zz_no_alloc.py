"""sf_attn_fwd_noalloc (the allocation-free attention entry point) against
sf_attn_fwd with a caller workspace, through the C-ABI.

Both run the same kernels with the same key split, so the outputs must be
bit-identical.  Two calls in a row on the shared scratch, the second smaller,
then a forced split count whose partials exceed the scratch (rejected with
SF_ESCRATCH before any launch)."""
import ctypes

import pytest
import torch

from servoflow_amd import abi
from servoflow_amd.attention import attention, make_desc

pytestmark = pytest.mark.gpu


def _rand(shape, seed, dev):
    g = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn(shape, generator=g).to(dev).to(torch.bfloat16)


def _noalloc(q, k, v, out, **kw):
    desc = make_desc(q, k, v, out, **kw)
    st = abi.lib().sf_attn_fwd_noalloc(ctypes.byref(desc), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                       out.data_ptr(), torch.cuda.current_stream().cuda_stream)
    return st, desc


def _case(B, Sk, seed, valid=None, out_dtype=torch.float32):
    dev = torch.device("cuda:0")
    H, Sq, D = 32, 67, 64
    q = _rand((B, H, Sq, D), seed, dev)
    k = _rand((B, H, Sk, D), seed + 1, dev)
    v = _rand((B, H, Sk, D), seed + 2, dev)
    vl = torch.tensor(valid, dtype=torch.int32, device=dev) if valid is not None else None
    ref = attention(q, k, v, valid_len=vl, out_dtype=out_dtype)
    got = torch.full_like(ref, float("nan"))
    print(f"noalloc case B={B} Sk={Sk} valid={valid}", flush=True)
    st, desc = _noalloc(q, k, v, got, valid_len=vl)
    abi.check(st, "sf_attn_fwd_noalloc")
    torch.cuda.synchronize()
    return ref, got, desc


def test_noalloc_matches_workspace_entry_point_twice():
    # first call: image keys at batch 1 (7 key splits: the scratch is used)
    ref1, got1, d1 = _case(1, 4374, 10)
    n1 = abi.lib().sf_attn_workspace_bytes(ctypes.byref(d1))
    assert 0 < n1 <= abi.SF_ATTN_NOALLOC_SCRATCH_BYTES
    assert torch.equal(got1, ref1)
    # second call, smaller: 1100 keys with a valid length (5 key splits,
    # fewer partial rows than the first call left in the scratch)
    ref2, got2, d2 = _case(1, 1100, 20, valid=[800], out_dtype=torch.bfloat16)
    n2 = abi.lib().sf_attn_workspace_bytes(ctypes.byref(d2))
    assert 0 < n2 < n1
    assert torch.equal(got2, ref2)
    # and the first shape again after the smaller one
    ref3, got3, _ = _case(1, 4374, 30)
    assert torch.equal(got3, ref3)


def test_noalloc_rejects_partials_beyond_scratch():
    dev = torch.device("cuda:0")
    B, H, Sq, Sk, D = 4, 32, 67, 4374, 64
    q = torch.zeros((B, H, Sq, D), dtype=torch.bfloat16, device=dev)
    k = torch.zeros((B, H, Sk, D), dtype=torch.bfloat16, device=dev)
    out = torch.full((B, H, Sq, D), 7.0, dtype=torch.float32, device=dev)
    desc = make_desc(q, k, k, out, num_splits=32)
    assert abi.lib().sf_attn_workspace_bytes(ctypes.byref(desc)) > abi.SF_ATTN_NOALLOC_SCRATCH_BYTES
    st, _ = _noalloc(q, k, k, out, num_splits=32)
    assert st == abi.SF_ESCRATCH
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())   # nothing was launched
