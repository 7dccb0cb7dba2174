"""GPU parity of sf_attn_fwd with fp16 and fp32 Q/K/V against the CPU oracle.

The reference dispatches fp16 (its default compute dtype, config.h:57) to
flash attention and fp32 to its naive kernel (attention.cu:183-197); here
fp16 runs the 16-bit MFMA kernels with the fp16 instruction for S = K.Q^T
(V needs no conversion) and fp32 runs a kernel on the fp32 MFMA.  Inputs are
N(0,1) from the oracle's generator, rounded to the input type; the oracle
receives the same rounded values.

Tolerances (fp32 output): fp16 inputs with the default P.V form (P rounded
to fp16) max-abs <= 2e-2 and mean-rel <= 1e-3, the exact form (P as an fp16
hi/lo pair) mean-rel <= 2e-5; fp32 inputs (no rounding below fp32 anywhere)
max-abs <= 1e-4 and mean-rel <= 1e-5.
"""
import numpy as np
import pytest
import torch

from _util import assert_close_bf16, mean_rel
from oracle import oracle as O
from servoflow_amd.attention import attention

pytestmark = pytest.mark.gpu
DEV = "cuda"


def f16r(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


def inputs(seed, B, H, Sq, Sk, dt):
    rnd = f16r if dt == torch.float16 else (lambda x: np.asarray(x, np.float32))
    q = rnd(O.randn(seed, (B, H, Sq, 64)))
    k = rnd(O.randn(seed + 1, (B, H, Sk, 64)))
    v = rnd(O.randn(seed + 2, (B, H, Sk, 64)))
    return q, k, v


def run(q, k, v, dt, out_dtype=torch.float32, valid=None, **kw):
    to = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(DEV).to(dt)  # noqa: E731
    vl = torch.from_numpy(np.asarray(valid, np.int32)).to(DEV) if valid is not None else None
    print(f"attention dtype={dt} q{q.shape} k{k.shape} valid={valid} {kw}", flush=True)
    out = attention(to(q), to(k), to(v), out_dtype=out_dtype, valid_len=vl, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def check_f32(got, ref, what):
    mx = float(np.abs(got - ref).max())
    mr = mean_rel(got, ref)
    print(f"{what}: max-abs {mx:.2e} mean-rel {mr:.2e}")
    assert np.isfinite(got).all(), what
    assert mx <= 1e-4 and mr <= 1e-5, f"{what}: max-abs {mx:.3e}, mean-rel {mr:.3e}"


def check_f16_exact(got, ref, what):
    mr = mean_rel(got, ref)
    print(f"{what}: mean-rel {mr:.2e}")
    assert_close_bf16(got, ref, what)
    assert mr <= 2e-5, f"{what}: mean-rel {mr:.3e}"


# ---- configuration 1: self-attention 1 x 32 x 67 x 67 -------------------------

def test_self_attention_fp32_config1():
    q, k, v = inputs(201, 1, 32, 67, 67, torch.float32)
    check_f32(run(q, k, v, torch.float32), O.attention_f32(q, k, v), "self fp32")


def test_self_attention_fp16():
    q, k, v = inputs(211, 1, 32, 67, 67, torch.float16)
    check_f16_exact(run(q, k, v, torch.float16), O.attention_f32(q, k, v), "self fp16")


# ---- configuration 2: cross-attention, image and language keys ---------------

@pytest.mark.parametrize("exact", [False, True])
def test_cross_image_fp16_b1(exact):
    q, k, v = inputs(221, 1, 32, 67, 4374, torch.float16)
    got = run(q, k, v, torch.float16, exact_pv=exact)
    ref = O.attention_f32(q, k, v)
    if exact:
        check_f16_exact(got, ref, "img fp16 exact")
    else:
        assert_close_bf16(got, ref, "img fp16")


def test_cross_image_fp32_b1():
    q, k, v = inputs(231, 1, 32, 67, 4374, torch.float32)
    check_f32(run(q, k, v, torch.float32), O.attention_f32(q, k, v), "img fp32")


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_cross_language_valid_len_b8(dt):
    q, k, v = inputs(241, 8, 32, 67, 1024, dt)
    vl = np.random.default_rng(9).integers(32, 1025, size=8).astype(np.int32)
    got = run(q, k, v, dt, valid=vl)
    ref = O.attention_f32(q, k, v, valid_len=vl)
    if dt == torch.float32:
        check_f32(got, ref, "lang fp32 B=8")
    else:
        assert_close_bf16(got, ref, "lang fp16 B=8")


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_cross_image_b8_all_elements(dt):
    q, k, v = inputs(251, 8, 32, 67, 4374, dt)
    got = run(q, k, v, dt)
    for b in range(8):
        ref = O.attention_f32(q[b:b + 1], k[b:b + 1], v[b:b + 1])
        if dt == torch.float32:
            check_f32(got[b:b + 1], ref, f"img fp32 B=8 b={b}")
        else:
            assert_close_bf16(got[b:b + 1], ref, f"img fp16 B=8 b={b}")


# ---- fp32 path: split counts, causal, key-padding mask ------------------------

@pytest.mark.parametrize("ns", [1, 3, 16])
def test_fp32_split_count_invariance(ns):
    q, k, v = inputs(261, 1, 8, 67, 1500, torch.float32)
    check_f32(run(q, k, v, torch.float32, num_splits=ns), O.attention_f32(q, k, v), f"fp32 ns={ns}")


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_causal(dt):
    q, k, v = inputs(271, 2, 4, 67, 67, dt)
    got = run(q, k, v, dt, is_causal=True)
    ref = O.attention_f32(q, k, v, causal=True)
    if dt == torch.float32:
        check_f32(got, ref, "causal fp32")
    else:
        check_f16_exact(got, ref, "causal fp16")


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_key_padding_mask_matches_gathered_keys(dt):
    """A boolean key-padding mask equals attention over the kept keys."""
    B, H, Sq, Sk = 2, 4, 67, 700
    q, k, v = inputs(281, B, H, Sq, Sk, dt)
    rng = np.random.default_rng(3)
    keep = rng.random((B, Sk)) < 0.6
    pad = (Sk + 3) & ~3
    m = np.zeros((B, pad), np.uint8)
    m[:, :Sk] = keep
    mask = torch.from_numpy(m).to(DEV)[:, :Sk]
    got = run(q, k, v, dt, kv_mask=mask)
    for b in range(B):
        idx = np.nonzero(keep[b])[0]
        ref = O.attention_f32(q[b:b + 1], k[b:b + 1][:, :, idx], v[b:b + 1][:, :, idx])
        if dt == torch.float32:
            check_f32(got[b:b + 1], ref, f"mask fp32 b={b}")
        else:
            assert_close_bf16(got[b:b + 1], ref, f"mask fp16 b={b}")


def within_one_ulp(lo, rounded, mant_bits, what):
    """lo (a narrow output) is the fp32 output rounded: equal in nearly every
    element and never more than one unit in the last place apart (the two
    launches may contract the final scaling differently)."""
    ulp = np.abs(rounded) * 2.0 ** -mant_bits + 2.0 ** -24
    assert np.all(np.abs(lo - rounded) <= ulp), what
    assert np.mean(lo == rounded) > 0.99, what


def test_fp16_output_is_rounded_fp32_output():
    q, k, v = inputs(291, 1, 32, 67, 4374, torch.float16)
    f32 = run(q, k, v, torch.float16, out_dtype=torch.float32)
    f16 = run(q, k, v, torch.float16, out_dtype=torch.float16)
    within_one_ulp(f16, f16r(f32), 10, "fp16 out")


def test_fp32_output_kinds_agree():
    """bf16 and fp16 outputs of the fp32 kernel are its fp32 output rounded."""
    q, k, v = inputs(301, 1, 8, 67, 300, torch.float32)
    f32 = run(q, k, v, torch.float32, out_dtype=torch.float32)
    f16 = run(q, k, v, torch.float32, out_dtype=torch.float16)
    b16 = run(q, k, v, torch.float32, out_dtype=torch.bfloat16)
    within_one_ulp(f16, f16r(f32), 10, "fp16 out of fp32 in")
    within_one_ulp(b16, O.bf16_round(f32), 7, "bf16 out of fp32 in")
