"""GPU parity of sf_attn_fwd (libsf_hip_kernels.so) against the CPU oracle.

Inputs are N(0,1) from the oracle's SplitMix64/Box-Muller generator, rounded
to bf16; the oracle receives the same rounded values in fp32.  The kernel's
fp32 output must satisfy max-abs <= 2e-2 and sum|d|/sum|ref| <= 1e-3; its bf16
output must be the fp32 output rounded to nearest (within one bf16 ulp).
Full-size shapes are the benchmarked ops: self-attention 67x67, image
cross-attention 67x4374 and language cross-attention 67x<=1024 with a
per-batch valid length, 32 heads x 64, batch 1 and 8.
"""
import numpy as np
import pytest
import torch

from _util import assert_close_bf16, mean_rel
from oracle import oracle as O
from servoflow_amd import abi
from servoflow_amd.attention import attention, make_desc, workspace_bytes

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rounded(seed, shape, scale=1.0):
    return O.bf16_round(O.randn(seed, shape) * scale)


def to_dev(x, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(x)).to(DEV).to(dtype)


def run(q, k, v, out_dtype=torch.float32, **kw):
    out = attention(to_dev(q), to_dev(k), to_dev(v), out_dtype=out_dtype, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def lang_valid_lengths(seed, B, lo=32, hi=1024):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=B).astype(np.int32)


def test_self_attention_config1():
    q, k, v = (rounded(s, (1, 32, 67, 64)) for s in (101, 102, 103))
    got = run(q, k, v)
    ref = O.attention_f32(q, k, v)
    assert_close_bf16(got, ref, "self 1x32x67x67")


def test_cross_image_b1():
    q = rounded(111, (1, 32, 67, 64))
    k, v = rounded(112, (1, 32, 4374, 64)), rounded(113, (1, 32, 4374, 64))
    got = run(q, k, v)
    assert_close_bf16(got, O.attention_f32(q, k, v), "cross img B=1")


def test_cross_image_b8_all_elements():
    B = 8
    q = rounded(121, (B, 32, 67, 64))
    k, v = rounded(122, (B, 32, 4374, 64)), rounded(123, (B, 32, 4374, 64))
    got = run(q, k, v)
    for b in range(B):
        ref = O.attention_f32(q[b:b + 1], k[b:b + 1], v[b:b + 1])
        assert_close_bf16(got[b:b + 1], ref, f"cross img B=8 b={b}")


@pytest.mark.parametrize("B", [1, 8])
def test_cross_language_valid_len(B):
    q = rounded(131 + B, (B, 32, 67, 64))
    k, v = rounded(132 + B, (B, 32, 1024, 64)), rounded(133 + B, (B, 32, 1024, 64))
    vl = lang_valid_lengths(7 + B, B)
    got = run(q, k, v, valid_len=to_dev(vl, torch.int32))
    ref = O.attention_f32(q, k, v, valid_len=vl)
    assert_close_bf16(got, ref, f"cross lang B={B} valid={vl.tolist()}")
    # masked(valid = L) == attention over K[:L], V[:L] (reference truncation)
    b = int(np.argmin(vl))
    L = int(vl[b])
    trunc = run(q[b:b + 1], k[b:b + 1, :, :L].copy(), v[b:b + 1, :, :L].copy())
    # (the two runs tile the keys differently: equal up to fp16-P rounding;
    # the exact form agrees to ~1e-5)
    assert np.abs(trunc - got[b:b + 1]).max() < 1e-3
    assert mean_rel(trunc, got[b:b + 1]) < 5e-4
    ex = run(q, k, v, valid_len=to_dev(vl, torch.int32), exact_pv=True)[b:b + 1]
    ex_trunc = run(q[b:b + 1], k[b:b + 1, :, :L].copy(), v[b:b + 1, :, :L].copy(), exact_pv=True)
    assert np.abs(ex_trunc - ex).max() < 1e-4


def test_bf16_output_is_rounded_fp32_output():
    q = rounded(141, (1, 32, 67, 64))
    k, v = rounded(142, (1, 32, 4374, 64)), rounded(143, (1, 32, 4374, 64))
    f32 = run(q, k, v, out_dtype=torch.float32)
    b16 = run(q, k, v, out_dtype=torch.bfloat16)
    r = O.bf16_round(f32)
    ulp = np.abs(r) * 2.0 ** -7 + 1e-30
    assert np.all(np.abs(b16 - r) <= ulp)
    assert np.mean(b16 == r) > 0.99


@pytest.mark.parametrize("ns", [1, 3, 16, 40])
def test_split_count_invariance(ns):
    q = rounded(151, (1, 8, 67, 64))
    k, v = rounded(152, (1, 8, 4374, 64)), rounded(153, (1, 8, 4374, 64))
    got = run(q, k, v, num_splits=ns)
    assert_close_bf16(got, O.attention_f32(q, k, v), f"num_splits={ns}")


@pytest.mark.parametrize("ns", [8, 9])
def test_ring_variants_image_b1(ns):
    """num_splits = 8 gives 256 workgroups (one per CU, splits of 4-5
    tiles), 9 gives 288 (more workgroups than CUs); both against the oracle,
    with and without valid lengths."""
    q = rounded(155, (1, 32, 67, 64))
    k, v = rounded(156, (1, 32, 4374, 64)), rounded(157, (1, 32, 4374, 64))
    got = run(q, k, v, num_splits=ns)
    assert_close_bf16(got, O.attention_f32(q, k, v), f"img B=1 num_splits={ns}")
    vl = np.array([3001], np.int32)
    got = run(q, k, v, num_splits=ns, valid_len=to_dev(vl, torch.int32))
    assert_close_bf16(got, O.attention_f32(q, k, v, valid_len=vl), f"img B=1 num_splits={ns} valid=3001")


@pytest.mark.parametrize("B,Sk,ns,vl", [(1, 4374, 0, None), (8, 1024, 0, "rand"), (2, 700, 3, None),
                                        (1, 129, 0, [100])])
def test_pv_forms_against_oracle(B, Sk, ns, vl):
    """The key-split kernel's default P.V form (fp16) and the exact form
    (bf16 V, P as a bf16 hi/lo pair) against the oracle."""
    q = rounded(162, (B, 32, 67, 64))
    k, v = rounded(163, (B, 32, Sk, 64)), rounded(164, (B, 32, Sk, 64))
    kw = dict(num_splits=ns)
    vld = None
    if vl is not None:
        vld = lang_valid_lengths(9, B) if vl == "rand" else np.asarray(vl, np.int32)
        kw["valid_len"] = to_dev(vld, torch.int32)
    fast = run(q, k, v, **kw)
    exact = run(q, k, v, exact_pv=True, **kw)
    ref = O.attention_f32(q, k, v, valid_len=vld)
    assert_close_bf16(fast, ref, f"fp16 P.V B={B} Sk={Sk}")
    assert_close_bf16(exact, ref, f"exact P.V B={B} Sk={Sk}")
    assert mean_rel(exact, ref) < 1e-4
    assert mean_rel(fast, ref) < 5e-4


@pytest.mark.parametrize("ns", [0, 1, 4])
def test_v_beyond_fp16_range(ns):
    """fp16 form: V is converted to fp16 with rounding to nearest, exact in
    fp16's normal range and +-inf above 2^16, so a V element with |v| >= 2^16 (or an inf or NaN)
    makes its head-dim column non-finite (inf or NaN) in every output row,
    through the splits and their merge, and leaves every other column
    bit-identical to the run without it (the P.V contraction is column-wise).
    65280, the largest bf16 below 2^16, is in range.  The exact form handles
    the finite cases."""
    q = rounded(165, (1, 32, 67, 64))
    k, v = rounded(166, (1, 32, 2000, 64)), rounded(167, (1, 32, 2000, 64))
    clean = run(q, k, v, num_splits=ns)
    vw = v.copy()
    vw[0, 3, 1000, 5] = 65280.0                 # in range
    vw[0, 9, 1500, 7] = 65536.0                 # 2^16
    vw[0, 17, :40, :] *= 3.0e5                  # every column gets elements >= 2^16
    vw[0, 22, 7, 63] = -np.inf
    vw[0, 30, 1999, 0] = np.nan
    vw = O.bf16_round(vw)
    got = run(q, k, vw, num_splits=ns)
    bad = {9: [7], 17: list(range(64)), 22: [63], 30: [0]}
    for hh, cols in bad.items():
        assert not np.isfinite(got[0, hh][:, cols]).any(), hh
        rest = [c for c in range(64) if c not in cols]
        assert np.array_equal(got[0, hh][:, rest], clean[0, hh][:, rest]), hh
    ref = O.attention_f32(q, k, vw)
    g3, r3 = got[0, 3].astype(np.float64), ref[0, 3].astype(np.float64)   # outputs up to ~1e4
    assert np.abs(g3 - r3).max() <= 2e-2 * max(1.0, np.abs(r3).max())
    assert np.abs(g3 - r3).sum() <= 5e-4 * np.abs(r3).sum()
    for hh in (0, 1, 8, 31):
        assert np.array_equal(got[0, hh], clean[0, hh])
    exact = run(q, k, vw, num_splits=ns, exact_pv=True)
    for hh in (3, 9, 17):
        g_, r_ = exact[0, hh].astype(np.float64), ref[0, hh].astype(np.float64)
        assert np.abs(g_ - r_).max() <= 2e-2 * max(1.0, np.abs(r_).max())
        assert np.abs(g_ - r_).sum() <= 1e-4 * np.abs(r_).sum()


def test_causal_matches_oracle():
    q, k, v = (rounded(s, (1, 4, 67, 64)) for s in (161, 162, 163))
    got = run(q, k, v, is_causal=True)
    assert_close_bf16(got, O.attention_f32(q, k, v, causal=True), "causal 67")


def test_bshd_output_view_matches_bhsd():
    q = rounded(171, (2, 32, 67, 64))
    k, v = rounded(172, (2, 32, 700, 64)), rounded(173, (2, 32, 700, 64))
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    bhsd = attention(qd, kd, vd, out_dtype=torch.float32)
    seq = torch.empty(2, 67, 32, 64, device=DEV, dtype=torch.float32)
    attention(qd, kd, vd, out=seq.permute(0, 2, 1, 3))
    torch.cuda.synchronize()
    assert torch.equal(seq.permute(0, 2, 1, 3), bhsd)


@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 1, 1, 1), (1, 2, 3, 33), (2, 3, 200, 300),
                                       (1, 1, 81, 129), (3, 2, 67, 5000)])
def test_edge_shapes(B, H, Sq, Sk):
    q, k, v = rounded(181, (B, H, Sq, 64)), rounded(182, (B, H, Sk, 64)), rounded(183, (B, H, Sk, 64))
    got = run(q, k, v)
    assert_close_bf16(got, O.attention_f32(q, k, v), f"edge {B},{H},{Sq},{Sk}")


def test_valid_len_zero_gives_zeros_and_overlong_is_clamped():
    q = rounded(191, (3, 2, 67, 64))
    k, v = rounded(192, (3, 2, 256, 64)), rounded(193, (3, 2, 256, 64))
    vl = np.array([0, 1000, 17], np.int32)
    got = run(q, k, v, valid_len=to_dev(vl, torch.int32))
    assert np.all(got[0] == 0)
    ref = O.attention_f32(q, k, v, valid_len=vl)
    assert_close_bf16(got, ref, "valid 0/overlong/17")


def test_constant_inputs_bench_attention_case():
    x = np.full((1, 32, 67, 64), 0.01, np.float32)
    c = float(O.bf16_round(np.array([0.01], np.float32))[0])
    got = run(x, x, x)
    assert np.abs(got - c).max() < 1e-6


def test_sharp_softmax_stays_stable():
    q = rounded(201, (1, 4, 67, 64), scale=6.0)
    k, v = rounded(202, (1, 4, 2000, 64), scale=6.0), rounded(203, (1, 4, 2000, 64))
    got = run(q, k, v)
    assert_close_bf16(got, O.attention_f32(q, k, v), "sharp")


def test_graph_capture_replays_match_eager():
    q = to_dev(rounded(211, (1, 32, 67, 64)))
    k, v = to_dev(rounded(212, (1, 32, 4374, 64))), to_dev(rounded(213, (1, 32, 4374, 64)))
    out = torch.empty(1, 32, 67, 64, device=DEV, dtype=torch.float32)
    from servoflow_amd.attention import make_desc, workspace_bytes
    ws = torch.zeros(workspace_bytes(make_desc(q, k, v, out)), dtype=torch.uint8, device=DEV)
    attention(q, k, v, out=out, workspace=ws)
    torch.cuda.synchronize()
    eager = out.clone()
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            attention(q, k, v, out=out, workspace=ws)
    torch.cuda.current_stream().wait_stream(s)
    for i in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), f"replay {i}"
        _ = (q.float() * 2).sum().item()      # eager work between replays


def test_error_paths_on_device():
    q = to_dev(rounded(221, (1, 2, 67, 64)))
    k = to_dev(rounded(222, (1, 2, 4374, 64)))
    with pytest.raises(abi.SfError) as e:
        attention(q, k, k, out_dtype=torch.float32, workspace=torch.empty(8, dtype=torch.uint8, device=DEV),
                  num_splits=4)
    assert e.value.status == abi.SF_EWORKSPACE
    q128 = torch.zeros(1, 2, 4, 128, device=DEV, dtype=torch.bfloat16)
    with pytest.raises(abi.SfError) as e:
        attention(q128, q128, q128)
    assert e.value.status == abi.SF_ENOTSUP


def test_workspace_reuse_across_calls():
    from servoflow_amd.attention import make_desc, workspace_bytes
    q = to_dev(rounded(231, (2, 32, 67, 64)))
    k, v = to_dev(rounded(232, (2, 32, 1500, 64))), to_dev(rounded(233, (2, 32, 1500, 64)))
    out = torch.empty(2, 32, 67, 64, device=DEV, dtype=torch.float32)
    need = workspace_bytes(make_desc(q, k, v, out, num_splits=5))
    ws = torch.full((need,), 0x7f, dtype=torch.uint8, device=DEV)   # garbage contents are fine
    ref = None
    for i in range(3):
        attention(q, k, v, out=out, workspace=ws, num_splits=5)
        torch.cuda.synchronize()
        if ref is None:
            ref = out.clone()
        assert torch.equal(out, ref), f"call {i}"
        # a smaller problem reusing the same workspace in between
        attention(q[:1], k[:1, :, :700], v[:1, :, :700], workspace=ws, num_splits=3)
    torch.cuda.synchronize()
    assert_close_bf16(ref.cpu().numpy(), O.attention_f32(*(x.float().cpu().numpy() for x in (q, k, v))),
                      "reuse")


@pytest.mark.parametrize("Sq,Sk,causal,vl", [(67, 67, False, None), (67, 128, False, [128, 5, 0]),
                                            (200, 100, True, None), (16, 2, False, [1, 2, 2]),
                                            (1, 97, False, [97, 96, 33]), (67, 64, True, [64, 40, 1])])
def test_short_key_path(Sq, Sk, causal, vl):
    """Sk <= 128 runs the one-wave short-key kernel (single-pass softmax, V
    read through LDS transpose loads); it must agree with the oracle and with
    the split kernel (forced by num_splits=2) on the same inputs."""
    B, H = 3, 2
    q, k, v = rounded(241, (B, H, Sq, 64)), rounded(242, (B, H, Sk, 64)), rounded(243, (B, H, Sk, 64))
    kw = dict(is_causal=causal)
    vld = None
    if vl is not None:
        vld = np.asarray(vl, np.int32)
        kw["valid_len"] = to_dev(vld, torch.int32)
    got = run(q, k, v, **kw)
    ref = O.attention_f32(q, k, v, causal=causal, valid_len=vld)
    assert_close_bf16(got, ref, f"short {Sq}x{Sk} causal={causal} vl={vl}")
    split = run(q, k, v, num_splits=2, exact_pv=True, **kw)
    assert np.abs(split - got).max() < 1e-4
    if vl is not None and 0 in vl:
        assert np.all(got[list(vl).index(0)] == 0)


def test_short_key_path_strided_output_and_graph():
    q = to_dev(rounded(251, (2, 32, 67, 64)))
    k, v = to_dev(rounded(252, (2, 32, 67, 64))), to_dev(rounded(253, (2, 32, 67, 64)))
    bhsd = attention(q, k, v, out_dtype=torch.bfloat16)
    seq = torch.empty(2, 67, 32, 64, device=DEV, dtype=torch.bfloat16)   # [B, S, H*64] as the block uses
    g = torch.cuda.CUDAGraph()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            attention(q, k, v, out=seq.permute(0, 2, 1, 3))
    torch.cuda.current_stream().wait_stream(s)
    for i in range(3):
        seq.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(seq.permute(0, 2, 1, 3), bhsd), f"replay {i}"


def _masked_reference(q, k, v, mask):
    """Key-padding mask == attention over the kept keys only (per batch)."""
    B, H, Sq, D = q.shape
    ref = np.zeros((B, H, Sq, D), np.float32)
    for b in range(B):
        keep = np.flatnonzero(mask[b])
        if keep.size:
            ref[b:b + 1] = O.attention_f32(q[b:b + 1], np.ascontiguousarray(k[b:b + 1][:, :, keep]),
                                           np.ascontiguousarray(v[b:b + 1][:, :, keep]))
    return ref


@pytest.mark.parametrize("Sk", [67, 130, 1000, 4374])
def test_key_padding_mask(Sk):
    """A boolean key mask [B, Sk] (the key-padding form of dit_block.h:141)
    equals attention over the kept keys; combined with valid_len by AND; a
    row with nothing kept yields zeros."""
    B, H, Sq = 3, 2, 67
    q, k, v = rounded(261, (B, H, Sq, 64)), rounded(262, (B, H, Sk, 64)), rounded(263, (B, H, Sk, 64))
    rng = np.random.default_rng(Sk)
    mask = rng.random((B, Sk)) < 0.6
    mask[2] = False
    stride = (Sk + 3) // 4 * 4
    md = torch.zeros(B, stride, dtype=torch.uint8, device=DEV)
    md[:, :Sk] = torch.from_numpy(mask.astype(np.uint8)).to(DEV)
    got = run(q, k, v, kv_mask=md[:, :Sk])
    ref = _masked_reference(q, k, v, mask)
    assert_close_bf16(got, ref, f"key mask Sk={Sk}")
    assert np.all(got[2] == 0)
    # AND with valid lengths
    vl = np.array([Sk // 2, Sk, 5], np.int32)
    got2 = run(q, k, v, kv_mask=md[:, :Sk], valid_len=to_dev(vl, torch.int32))
    m2 = mask.copy()
    for b in range(B):
        m2[b, vl[b]:] = False
    assert_close_bf16(got2, _masked_reference(q, k, v, m2), f"key mask & valid Sk={Sk}")


@pytest.mark.parametrize("exact_pv", [False, True])
def test_full_size_b8_image_properties(exact_pv):
    """The benchmarked batch-8 image shape (8x32x67x4374), checked through
    properties that hold at any size: doubling V doubles the fp32 output bit
    for bit (the fp16 conversion of V -- exact in fp16's normal range, so V
    is kept at |v| >= 2^-13 here --, the bf16 (hi, lo) form and the fp32
    accumulations all scale exactly by 2), and a V whose rows are all one
    vector returns that vector in every query row (the weights sum to the
    row sum they are divided by)."""
    B, H, Sq, Sk = 8, 32, 67, 4374
    dev = torch.device(DEV)
    g = torch.Generator(device=dev)
    g.manual_seed(4374)
    q = torch.randn(B, H, Sq, 64, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Sk, 64, device=dev, generator=g)
    v = (torch.sign(v) * v.abs().clamp(min=2.0 ** -13)).to(torch.bfloat16)
    o1 = attention(q, k, v, out_dtype=torch.float32, exact_pv=exact_pv)
    o2 = attention(q, k, (2 * v.float()).to(torch.bfloat16), out_dtype=torch.float32, exact_pv=exact_pv)
    torch.cuda.synchronize()
    assert torch.isfinite(o1).all()
    assert torch.equal(o2, 2 * o1)
    row = torch.randn(B, H, 1, 64, device=dev, generator=g).to(torch.bfloat16)
    oc = attention(q, k, row.expand(B, H, Sk, 64).contiguous(), out_dtype=torch.float32, exact_pv=exact_pv)
    torch.cuda.synchronize()
    ref = row.float().expand(B, H, Sq, 64)
    assert float((oc - ref).abs().max()) <= 1e-5 * float(ref.abs().max())


@pytest.mark.parametrize("B,H,Sq,Sk", [(1, 2, 100, 65536), (1, 1, 1000, 2048)])
def test_long_keys_and_many_query_chunks(B, H, Sq, Sk):
    """65536 keys (512 tiles, 64 splits' worth: the split cap) and 1000
    queries (13 query chunks of 80 rows) against the oracle."""
    q, k, v = rounded(191, (B, H, Sq, 64)), rounded(192, (B, H, Sk, 64)), rounded(193, (B, H, Sk, 64))
    got = run(q, k, v)
    assert_close_bf16(got, O.attention_f32(q, k, v), f"long {B},{H},{Sq},{Sk}")


@pytest.mark.parametrize("B,H,Sq,Sk,causal,vl,dt", [(8, 32, 67, 67, False, None, torch.bfloat16),
                                                    (16, 32, 67, 67, False, None, torch.bfloat16),
                                                    (32, 32, 67, 67, False, None, torch.bfloat16),
                                                    (8, 32, 81, 100, True, "rand", torch.bfloat16),
                                                    (4, 64, 67, 67, False, "rand", torch.float16)])
def test_short_keys_grouped_waves(B, H, Sq, Sk, causal, vl, dt):
    """Short key sets at B*H >= 256 (every batch size) run a head's query
    blocks as the five waves of one workgroup sharing K and V in LDS:
    against the oracle, and bit-identical to the same heads run one batch
    element at a time (B*H < 256: one wave per workgroup)."""
    q, k, v = rounded(241, (B, H, Sq, 64)), rounded(242, (B, H, Sk, 64)), rounded(243, (B, H, Sk, 64))
    lens = None if vl is None else np.random.default_rng(244).integers(1, Sk + 1, size=B).astype(np.int32)
    kw = {"is_causal": causal}
    dq, dk, dv = (to_dev(x, dt) for x in (q, k, v))
    full = attention(dq, dk, dv, out_dtype=torch.float32,
                     valid_len=None if lens is None else to_dev(lens, torch.int32), **kw)
    torch.cuda.synchronize()
    got = full.float().cpu().numpy()
    ref = O.attention_f32(q, k, v, causal=causal, valid_len=lens)
    assert_close_bf16(got, ref, f"grouped short keys {B},{H},{Sq},{Sk}")
    for b in range(B):
        one = attention(dq[b:b + 1], dk[b:b + 1], dv[b:b + 1], out_dtype=torch.float32,
                        valid_len=None if lens is None else to_dev(lens[b:b + 1], torch.int32), **kw)
        torch.cuda.synchronize()
        assert np.array_equal(one.float().cpu().numpy()[0], got[b]), b


def test_short_keys_grouped_large_bh_causal_ragged_mask():
    """B*H = 1024 on the grouped five-wave workgroups with causal rows,
    random valid lengths (zeros included) and a key-padding mask at once:
    against an fp64 closed form (softmax over the allowed keys k <=
    valid_len, mask[k], k <= q; zeros for a row with none), and
    bit-identical to the same heads run one batch element at a time (one
    wave per workgroup)."""
    B, H, Sq, Sk = 32, 32, 67, 67
    q, k, v = rounded(641, (B, H, Sq, 64)), rounded(642, (B, H, Sk, 64)), rounded(643, (B, H, Sk, 64))
    rng = np.random.default_rng(644)
    lens = rng.integers(0, Sk + 1, size=B).astype(np.int32)
    lens[[3, 17]] = 0
    mask = rng.random((B, Sk)) < 0.7
    stride = (Sk + 3) // 4 * 4
    md = torch.zeros(B, stride, dtype=torch.uint8, device=DEV)
    md[:, :Sk] = torch.from_numpy(mask.astype(np.uint8)).to(DEV)
    dq, dk, dv = (to_dev(x, torch.bfloat16) for x in (q, k, v))
    full = attention(dq, dk, dv, out_dtype=torch.float32, is_causal=True, valid_len=to_dev(lens, torch.int32),
                     kv_mask=md[:, :Sk])
    torch.cuda.synchronize()
    got = full.cpu().numpy()
    allowed = mask[:, None, None, :] & (np.arange(Sk)[None, None, None, :] < lens[:, None, None, None]) & \
        (np.arange(Sk)[None, None, None, :] <= np.arange(Sq)[None, None, :, None])
    sc = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), k.astype(np.float64)) / 8.0
    sc = np.where(allowed, sc, -np.inf)
    mx = np.max(sc, axis=-1, keepdims=True)
    p = np.where(allowed, np.exp(sc - np.where(np.isfinite(mx), mx, 0.0)), 0.0)
    den = p.sum(-1, keepdims=True)
    ref = np.einsum("bhqk,bhkd->bhqd", p / np.where(den > 0, den, 1.0), v.astype(np.float64))
    assert_close_bf16(got, ref, "grouped B*H=1024 causal + valid lengths + key mask")
    assert not got[3].any() and not got[17].any()
    for b in range(B):
        one = attention(dq[b:b + 1], dk[b:b + 1], dv[b:b + 1], out_dtype=torch.float32, is_causal=True,
                        valid_len=to_dev(lens[b:b + 1], torch.int32), kv_mask=md[b:b + 1, :Sk])
        torch.cuda.synchronize()
        assert np.array_equal(one.cpu().numpy()[0], got[b]), b


@pytest.mark.parametrize("B,H,Sq,Sk,causal,vl,dt,exact", [
    (1, 32, 67, 1024, False, "rand", torch.bfloat16, False),   # batch-1 language call
    (1, 3, 67, 600, False, None, torch.bfloat16, False),       # one head group, 5 of 8 slots empty
    (2, 5, 200, 700, False, None, torch.bfloat16, False),      # 13 query blocks, 2 groups (last padded)
    (1, 4, 150, 150, True, None, torch.bfloat16, False),       # causal, 10 blocks
    (4, 32, 67, 1024, False, "rand", torch.float16, False),
    (1, 32, 67, 1024, False, "rand", torch.bfloat16, True),    # exact P.V form
])
def test_query_block_grid(B, H, Sq, Sk, causal, vl, dt, exact):
    """Calls whose 80-row grid would leave CUs idle and whose keys fit 1024
    run one workgroup per 16-row query block over all keys (no split), the
    blocks of a head on one XCD: against the oracle, bit-identical per batch
    element to that element run alone, and within the fp16-P rounding of the
    key-split kernel (forced with num_splits)."""
    q, k, v = rounded(251, (B, H, Sq, 64)), rounded(252, (B, H, Sk, 64)), rounded(253, (B, H, Sk, 64))
    lens = None if vl is None else lang_valid_lengths(254 + B, B, 1, Sk)
    kw = {"is_causal": causal, "exact_pv": exact}
    dq, dk, dv = (to_dev(x, dt) for x in (q, k, v))
    vdev = None if lens is None else to_dev(lens, torch.int32)
    got = attention(dq, dk, dv, out_dtype=torch.float32, valid_len=vdev, **kw)
    split = attention(dq, dk, dv, out_dtype=torch.float32, valid_len=vdev, num_splits=2, **kw)
    torch.cuda.synchronize()
    got, split = got.cpu().numpy(), split.cpu().numpy()
    ref = O.attention_f32(q, k, v, causal=causal, valid_len=lens)
    assert_close_bf16(got, ref, f"query blocks {B},{H},{Sq},{Sk}")
    assert mean_rel(got, ref) < (1e-4 if exact else 5e-4)
    assert np.abs(got - split).max() < 1e-3
    for b in range(B):
        one = attention(dq[b:b + 1], dk[b:b + 1], dv[b:b + 1], out_dtype=torch.float32,
                        valid_len=None if lens is None else to_dev(lens[b:b + 1], torch.int32), **kw)
        torch.cuda.synchronize()
        assert np.array_equal(one.cpu().numpy()[0], got[b]), b


@pytest.mark.parametrize("B,H,Sk,vl,splits,scale,gamma,exact", [
    (1, 32, 1024, [517], 8, True, True, False),    # the batch-1 language call of the runtime
    (2, 32, 100, [100, 37], 4, False, True, False),  # <= 128 keys: still the query-block grid
    (1, 3, 300, None, 1, True, False, True),         # padded head group, no norm, exact P.V
])
def test_q_from_split_k_partials(B, H, Sk, vl, splits, scale, gamma, exact):
    """sf_attn_desc.q_partials: Q finished inside the attention from its
    projection's split-K partials (sum in slice order, row scale, bias,
    per-head RMSNorm, bf16) equals the attention over the same Q finished
    on the host, up to Q's rare one-ulp roundings (the norm's sum of squares
    is added in another order); q is not read."""
    import ctypes
    dev = torch.device(DEV)
    Sq, N = 67, H * 64
    g = torch.Generator(device=dev).manual_seed(300 + splits)
    part = torch.randn(splits, B * Sq, N, device=dev, generator=g) * 0.3
    bias = torch.randn(N, device=dev, generator=g) * 0.1
    sc = (torch.rand(N, device=dev, generator=g) + 0.5) if scale else None
    gam = (torch.rand(64, device=dev, generator=g) + 0.5) if gamma else None
    q = part.sum(0, dtype=torch.float32) if splits == 1 else part[0].clone()
    for j in range(1, splits):
        q = q + part[j]                               # slice order
    q = q * (sc if sc is not None else 1.0) + bias
    q = q.view(B, Sq, H, 64).permute(0, 2, 1, 3).contiguous()
    if gam is not None:
        q = q * torch.rsqrt(q.pow(2).mean(-1, keepdim=True) + 1e-6) * gam
    qb = q.to(torch.bfloat16)
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    vld = None if vl is None else torch.tensor(vl, dtype=torch.int32, device=dev)
    ref = attention(qb, k, v, out_dtype=torch.float32, valid_len=vld, exact_pv=exact)
    out = torch.full((B, H, Sq, 64), float("nan"), device=dev, dtype=torch.float32)
    d = make_desc(qb, k, v, out, valid_len=vld, exact_pv=exact)
    d.q_partials, d.q_splits = part.data_ptr(), splits
    d.q_bias = bias.data_ptr()
    d.q_scale = sc.data_ptr() if sc is not None else None
    d.q_gamma = gam.data_ptr() if gam is not None else None
    d.q_eps = 1e-6
    st = abi.lib().sf_attn_fwd(ctypes.byref(d), None, k.data_ptr(), v.data_ptr(), out.data_ptr(), None, 0,
                               torch.cuda.current_stream().cuda_stream)
    assert st == abi.SF_OK, st
    torch.cuda.synchronize()
    assert torch.isfinite(out).all()
    diff = (out - ref).abs()
    assert float(diff.max()) < 2e-2 and float(diff.sum() / ref.abs().sum()) < 2e-3
    # rejected before any launch: key-split grids, a bad slice count, fp16
    kk = torch.zeros(1, H, 4374, 64, device=dev, dtype=torch.bfloat16)
    d2 = make_desc(qb[:1], kk, kk, out[:1])
    d2.q_partials, d2.q_splits = part.data_ptr(), splits
    assert abi.lib().sf_attn_fwd(ctypes.byref(d2), None, kk.data_ptr(), kk.data_ptr(), out.data_ptr(), None, 0,
                                 None) == abi.SF_ENOTSUP
    d.q_splits = 9
    assert abi.lib().sf_attn_fwd(ctypes.byref(d), None, k.data_ptr(), v.data_ptr(), out.data_ptr(), None, 0,
                                 None) == abi.SF_EINVAL
    d.q_splits, d.in_dtype = splits, abi.SF_F16
    assert abi.lib().sf_attn_fwd(ctypes.byref(d), None, k.data_ptr(), v.data_ptr(), out.data_ptr(), None, 0,
                                 None) == abi.SF_ENOTSUP


@pytest.mark.parametrize("deferred", [False, True])
@pytest.mark.parametrize("w8", [False, True])
def test_q_partials_bit_identical_to_heads_epilogue(w8, deferred):
    """The runtime's two routes to a batch-1 language cross-attention give
    the same bits: (a) the cross-q projection with the per-head RMSNorm
    epilogue (SF_EPI_HEADS, split-K + reduce) writing Q, then sf_attn_fwd;
    (b) the projection's partials (SF_EPI_PARTIALS) finished inside
    sf_attn_fwd (q_partials) -- the same sums, scale, bias and norm in the
    same order.  deferred: the projection's input rows are x * gamma of a
    deferred RMSNorm (sf_rmsnorm_deferred), scaled per row by a_row_ss on
    route (a) and q_row_ss on route (b)."""
    import ctypes
    from servoflow_amd import kernels as Kn
    dev = torch.device(DEV)
    B, H, S, D, Sk = 1, 32, 67, 2048, 1024
    g = torch.Generator(device=dev).manual_seed(41)
    a = torch.randn(B * S, D, device=dev, generator=g).to(torch.bfloat16)
    rss = None
    if deferred:
        x = torch.randn(B * S, D, device=dev, generator=g) * 3.0
        a, rss = Kn.rmsnorm_deferred(x, torch.rand(D, device=dev, generator=g) + 0.5)
    if w8:
        w = torch.randint(-127, 128, (D, D), device=dev, generator=g, dtype=torch.int8)
        ws = torch.rand(D, device=dev, generator=g) * 2e-4 + 1e-4
    else:
        w = (torch.randn(D, D, device=dev, generator=g) * 0.02).to(torch.bfloat16)
        ws = None
    bias = torch.randn(D, device=dev, generator=g) * 0.02
    gam = torch.rand(64, device=dev, generator=g) + 0.5
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    vl = torch.tensor([517], dtype=torch.int32, device=dev)
    q = torch.empty(B, H, S, 64, device=dev, dtype=torch.bfloat16)
    Kn.gemm_heads(a, w, bias, S, H, [q], (gam,), w_scale=ws, row_ss=rss, row_n=D)
    ref = attention(q, k, v, out_dtype=torch.float32, valid_len=vl)
    d = Kn._desc(a, w, None, abi.SF_ACT_NONE, ws)
    d.epilogue = abi.SF_EPI_PARTIALS
    ns = abi.lib().sf_gemm_num_splits(ctypes.byref(d))
    part = torch.empty(ns, B * S, D, device=dev, dtype=torch.float32)
    d.workspace, d.workspace_bytes = part.data_ptr(), part.numel() * 4
    abi.check(abi.lib().sf_gemm(ctypes.byref(d), torch.cuda.current_stream().cuda_stream), "partials")
    out = torch.empty(B, H, S, 64, device=dev, dtype=torch.float32)
    ad = make_desc(q, k, v, out, valid_len=vl)
    ad.q_partials, ad.q_splits = part.data_ptr(), ns
    ad.q_bias, ad.q_scale, ad.q_gamma, ad.q_eps = bias.data_ptr(), ws.data_ptr() if ws is not None else None, \
        gam.data_ptr(), 1e-6
    if deferred:
        ad.q_row_ss, ad.q_row_tiles, ad.q_row_n, ad.q_row_eps = rss.data_ptr(), rss.shape[0], D, 1e-6
    abi.check(abi.lib().sf_attn_fwd(ctypes.byref(ad), None, k.data_ptr(), v.data_ptr(), out.data_ptr(), None, 0,
                                    torch.cuda.current_stream().cuda_stream), "attention from partials")
    torch.cuda.synchronize()
    assert torch.equal(out, ref)


def _heads_epilogue(P, S, H, gammas):
    """sf_heads_bf16 (the per-head epilogue over a bf16 projection) on P
    [B*S, nsec*H*64]: section j RMS-normalised per head with gammas[j] (None:
    copied) and scattered to [B, H, S, 64]."""
    import ctypes
    M, N = P.shape
    outs = [torch.empty(M // S, H, S, 64, device=P.device, dtype=torch.bfloat16) for _ in range(N // (H * 64))]
    d = abi.GemmDesc()
    d.M, d.N = M, N
    d.epilogue = abi.SF_EPI_HEADS
    d.H, d.S, d.eps = H, S, 1e-6
    for j, o in enumerate(outs):
        d.head_out[j] = o.data_ptr()
        d.head_stride[j][:] = (o.stride(0), o.stride(1), o.stride(2))
        if gammas[j] is not None:
            d.head_gamma[j] = gammas[j].data_ptr()
    abi.check(abi.lib().sf_heads_bf16(ctypes.byref(d), P.data_ptr(), P.stride(0),
                                      torch.cuda.current_stream().cuda_stream), "sf_heads_bf16")
    return outs


def _rows_as_heads(P, S, H, section):
    """[B, H, S, 64] view of section `section` of the projection rows P."""
    B = P.shape[0] // S
    return P.view(B, S, -1, H, 64)[:, :, section].permute(0, 2, 1, 3)


@pytest.mark.parametrize("B", [3, 16, 32])
def test_qk_norm_on_load_self_attention_bit_identical(B):
    """The self-attention reading Q, K and V straight from the QKV
    projection's bf16 rows, q_norm / k_norm applied as the rows are loaded
    (q_gamma / k_gamma), gives the bits of the per-head epilogue pass
    (sf_heads_bf16: split_qkv + apply_qk_norm) followed by the attention on
    [B, H, S, 64] -- the two routes of the runtime above 160 rows."""
    H, S = 32, 67
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(300 + B)
    P = (torch.randn(B * S, 3 * H * 64, device=dev, generator=g) * 3.0).to(torch.bfloat16)
    gq = torch.rand(64, device=dev, generator=g) + 0.5
    gk = torch.rand(64, device=dev, generator=g) + 0.5
    q, k, v = _heads_epilogue(P, S, H, (gq, gk, None))
    ref = attention(q, k, v, out_dtype=torch.float32)
    got = attention(*(_rows_as_heads(P, S, H, j) for j in range(3)), out_dtype=torch.float32,
                    q_gamma=gq, k_gamma=gk)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("B,Sk,lang,exact", [(16, 4374, False, False), (3, 4374, False, True),
                                             (3, 1024, True, False), (16, 1024, True, False)])
def test_q_norm_on_load_cross_attention_bit_identical(B, Sk, lang, exact):
    """Cross-attention with Q read from the cross-q projection's bf16 rows
    and q_norm applied on load equals the per-head epilogue pass + attention
    bit for bit, on every grid the runtime uses above 160 rows: one
    workgroup per (batch, head) (batch 16), key splits + merge (batch-3
    image), one workgroup per 16-row query block (batch-3 language)."""
    H, S = 32, 67
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(400 + B + Sk)
    P = (torch.randn(B * S, H * 64, device=dev, generator=g) * 3.0).to(torch.bfloat16)
    gq = torch.rand(64, device=dev, generator=g) + 0.5
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    vl = None
    if lang:
        vl = torch.from_numpy(lang_valid_lengths(B, B)).to(dev)
    (q,) = _heads_epilogue(P, S, H, (gq,))
    ref = attention(q, k, v, out_dtype=torch.float32, valid_len=vl, exact_pv=exact)
    got = attention(_rows_as_heads(P, S, H, 0), k, v, out_dtype=torch.float32, valid_len=vl, exact_pv=exact,
                    q_gamma=gq)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("B,S,lens", [(8, 40, None), (8, 67, (20, 67, 33, 1, 0, 48, 64, 17)),
                                      (12, 100, None)])
def test_qk_norm_on_load_grouped_waves(B, S, lens):
    """Grouped short-key workgroups (B*H >= 256: one wave per 16-query block)
    share the K normalisation through LDS: wave w normalises K blocks w, w+5
    and the others read them.  Bit-identical to the per-head epilogue pass +
    attention with waves past the queries (S = 40: two of five), key valid
    lengths that leave whole blocks unnormalised (0, 1, 17, ...) and two
    K blocks per wave (S = 100: blocks 0..6)."""
    H = 32
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(500 + B + S)
    P = (torch.randn(B * S, 3 * H * 64, device=dev, generator=g) * 2.0).to(torch.bfloat16)
    gq = torch.rand(64, device=dev, generator=g) + 0.5
    gk = torch.rand(64, device=dev, generator=g) + 0.5
    vl = None if lens is None else torch.tensor(lens, dtype=torch.int32, device=dev)
    q, k, v = _heads_epilogue(P, S, H, (gq, gk, None))
    ref = attention(q, k, v, out_dtype=torch.float32, valid_len=vl)
    got = attention(*(_rows_as_heads(P, S, H, j) for j in range(3)), out_dtype=torch.float32, valid_len=vl,
                    q_gamma=gq, k_gamma=gk)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("B", [3, 16, 32])
def test_qk_norm_on_load_fp16_self_attention(B):
    """The runtime's self-attention above 160 rows: Q, K and V read from the
    QKV projection's fp16 rows, q_norm / k_norm applied on load in fp32 and
    rounded to fp16, the fp16 contraction.  Against the fp32 oracle on the
    same normalisation (fp64, rounded to fp16) at the bf16 bar; every
    grouping of the short-key kernel (B*H = 96: one wave per workgroup;
    512, 1024: five)."""
    H, S = 32, 67
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(700 + B)
    P = (torch.randn(B * S, 3 * H * 64, device=dev, generator=g) * 3.0).to(torch.float16)
    gq = torch.rand(64, device=dev, generator=g) + 0.5
    gk = torch.rand(64, device=dev, generator=g) + 0.5
    got = attention(*(_rows_as_heads(P, S, H, j) for j in range(3)), out_dtype=torch.float32,
                    q_gamma=gq, k_gamma=gk)
    Ph = P.float().cpu().numpy().astype(np.float64).reshape(B, S, 3, H, 64).transpose(2, 0, 3, 1, 4)

    def norm16(x, gm):
        inv = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6)
        return (x * inv * gm.cpu().numpy().astype(np.float64)).astype(np.float16).astype(np.float32)

    q, k, v = norm16(Ph[0], gq), norm16(Ph[1], gk), Ph[2].astype(np.float32)
    ref = O.attention_f32(q, k, v)
    mx, mr = assert_close_bf16(got.cpu().numpy(), ref, f"fp16 rows self-attention B={B}")
    assert mr < 2e-4, mr


@pytest.mark.parametrize("B,Sk,lang,exact", [(16, 4374, False, False), (3, 4374, False, True),
                                             (3, 1024, True, False), (16, 1024, True, False)])
def test_q_f16_rows_cross_attention(B, Sk, lang, exact):
    """The runtime's cross-attention above 160 rows: Q from the cross-q
    projection's fp16 rows (q_f16), normalised on load and rounded to bf16,
    against the bf16 K/V cache.  For fp16 rows whose values are bf16
    numbers the result equals, bit for bit, the same rows given in bf16
    (both normalise the same floats in the same order); on general fp16
    rows it meets the bf16 bar against the oracle.  Every grid of the
    runtime: (batch, head) workgroups, key splits + merge, query blocks."""
    H, S = 32, 67
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(800 + B + Sk)
    P16 = (torch.randn(B * S, H * 64, device=dev, generator=g) * 3.0).to(torch.bfloat16)
    gq = torch.rand(64, device=dev, generator=g) + 0.5
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    vl = torch.from_numpy(lang_valid_lengths(B, B)).to(dev) if lang else None
    kw = dict(out_dtype=torch.float32, valid_len=vl, exact_pv=exact, q_gamma=gq)
    ref_b = attention(_rows_as_heads(P16, S, H, 0), k, v, **kw)
    got_b = attention(_rows_as_heads(P16.to(torch.float16), S, H, 0), k, v, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(ref_b).all()
    assert torch.equal(got_b, ref_b)
    Pf = (torch.randn(B * S, H * 64, device=dev, generator=g) * 3.0).to(torch.float16)
    got = attention(_rows_as_heads(Pf, S, H, 0), k, v, **kw)
    x = Pf.float().cpu().numpy().astype(np.float64).reshape(B, S, H, 64).transpose(0, 2, 1, 3)
    q = O.bf16_round((x / np.sqrt((x * x).mean(-1, keepdims=True) + 1e-6) *
                      gq.cpu().numpy().astype(np.float64)).astype(np.float32))
    ref = O.attention_f32(q, k.float().cpu().numpy(), v.float().cpu().numpy(),
                          valid_len=None if vl is None else vl.cpu().numpy())
    assert_close_bf16(got.cpu().numpy(), ref, f"fp16 Q rows cross-attention B={B} Sk={Sk}")


@pytest.mark.parametrize("B,Sk,vl,causal,mask", [
    (1, 4374, None, False, False),    # batch-1 image: key splits + merge
    (2, 4374, None, False, False),    # four splits
    (8, 4374, None, False, True),     # one workgroup per (b, h), key-padding mask
    (1, 1024, [517], False, False),   # batch-1 language: the query-block grid
    (8, 1024, "rand", False, False),  # ragged language keys, (b, h) grid
    (3, 300, [300, 0, 129], True, False),
])
def test_v_f16_matches_converting_bf16_v(B, Sk, vl, causal, mask):
    """sf_attn_desc.v_f16: V given in fp16 (the runtime converts its cached V
    once, sf_bf16_to_f16_below) against bf16 Q/K.  The fast P.V form
    converts a bf16 V to fp16 with the same rounding in registers, so the
    output is bit for bit the bf16-V call's on every grid of the ring
    kernel."""
    dev = torch.device(DEV)
    H, Sq = 32, 67
    g = torch.Generator(device=dev).manual_seed(900 + B + Sk)
    q = torch.randn(B, H, Sq, 64, device=dev, generator=g).to(torch.bfloat16)
    k = torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16)
    v = (torch.randn(B, H, Sk, 64, device=dev, generator=g) * 3.0).to(torch.bfloat16)
    v[0, 0, :4, :4] = torch.tensor([1e-6, -3e-7, 2.0 ** -20, 60000.0], device=dev).to(torch.bfloat16)
    v16 = v.to(torch.float16)   # round to nearest even, as the kernel's conversion
    kw = dict(out_dtype=torch.float32, is_causal=causal)
    if vl == "rand":
        kw["valid_len"] = torch.from_numpy(lang_valid_lengths(B + 1, B)).to(dev)
    elif vl is not None:
        kw["valid_len"] = torch.tensor(vl, dtype=torch.int32, device=dev)
    if mask:   # rows padded to a multiple of 4 bytes
        keep = torch.rand(B, (Sk + 3) // 4 * 4, device=dev, generator=g) > 0.3
        keep[:, 0] = True
        kw["kv_mask"] = keep[:, :Sk]
    ref = attention(q, k, v, **kw)
    got = attention(q, k, v16, **kw)
    torch.cuda.synchronize()
    assert torch.isfinite(ref).all()
    assert torch.equal(got, ref)


@pytest.mark.parametrize("Sq,Sk,vl", [(67, 67, None), (67, 128, [128, 5, 0]), (67, 100, [100, 37, 64])])
@pytest.mark.parametrize("B", [3, 8])
def test_v_f16_short_keys(B, Sq, Sk, vl):
    """At most 128 keys (the runtime's language cache read at few valid
    keys above 160 rows) the short-key kernel takes fp16 V with P as an fp16
    (hi, lo) pair: against the oracle at the bf16 bar and within 1e-4 of the
    bf16-V call (P carries more bits; V holds the same values); one wave per
    query block (B*H < 256) and the grouped five-wave form."""
    dev = torch.device(DEV)
    H = 32
    vl = None if vl is None else (vl * ((B + 2) // 3))[:B]
    q, k, v = rounded(261, (B, H, Sq, 64)), rounded(262, (B, H, Sk, 64)), rounded(263, (B, H, Sk, 64))
    kw = {}
    vld = None
    if vl is not None:
        vld = np.asarray(vl, np.int32)
        kw["valid_len"] = to_dev(vld, torch.int32)
    qd, kd, vd = to_dev(q), to_dev(k), to_dev(v)
    got = attention(qd, kd, vd.to(torch.float16), out_dtype=torch.float32, **kw).cpu().numpy()
    ref_b = attention(qd, kd, vd, out_dtype=torch.float32, **kw).cpu().numpy()
    ref = O.attention_f32(q, k, v, valid_len=vld)
    assert_close_bf16(got, ref, f"short fp16 V B={B} {Sq}x{Sk}")
    assert np.abs(got - ref_b).max() < 1e-4


def test_v_f16_rejected_forms():
    """v_f16 needs bf16 Q/K and the fast P.V form: SF_ENOTSUP with the exact
    form, fp16 or fp32 inputs, before any launch."""
    import ctypes
    dev = torch.device(DEV)
    q = torch.zeros(1, 2, 16, 64, device=dev, dtype=torch.bfloat16)
    kv = torch.zeros(1, 2, 256, 64, device=dev, dtype=torch.bfloat16)
    out = torch.zeros(1, 2, 16, 64, device=dev, dtype=torch.float32)
    for field, value in (("exact_pv", 1), ("in_dtype", abi.SF_F16), ("in_dtype", abi.SF_F32)):
        d = make_desc(q, kv, kv.to(torch.float16), out)
        assert d.v_f16 == 1
        setattr(d, field, value)
        st = abi.lib().sf_attn_fwd(ctypes.byref(d), q.data_ptr(), kv.data_ptr(), kv.data_ptr(), out.data_ptr(),
                                   None, 0, None)
        assert st == abi.SF_ENOTSUP, (field, st)


def test_bf16_to_f16_below_converts_only_in_range_buffers():
    """sf_bf16_to_f16_below: each buffer whose measured max |x| is below the
    limit becomes its fp16 rounding (torch's conversion, bit for bit); a
    buffer at or above the limit, or with a NaN, is left untouched."""
    import ctypes
    dev = torch.device(DEV)
    g = torch.Generator(device=dev).manual_seed(77)
    bufs = [(torch.randn(n, device=dev, generator=g) * 100).to(torch.bfloat16) for n in (4096 + 5, 1 << 16, 24, 40)]
    bufs[1][123] = 70000.0      # out of fp16 range
    bufs[2][3] = float("nan")
    bufs[3][7] = 65000.0        # in range, rounds to a different fp16 neighbour grid
    orig = [b.clone() for b in bufs]
    amax = torch.zeros(len(bufs), dtype=torch.float32, device=dev)
    jobs = (abi.AbsmaxJob * len(bufs))()
    for j, b in enumerate(bufs):
        jobs[j].p, jobs[j].n, jobs[j].out = b.data_ptr(), b.numel(), amax.data_ptr() + 4 * j
    s = torch.cuda.current_stream().cuda_stream
    abi.check(abi.lib().sf_absmax_bf16_batched(jobs, len(bufs), s), "absmax")
    abi.check(abi.lib().sf_bf16_to_f16_below(jobs, len(bufs), ctypes.c_float(65504.0), s), "to_f16")
    torch.cuda.synchronize()
    for j, b in enumerate(bufs):
        conv = bool(amax[j] < 65504.0)
        assert conv == (j in (0, 3)), (j, float(amax[j]))
        want = orig[j].to(torch.float16).view(torch.int16) if conv else orig[j].view(torch.int16)
        assert torch.equal(b.view(torch.int16), want), j
