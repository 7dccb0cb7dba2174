"""Pins the oracle's non-attention functions against the reference's own
known-answer tests and against library routines / closed forms:
RMSNorm (norm.cuh:89-171), GELU-tanh / SiLU (elementwise.cuh:35-68), linear
(gemm_bias_act), the split_ops.cuh index maps, int8 dequant
(quantization.cu:18-51, KATs test_quantization.cpp) and Schedule::linspace
(flow_matching.cpp:10-17, KATs test_sampler.cpp).
"""
import json
import math
import os

import numpy as np
import torch

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
KATS = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")))


def test_rms_norm_closed_form_and_torch():
    x = O.randn(1, (67, 2048))
    g = O.randn(2, (2048,)) * 0.1 + 1.0
    out = O.rms_norm(x, g, 1e-6)
    ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (2048,),
                                       torch.from_numpy(g).double(), eps=1e-6).numpy()
    assert np.abs(out - ref).max() < 1e-5


def test_rms_norm_constant_row():
    for c in (3.0, -0.25):
        x = np.full((2, 64), c, np.float32)
        out = O.rms_norm(x, np.ones(64, np.float32), 1e-6)
        assert np.abs(out - math.copysign(1.0, c)).max() < 1e-5


def test_fused_add_rms_norm_is_add_then_norm():
    a, r = O.randn(3, (5, 256)), O.randn(4, (5, 256))
    g = O.randn(5, (256,))
    out, res = O.fused_add_rms_norm(a, r, g)
    assert np.array_equal(res, a + r)
    assert np.array_equal(out, O.rms_norm(a + r, g))


def test_gelu_tanh_vs_torch():
    xs = np.linspace(-8, 8, 1001).astype(np.float32)
    ref = torch.nn.functional.gelu(torch.from_numpy(xs).double(), approximate="tanh").numpy()
    got = np.array([O.gelu_tanh(float(x)) for x in xs])
    assert np.all(np.abs(got - ref) <= 1e-6 * np.maximum(1.0, np.abs(ref)))
    assert O.gelu_tanh(0.0) == 0.0


def test_silu_vs_torch():
    xs = np.linspace(-20, 20, 801).astype(np.float32)
    ref = torch.nn.functional.silu(torch.from_numpy(xs).double()).numpy()
    got = np.array([O.silu(float(x)) for x in xs])
    assert np.all(np.abs(got - ref) <= 1e-6 * np.maximum(1.0, np.abs(ref)))


def test_linear_vs_numpy():
    x, W, b = O.randn(6, (67, 300)), O.randn(7, (129, 300)) * 0.02, O.randn(8, (129,))
    y = O.linear(x, W, b)
    ref = x.astype(np.float64) @ W.astype(np.float64).T + b
    assert np.abs(y - ref).max() < 1e-4
    y1 = O.linear(x, W, b, act=1)
    assert np.abs(y1 - torch.nn.functional.gelu(torch.from_numpy(ref), approximate="tanh").numpy()).max() < 1e-4
    y2 = O.linear(x, W, None, act=2)
    assert np.abs(y2 - torch.nn.functional.silu(torch.from_numpy(ref - b)).numpy()).max() < 1e-4


def test_layout_maps_match_numpy_views():
    B, S, H, D = 2, 5, 3, 4
    qkv = np.arange(B * S * 3 * H * D, dtype=np.float32).reshape(B, S, 3 * H * D)
    Q, K, V = O.split_qkv(qkv, H, D)
    view = qkv.reshape(B, S, 3, H, D).transpose(2, 0, 3, 1, 4)   # timm's view(B,S,3,H,hd)
    assert np.array_equal(Q, view[0]) and np.array_equal(K, view[1]) and np.array_equal(V, view[2])
    kv = qkv[:, :, : 2 * H * D].copy()
    K2, V2 = O.split_kv(kv, H, D)
    view2 = kv.reshape(B, S, 2, H, D).transpose(2, 0, 3, 1, 4)
    assert np.array_equal(K2, view2[0]) and np.array_equal(V2, view2[1])
    x = qkv[:, :, : H * D].copy()
    hx = O.seq_to_head(x, H, D)
    assert np.array_equal(hx, x.reshape(B, S, H, D).transpose(0, 2, 1, 3))
    assert np.array_equal(O.head_to_seq(hx), x)


def test_dequant_reference_kats():
    for key in ("dequant_per_tensor", "dequant_per_channel"):
        k = KATS[key]
        q = np.array(k["input"], np.int8).reshape(k["shape"])
        s = np.array(k["scale"], np.float32)
        out = O.dequant_int8(q, s, per_channel=len(k["scale"]) > 1)
        assert np.abs(out.ravel() - np.array(k["expected"])).max() <= k["tol"]


def test_dequant_exhaustive_int8_bit_exact():
    q = np.arange(-128, 128, dtype=np.int8).reshape(4, 64)
    s = np.array([1.0, 0.5, 3.0, 1.0 / 127], np.float32)
    out = O.dequant_int8(q, s)
    ref = q.astype(np.float32) * s[:, None]       # row = i / K
    assert np.array_equal(out, ref)


def test_quantize_rows_roundtrip_bound():
    W = O.randn(9, (64, 300)) * 0.02
    q, s = O.quantize_int8_rows(W)
    assert q.min() >= -127 and q.max() <= 127
    assert np.all(np.abs(q).max(axis=1) == 127)
    err = np.abs(O.dequant_int8(q, s) - W)
    assert np.all(err <= 0.5 * s[:, None] * (1 + 1e-6))


def test_linspace_reference_kats():
    k = KATS["linspace_4"]
    ts = O.linspace(k["num_steps"], k["t_start"], k["t_end"])
    assert len(ts) == k["len"] and ts[0] == k["first"] and ts[-1] == k["last"]
    assert np.all(np.abs((ts[:-1] - ts[1:]) - k["step"]) <= k["tol"])
    k1 = KATS["linspace_1"]
    assert list(O.linspace(k1["num_steps"], k1["t_start"], k1["t_end"])) == k1["values"]
    t5 = O.linspace(5)
    assert np.allclose(t5, [1.0, 0.8, 0.6, 0.4, 0.2, 0.0], atol=1e-7)
