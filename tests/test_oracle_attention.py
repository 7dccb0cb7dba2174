"""Pins the CPU oracle's attention (oracle/sf_oracle.c, restating
src/backend/cuda/ops/attention.cu:90-139) before it is trusted as the checker.

Pins: golden vectors from the fp64 closed form (cross-checked against torch
SDPA when written), the independent fp64 two-pass evaluation, torch SDPA
directly, and closed-form special cases: constant V, one key, Q = 0, equal
keys, key permutation, valid length == truncation, causal == per-query
truncation, and the bench_attention.cu constant-input case.
"""
import json
import os

import numpy as np
import pytest
import torch

from oracle import oracle as O

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

CASES = ["self_67", "cross_img_slice", "cross_lang_valid", "causal_9", "tiny_d16", "single_key"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_golden(golden_attention, name):
    g = golden_attention
    B, H, Sq, Sk, D, causal = (int(x) for x in g[f"{name}/meta"])
    valid = g[f"{name}/valid"]
    valid = valid if valid.size else None
    out = O.attention_f32(g[f"{name}/q"], g[f"{name}/k"], g[f"{name}/v"],
                          causal=bool(causal), valid_len=valid)
    ref = g[f"{name}/out"]
    assert out.shape == ref.shape
    assert np.abs(out - ref).max() < 2e-6
    out64 = O.attention_f64(g[f"{name}/q"], g[f"{name}/k"], g[f"{name}/v"],
                            causal=bool(causal), valid_len=valid)
    assert np.abs(out64 - ref).max() < 1e-12


def _rand(seed, *shape):
    return O.randn(seed, shape)


def test_oracle_vs_torch_sdpa():
    q, k, v = _rand(1, 2, 3, 67, 64), _rand(2, 2, 3, 500, 64), _rand(3, 2, 3, 500, 64)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(x.astype(np.float64)) for x in (q, k, v))).numpy()
    out = O.attention_f32(q, k, v)
    assert np.abs(out - ref).max() < 2e-6


def test_f32_vs_f64_random_scale():
    q, k, v = _rand(4, 1, 2, 67, 64), _rand(5, 1, 2, 300, 64), _rand(6, 1, 2, 300, 64)
    a = O.attention_f32(q, k, v, scale=0.3)
    b = O.attention_f64(q, k, v, scale=0.3)
    assert np.abs(a - b).max() < 1e-5
    # scale 0 means 1/sqrt(D) (attention.cu:150)
    assert np.array_equal(O.attention_f32(q, k, v, scale=0.0), O.attention_f32(q, k, v, scale=0.125))


def test_constant_v_returns_v():
    q, k = _rand(7, 1, 2, 10, 64), _rand(8, 1, 2, 50, 64)
    v = np.broadcast_to(_rand(9, 1, 2, 1, 64), (1, 2, 50, 64)).copy()
    out = O.attention_f32(q, k, v)
    assert np.abs(out - v[:, :, :1, :]).max() < 1e-5


def test_bench_attention_constant_case():
    kat = json.load(open(os.path.join(ROOT, "tests", "golden", "reference_kats.json")))
    c = kat["bench_attention_constant"]["value"]
    x = np.full((1, 2, 16, 64), c, np.float32)
    out = O.attention_f32(x, x, x)
    assert np.abs(out - kat["bench_attention_constant"]["expected"]).max() < 1e-7


def test_single_key_returns_v0():
    q, k, v = _rand(10, 1, 1, 5, 64), _rand(11, 1, 1, 1, 64), _rand(12, 1, 1, 1, 64)
    out = O.attention_f32(q, k, v)
    assert np.abs(out - v).max() < 1e-7


def test_zero_query_gives_mean_of_v():
    q = np.zeros((1, 1, 3, 64), np.float32)
    k, v = _rand(13, 1, 1, 40, 64), _rand(14, 1, 1, 40, 64)
    out = O.attention_f32(q, k, v)
    assert np.abs(out - v.mean(axis=2, keepdims=True)).max() < 1e-6


def test_equal_keys_give_mean_of_v():
    q = _rand(15, 1, 1, 3, 64)
    k = np.broadcast_to(_rand(16, 1, 1, 1, 64), (1, 1, 40, 64)).copy()
    v = _rand(17, 1, 1, 40, 64)
    out = O.attention_f32(q, k, v)
    assert np.abs(out - v.mean(axis=2, keepdims=True)).max() < 1e-6


def test_key_permutation_invariance():
    q, k, v = _rand(18, 1, 2, 8, 64), _rand(19, 1, 2, 90, 64), _rand(20, 1, 2, 90, 64)
    perm = np.random.default_rng(3).permutation(90)
    a = O.attention_f32(q, k, v)
    b = O.attention_f32(q, k[:, :, perm], v[:, :, perm])
    assert np.abs(a - b).max() < 2e-6


def test_valid_len_equals_truncation():
    q, k, v = _rand(21, 3, 2, 67, 64), _rand(22, 3, 2, 128, 64), _rand(23, 3, 2, 128, 64)
    vl = np.array([32, 77, 128], np.int32)
    out = O.attention_f32(q, k, v, valid_len=vl)
    for b, L in enumerate(vl):
        ref = O.attention_f32(q[b:b + 1], k[b:b + 1, :, :L], v[b:b + 1, :, :L])
        assert np.array_equal(out[b:b + 1], ref)


def test_valid_len_zero_and_clamp():
    q, k, v = _rand(24, 2, 1, 4, 64), _rand(25, 2, 1, 16, 64), _rand(26, 2, 1, 16, 64)
    out = O.attention_f32(q, k, v, valid_len=np.array([0, 99], np.int32))
    assert np.all(out[0] == 0)
    assert np.array_equal(out[1:], O.attention_f32(q[1:], k[1:], v[1:]))


def test_causal_equals_per_query_truncation():
    q, k, v = _rand(27, 1, 2, 12, 64), _rand(28, 1, 2, 12, 64), _rand(29, 1, 2, 12, 64)
    out = O.attention_f32(q, k, v, causal=True)
    for i in range(12):
        ref = O.attention_f32(q[:, :, i:i + 1], k[:, :, :i + 1], v[:, :, :i + 1])
        assert np.abs(out[:, :, i:i + 1] - ref).max() < 1e-7


def test_batch_equals_independent_batches():
    q, k, v = _rand(30, 4, 2, 9, 64), _rand(31, 4, 2, 33, 64), _rand(32, 4, 2, 33, 64)
    out = O.attention_f32(q, k, v)
    for b in range(4):
        assert np.array_equal(out[b:b + 1], O.attention_f32(q[b:b + 1], k[b:b + 1], v[b:b + 1]))


def test_randn_is_standard_normal_and_deterministic():
    a = O.randn(42, (200000,))
    assert np.array_equal(a, O.randn(42, (200000,)))
    assert not np.array_equal(a, O.randn(43, (200000,)))
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01


def test_bf16_round_matches_torch():
    x = O.randn(44, (100000,)) * 37.0
    x[:4] = [np.inf, -np.inf, 0.0, -0.0]
    ref = torch.from_numpy(x).to(torch.bfloat16).to(torch.float32).numpy()
    assert np.array_equal(O.bf16_round(x), ref)
