"""Writes the golden fixtures under tests/golden/ (run from the repo root).

Nothing here uses the oracle or the kernels:
  * attention_small.npz — inputs from numpy's PCG64 generator, expected
    outputs from the closed form softmax(Q K^T * scale) V evaluated in fp64
    with numpy, and cross-checked at generation time against
    torch.nn.functional.scaled_dot_product_attention in fp64 (a library
    routine).  Valid-length cases are the closed form over K[:L], V[:L] (the
    reference's truncation of padded language, rdt1b.cpp:426); causal cases
    keep key k for query q iff k <= q (attention.cu:117).
  * reference_kats.json — the known-answer tests of the reference's own unit
    tests: tests/unit/test_quantization.cpp:20-46, 60-93 and
    tests/unit/test_sampler.cpp:8-32 (data only).
"""
import json
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def closed_form(q, k, v, scale, causal=False, valid=None):
    q, k, v = (x.astype(np.float64) for x in (q, k, v))
    B, H, Sq, D = q.shape
    Sk = k.shape[2]
    out = np.zeros((B, H, Sq, D))
    for b in range(B):
        L = Sk if valid is None else int(valid[b])
        s = np.einsum("hqd,hkd->hqk", q[b], k[b, :, :L]) * scale
        if causal:
            qi = np.arange(Sq)[:, None]
            ki = np.arange(L)[None, :]
            s = np.where(ki <= qi, s, -np.inf)
        s = s - s.max(-1, keepdims=True)
        p = np.exp(s)
        p /= p.sum(-1, keepdims=True)
        out[b] = np.einsum("hqk,hkd->hqd", p, v[b, :, :L])
    return out


def sdpa(q, k, v, scale, causal=False, valid=None):
    B = q.shape[0]
    outs = []
    for b in range(B):
        L = k.shape[2] if valid is None else int(valid[b])
        tq, tk, tv = (torch.from_numpy(x[b:b + 1].astype(np.float64)) for x in (q, k[:, :, :L], v[:, :, :L]))
        outs.append(torch.nn.functional.scaled_dot_product_attention(
            tq, tk, tv, scale=scale, is_causal=causal).numpy())
    return np.concatenate(outs, 0)


def attention_cases():
    rng = np.random.default_rng(20261201)
    cases = {
        # name: (B, H, Sq, Sk, D, causal, valid)
        "self_67": (1, 2, 67, 67, 64, False, None),
        "cross_img_slice": (1, 1, 67, 300, 64, False, None),
        "cross_lang_valid": (2, 1, 67, 160, 64, False, [37, 160]),
        "causal_9": (1, 1, 9, 9, 64, True, None),
        "tiny_d16": (2, 3, 5, 7, 16, False, None),
        "single_key": (1, 1, 4, 1, 64, False, None),
    }
    arrays = {}
    for name, (B, H, Sq, Sk, D, causal, valid) in cases.items():
        q = rng.standard_normal((B, H, Sq, D)).astype(np.float32)
        k = rng.standard_normal((B, H, Sk, D)).astype(np.float32)
        v = rng.standard_normal((B, H, Sk, D)).astype(np.float32)
        scale = 1.0 / np.sqrt(D)
        ref = closed_form(q, k, v, scale, causal, valid)
        chk = sdpa(q, k, v, scale, causal, valid)
        err = np.abs(ref - chk).max()
        assert err < 1e-12, (name, err)
        arrays[f"{name}/q"] = q
        arrays[f"{name}/k"] = k
        arrays[f"{name}/v"] = v
        arrays[f"{name}/out"] = ref
        arrays[f"{name}/meta"] = np.array([B, H, Sq, Sk, D, int(causal)], dtype=np.int64)
        arrays[f"{name}/valid"] = np.array(valid if valid is not None else [], dtype=np.int32)
    np.savez_compressed(os.path.join(HERE, "attention_small.npz"), **arrays)


def reference_kats():
    kats = {
        "source": "servoflow tests/unit/test_quantization.cpp and tests/unit/test_sampler.cpp",
        "dequant_per_tensor": {  # test_quantization.cpp:15-46
            "shape": [2, 4], "input": [-10, -5, 0, 5, 10, 20, 30, 40], "scale": [0.5],
            "expected": [-5.0, -2.5, 0.0, 2.5, 5.0, 10.0, 15.0, 20.0], "tol": 1e-2},
        "dequant_per_channel": {  # test_quantization.cpp:55-93
            "shape": [2, 4], "input": [10, 10, 10, 10, 20, 20, 20, 20], "scale": [0.5, 2.0],
            "expected": [5.0] * 4 + [40.0] * 4, "tol": 1e-2},
        "linspace_4": {  # test_sampler.cpp:8-21
            "num_steps": 4, "t_start": 1.0, "t_end": 0.0, "first": 1.0, "last": 0.0,
            "step": 0.25, "tol": 1e-6, "len": 5},
        "linspace_1": {  # test_sampler.cpp:23-32
            "num_steps": 1, "t_start": 1.0, "t_end": 0.0, "values": [1.0, 0.0], "len": 2},
        "bench_attention_constant": {  # benchmarks/bench_attention.cu:50-52 (fill 0.01)
            "value": 0.01, "expected": 0.01},
    }
    with open(os.path.join(HERE, "reference_kats.json"), "w") as f:
        json.dump(kats, f, indent=1)


if __name__ == "__main__":
    attention_cases()
    reference_kats()
    print("wrote", sorted(os.listdir(HERE)))
