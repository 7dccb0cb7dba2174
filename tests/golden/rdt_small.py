"""Reduced RDT-1B configuration and seeded parameters shared by the fixture
generator (make_rdt_golden.py) and the oracle tests (test_oracle_rdt.py).

Parameters and inputs come from the oracle's own SplitMix64 / Box-Muller
generator (oracle.randn), so the generator and the tests rebuild exactly the
same values from (seed, name) and the fixture stores only expected outputs.
Names are the reference checkpoint keys (the key set that
tests/alignment/test_rdt1b_alignment.py:213-257 `load_weights` reads).

Shapes: hidden 128 = 2 heads x 64 (head order matters with two heads), 3
blocks (language, image, language: the even/odd alternation), 8 action
tokens (sequence 11), 40 image tokens, language padded to 16 with per-batch
valid lengths 11 and 7.
"""
from __future__ import annotations

import zlib

import numpy as np

from oracle import oracle as O
from oracle.rdt import RdtConfig

CFG = RdtConfig(hidden=128, layers=3, heads=2, action_dim=16, horizon=8, freq_dim=32,
                state_dim=16, lang_max=16, img_len=40, num_train_timesteps=1000,
                ctrl_freq=25, num_steps=3)
LANG_TOKEN_DIM = 64
IMG_TOKEN_DIM = 48
LANG_LEN = (11, 7)       # valid language tokens of batch elements 0 and 1
T_VALUES = (1.0, 0.6, 0.2)   # timesteps of the single-step fixtures
BASE_SEED = 20261202

# the reference's config dict (test_rdt1b_alignment.py:50-64) at this size
REF_CFG = {
    "hidden_size": CFG.hidden, "num_heads": CFG.heads, "head_dim": 64, "depth": CFG.layers,
    "action_dim": CFG.action_dim, "pred_horizon": CFG.horizon, "img_cond_len": CFG.img_len,
    "img_token_dim": IMG_TOKEN_DIM, "lang_token_dim": LANG_TOKEN_DIM,
    "state_token_dim": CFG.state_dim, "max_lang_cond_len": CFG.lang_max,
    "sincos_dim": CFG.freq_dim, "x_seq_len": CFG.horizon + 3,
}


def param_shapes(cfg=CFG):
    """name -> shape for every parameter of the model, checkpoint names."""
    D, A = cfg.hidden, cfg.action_dim
    s = {}

    def lin(name, n, k):
        s[name + ".weight"] = (n, k)
        s[name + ".bias"] = (n,)

    lin("lang_adaptor.0", D, LANG_TOKEN_DIM)
    lin("lang_adaptor.2", D, D)
    lin("img_adaptor.0", D, IMG_TOKEN_DIM)
    lin("img_adaptor.2", D, D)
    lin("state_adaptor.0", D, 2 * cfg.state_dim)
    lin("state_adaptor.2", D, D)
    lin("state_adaptor.4", D, D)
    for e in ("t_embedder", "freq_embedder"):
        lin(e + ".mlp.0", D, cfg.freq_dim)
        lin(e + ".mlp.2", D, D)
    s["x_pos_embed"] = (1, cfg.horizon + 3, D)
    s["lang_cond_pos_embed"] = (1, cfg.lang_max, D)
    s["img_cond_pos_embed"] = (1, cfg.img_len, D)
    for i in range(cfg.layers):
        p = f"blocks.{i}."
        for n in ("norm1", "norm2", "norm3"):
            s[p + n + ".weight"] = (D,)
        lin(p + "attn.qkv", 3 * D, D)
        s[p + "attn.q_norm.weight"] = (64,)
        s[p + "attn.k_norm.weight"] = (64,)
        lin(p + "attn.proj", D, D)
        lin(p + "cross_attn.q", D, D)
        lin(p + "cross_attn.kv", 2 * D, D)
        s[p + "cross_attn.q_norm.weight"] = (64,)
        s[p + "cross_attn.k_norm.weight"] = (64,)
        lin(p + "cross_attn.proj", D, D)
        lin(p + "ffn.fc1", D, D)
        lin(p + "ffn.fc2", D, D)
    s["final_layer.norm_final.weight"] = (D,)
    lin("final_layer.ffn_final.fc1", D, D)
    lin("final_layer.ffn_final.fc2", A, D)
    return s


def _seed(name):
    return BASE_SEED * 1000003 + zlib.crc32(name.encode())


def make_params(cfg=CFG):
    """Seeded parameters: linear weights N(0, 1/fan_in), biases N(0, 0.1^2),
    RMSNorm gammas 1 + N(0, 0.2^2) (so a swapped or dropped gamma shows),
    position embeddings N(0, 0.5^2) (non-zero, unlike the PyTorch init)."""
    out = {}
    for name, shape in param_shapes(cfg).items():
        if "norm" in name:
            v = 1.0 + O.randn(_seed(name), shape, 0.2)
        elif "pos_embed" in name:
            v = O.randn(_seed(name), shape, 0.5)
        elif name.endswith(".bias"):
            v = O.randn(_seed(name), shape, 0.1)
        else:
            v = O.randn(_seed(name), shape, 1.0 / np.sqrt(shape[1]))
        out[name] = np.ascontiguousarray(v, np.float32)
    return out


def make_inputs(cfg=CFG):
    """Raw inputs of the two batch elements: language tokens padded to
    lang_max (rows past LANG_LEN[b] hold noise that must be masked), image
    tokens, robot state and the noisy action chunk."""
    B = len(LANG_LEN)
    lang = O.randn(_seed("in.lang"), (B, cfg.lang_max, LANG_TOKEN_DIM))
    img = O.randn(_seed("in.img"), (B, cfg.img_len, IMG_TOKEN_DIM))
    state = O.randn(_seed("in.state"), (B, cfg.state_dim))
    noisy = O.randn(_seed("in.noisy"), (B, cfg.horizon, cfg.action_dim))
    return {"lang_tok": lang, "img_tok": img, "state": state, "noisy": noisy,
            "lang_len": np.array(LANG_LEN, np.int32)}
