"""CPU restatement of the RDT-1B block, denoise step and Euler loop.

TEST INFRASTRUCTURE ONLY: the checker for the MI355X model runtime
(servoflow_amd/host).  Orchestration is numpy; every contraction,
normalisation and attention runs in the C oracle (oracle/sf_oracle.c).

Parameters are a dict name -> float32 array, named as in the reference
checkpoint (tests/alignment/test_rdt1b_alignment.py:213-257,
docs/RDT1B_ARCHITECTURE.md key list).

`rb` (round to storage precision) names the storage points where values
are rounded, to model a pipeline that stores them in 16-bit types:
  True   every point below rounded to bf16 (GEMM inputs, per-head q/k/v,
         attention outputs, the cross-attention K/V cache, condition tokens,
         embeddings);
  False  none: the pure fp32 restatement;
  a set  of point names rounded to bf16;
  a dict point name -> "bf16" or "f16", e.g. storage_points(ffn16=True) for
         the MI355X runtime at batch <= 2, which stores the FFN inputs (the
         norm3 output and the GELU hidden) in fp16.
The residual stream stays fp32 throughout; the block's projection outputs
stay fp32 except at the "gemm" point.  The reference's own bf16 build rounds
at all of these points and also rounds the residual (norm.cuh:146).

Points: "cond" condition tokens + position embedding, "kv" cross K/V cache,
"n1" norm1 / norm_final outputs, "qkv" per-head q/k/v (self and cross),
"a" attention outputs, "n2" / "n3" norm2 / norm3 outputs, "h" FFN and final
hidden, "emb" timestep-embedding inputs, "adapt" adaptor inputs / hidden,
"state" the state token, "gemm" the block projections' outputs before
the residual add (attention / cross proj, fc2; the bf16 outputs of the
reference's cuBLASLt epilogues, cuda_backend.cu:414-447), "hgemm" the
per-head projections' outputs before the per-head norm (qkv, cross q; the
"gemm" setting when a dict or set of points leaves it out), "cq" the
cross-attention's per-head q (the "qkv" setting when left out), "kvgemm"
the cross K/V projection's output before split_kv / k_norm
(dit_block.cu:291-308), rounded when the projection has more than 160 rows
(the runtime's library path).
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from . import oracle as O


@dataclass
class RdtConfig:
    hidden: int = 2048
    layers: int = 28
    heads: int = 32
    action_dim: int = 128
    horizon: int = 64
    freq_dim: int = 256
    state_dim: int = 128
    lang_max: int = 1024
    img_len: int = 4374
    num_train_timesteps: int = 1000
    ctrl_freq: int = 25
    num_steps: int = 5
    eps: float = 1e-6

    @property
    def seq(self):            # t, freq, state, actions (config.h:64)
        return self.horizon + 3


ALL_POINTS = frozenset({"cond", "kv", "kvgemm", "n1", "qkv", "cq", "a", "n2", "n3", "h", "emb", "adapt",
                        "state"})


def storage_points(ffn16, gemm16=False, act16=False):
    """How the MI355X runtime stores each point: bf16 everywhere, except
    ffn16: the FFN inputs n3 and h in fp16;
    gemm16: the block projections' products ("gemm", "hgemm") in bf16
            (fp32 otherwise);
    act16 (the runtime above 160 rows, with ffn16): every projection input
            in fp16 (norm outputs "n1" / "n2", attention outputs "a"), the
            products in fp16 ("gemm", "hgemm"), the self-attention's per-head
            q / k / v in fp16 ("qkv"); the cross-attention's q ("cq") stays
            bf16 (its K / V cache is bf16)."""
    pts = {p: "bf16" for p in ALL_POINTS}
    if ffn16:
        pts["n3"] = pts["h"] = "f16"
    if gemm16:
        pts["gemm"] = pts["hgemm"] = "bf16"
    if act16:
        for p in ("n1", "n2", "a", "qkv", "gemm", "hgemm"):
            pts[p] = "f16"
    return pts


def runtime_points(rows):
    """The MI355X runtime's storage at `rows` = batch * 67 projection rows:
    the split-K regime (<= 160) keeps bf16 inputs with fp16 FFN inputs and
    fp32 products, and norm1 / norm2 in their deferred form ("defer": the
    rows x * gamma are stored, the projection's output rows scaled by
    1/rms after the product); the library regime (> 160) keeps fp16 inputs
    and fp16 products (storage_points)."""
    pts = storage_points(True, act16=rows > 160)
    if rows <= 160:
        pts["defer"] = True
    return pts


def _f16_round(x):
    return np.asarray(x, np.float32).astype(np.float16).astype(np.float32)


_FALLBACK = {"hgemm": "gemm", "cq": "qkv"}


def _r(x, rb, point):
    if rb is True:
        return O.bf16_round(x)
    if isinstance(rb, (dict, set, frozenset)) and point not in rb and point in _FALLBACK:
        point = _FALLBACK[point]
    if isinstance(rb, dict):
        mode = rb.get(point)
        if mode == "bf16":
            return O.bf16_round(x)
        if mode == "f16":
            return _f16_round(x)
    elif rb and point in rb:
        return O.bf16_round(x)
    return np.ascontiguousarray(x, np.float32)


def heads_of(x, H):
    """[B,S,H*64] -> [B,H,S,64] (seq_to_head, split_ops.cuh:123-137)."""
    return O.seq_to_head(x, H, 64)


def cross_kv(p, i, cond, cfg, rb=True):
    """K/V of block i's cross-attention over condition tokens cond [B,Sc,D]:
    kv = c Wkv^T + b, split_kv, k_norm on K (dit_block.cu:288-308)."""
    pre = f"blocks.{i}.cross_attn."
    B, Sc, D = cond.shape
    kv = O.linear(cond, p[pre + "kv.weight"], p[pre + "kv.bias"]).reshape(B, Sc, 2 * D)
    if B * Sc > 160:   # the runtime's library path stores this product in bf16
        kv = _r(kv, rb, "kvgemm")
    K, V = O.split_kv(kv, cfg.heads, 64)
    K = O.rms_norm(K, p[pre + "k_norm.weight"], cfg.eps)
    return _r(K, rb, "kv"), _r(V, rb, "kv")


def _deferred_linear(x, gamma, W, b, eps, rb, point):
    """RMSNorm(x) W^T + b in the runtime's deferred form: the stored input
    rows are x * gamma (rounded at `point`), the row's 1/rms multiplies the
    product before the bias -- equal in exact arithmetic, (s a) W^T =
    s (a W^T)."""
    x = np.asarray(x, np.float32)
    a = _r(x * np.asarray(gamma, np.float32), rb, point)
    s = (1.0 / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + eps)).astype(np.float32)
    return O.linear(a, W) * s + np.asarray(b, np.float32)


def rdt_block(p, i, x, ck, cv, cond_len, cfg, rb=True):
    """RDTBlock::forward, src/models/rdt1b/dit_block.cu:349-387, with the
    cross-attention K/V precomputed (cross_kv).  x [B,S,D] fp32, updated."""
    B, S, D = x.shape
    H = cfg.heads
    pre = f"blocks.{i}."
    defer = isinstance(rb, dict) and rb.get("defer", False)
    # self-attention branch (dit_block.cu:198-238)
    if defer:
        qkv = _r(_deferred_linear(x, p[pre + "norm1.weight"], p[pre + "attn.qkv.weight"],
                                  p[pre + "attn.qkv.bias"], cfg.eps, rb, "n1"), rb, "hgemm")
    else:
        n1 = _r(O.rms_norm(x, p[pre + "norm1.weight"], cfg.eps), rb, "n1")
        qkv = _r(O.linear(n1, p[pre + "attn.qkv.weight"], p[pre + "attn.qkv.bias"]), rb, "hgemm")
    Q, K, V = O.split_qkv(qkv.reshape(B, S, 3 * D), H, 64)
    Q = _r(O.rms_norm(Q, p[pre + "attn.q_norm.weight"], cfg.eps), rb, "qkv")
    K = _r(O.rms_norm(K, p[pre + "attn.k_norm.weight"], cfg.eps), rb, "qkv")
    V = _r(V, rb, "qkv")
    a = _r(O.head_to_seq(O.attention_f32(Q, K, V)), rb, "a")
    x = x + _r(O.linear(a, p[pre + "attn.proj.weight"], p[pre + "attn.proj.bias"]), rb, "gemm")
    # cross-attention branch (dit_block.cu:274-326), norm2 from fused_add_rms_norm
    if defer:
        cq = _r(_deferred_linear(x, p[pre + "norm2.weight"], p[pre + "cross_attn.q.weight"],
                                 p[pre + "cross_attn.q.bias"], cfg.eps, rb, "n2"), rb, "hgemm")
    else:
        n2 = _r(O.rms_norm(x, p[pre + "norm2.weight"], cfg.eps), rb, "n2")
        cq = _r(O.linear(n2, p[pre + "cross_attn.q.weight"], p[pre + "cross_attn.q.bias"]), rb, "hgemm")
    cq = _r(O.rms_norm(heads_of(cq.reshape(B, S, D), H), p[pre + "cross_attn.q_norm.weight"], cfg.eps), rb, "cq")
    ca = _r(O.head_to_seq(O.attention_f32(cq, ck, cv, valid_len=cond_len)), rb, "a")
    x = x + _r(O.linear(ca, p[pre + "cross_attn.proj.weight"], p[pre + "cross_attn.proj.bias"]), rb, "gemm")
    # FFN branch (Mlp::forward, dit_block.cu:143-163: fc1 + GELU, fc2)
    n3 = _r(O.rms_norm(x, p[pre + "norm3.weight"], cfg.eps), rb, "n3")
    h = _r(O.linear(n3, p[pre + "ffn.fc1.weight"], p[pre + "ffn.fc1.bias"], act=1), rb, "h")
    return x + _r(O.linear(h, p[pre + "ffn.fc2.weight"], p[pre + "ffn.fc2.bias"]), rb, "gemm")


def timestep_embed(p, name, step, cfg, rb=True):
    """TimestepEmbedding::forward, dit_block.cu:102-127: sincos row ->
    Linear + SiLU -> Linear.  Returns [1, D] fp32."""
    table = O.sincos_table(cfg.num_train_timesteps, cfg.freq_dim)
    step = max(0, min(int(step), cfg.num_train_timesteps - 1))
    e = _r(table[step:step + 1], rb, "emb")
    hdn = _r(O.linear(e, p[name + ".mlp.0.weight"], p[name + ".mlp.0.bias"], act=2), rb, "emb")
    return O.linear(hdn, p[name + ".mlp.2.weight"], p[name + ".mlp.2.bias"])


def mlp_adaptor(p, name, x, depth, rb=True):
    """MlpAdaptor::forward, rdt1b.cpp:56-85: (Linear + GELU) x (depth-1), Linear."""
    h = _r(x, rb, "adapt")
    for j in range(depth - 1):
        h = _r(O.linear(h, p[f"{name}.{2 * j}.weight"], p[f"{name}.{2 * j}.bias"], act=1), rb, "adapt")
    return O.linear(h, p[f"{name}.{2 * (depth - 1)}.weight"], p[f"{name}.{2 * (depth - 1)}.bias"])


def state_token(p, state, cfg, rb=True):
    """The condition's state token of RDT1BModel::encode_condition
    (rdt1b.cpp:202-229): state_adaptor(cat(state, zeros)), [B, D].  (The
    reference's Python model feeds an all-ones mask instead,
    test_rdt1b_alignment.py:204-208; the C++ form is the one restated.)"""
    st_in = np.concatenate([state, np.zeros_like(state)], axis=-1)
    return mlp_adaptor(p, "state_adaptor", st_in, 3, rb)


def condition_tokens(p, lang_c, img_c, cfg, rb=True):
    """lang_c + lang_cond_pos_embed[:L], img_c + img_cond_pos_embed
    (rdt1b.cpp:342-349), rounded where the GPU stores them."""
    L = lang_c.shape[1]
    lang = _r(lang_c + p["lang_cond_pos_embed"][:, :L], rb, "cond")
    img = _r(img_c + p["img_cond_pos_embed"], rb, "cond")
    return lang, img


def encode_caches(p, lang_c, img_c, cfg, rb=True):
    """Per-layer cross K/V caches (even layers: language, odd: image,
    dit_block.cu:369)."""
    lang, img = condition_tokens(p, lang_c, img_c, cfg, rb)
    return [cross_kv(p, i, lang if i % 2 == 0 else img, cfg, rb) for i in range(cfg.layers)]


def denoise_step(p, x_t, t, state_tok, caches, lang_len, cfg, rb=True):
    """RDT1BModel::denoise_step, src/models/rdt1b/rdt1b.cpp:254-369 (batch
    generalised): x_t [B,T,A] fp32, state_tok [B,D] (the condition's state
    token), returns the velocity [B,T,A]."""
    B, T, A = x_t.shape
    D = cfg.hidden
    ones = np.ones_like(x_t)
    act_in = np.concatenate([x_t, ones], axis=-1)                      # :289-300
    action_traj = mlp_adaptor(p, "state_adaptor", act_in, 3, rb)       # :302
    t_int = O.timestep_index(t, cfg.num_train_timesteps)              # :312-313
    t_emb = timestep_embed(p, "t_embedder", t_int, cfg, rb)
    f_emb = timestep_embed(p, "freq_embedder", cfg.ctrl_freq, cfg, rb)
    x = np.empty((B, T + 3, D), np.float32)
    x[:, 0] = t_emb[0]
    x[:, 1] = f_emb[0]
    x[:, 2] = _r(state_tok, rb, "state")
    x[:, 3:] = action_traj
    x = x + p["x_pos_embed"]                                            # :340
    for i in range(cfg.layers):                                         # :353-355
        ck, cv = caches[i]
        x = rdt_block(p, i, x, ck, cv, lang_len if i % 2 == 0 else None, cfg, rb)
    # FinalLayer::forward (dit_block.cu:407-412), last T tokens (rdt1b.cpp:362)
    nf = _r(O.rms_norm(x, p["final_layer.norm_final.weight"], cfg.eps), rb, "n1")
    hf = _r(O.linear(nf, p["final_layer.ffn_final.fc1.weight"], p["final_layer.ffn_final.fc1.bias"], act=1), rb,
            "h")
    out = O.linear(hf, p["final_layer.ffn_final.fc2.weight"], p["final_layer.ffn_final.fc2.bias"])
    return out[:, 3:]


def sample(p, x_init, state_tok, caches, lang_len, cfg, rb=True):
    """FlowMatchingSampler::sample, src/sampling/flow_matching.cpp:25-93:
    t_i = linspace(1 -> 0), x <- x + (t_{i+1} - t_i) v(x, t_i)."""
    ts = O.linspace(cfg.num_steps, 1.0, 0.0)
    x = np.array(x_init, np.float32, copy=True)
    for s in range(cfg.num_steps):
        v = denoise_step(p, x, float(ts[s]), state_tok, caches, lang_len, cfg, rb)
        dt = np.float32(ts[s + 1] - ts[s])
        x = x + dt * v                                                   # :77-78
    return x
