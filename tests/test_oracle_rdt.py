"""Pins the oracle's model composition (oracle/rdt.py) and its timestep
helpers against the reference's own definition of RDT-1B.

The fixture tests/golden/rdt_small.npz holds outputs of the reference's
PyTorch model (tests/alignment/test_rdt1b_alignment.py:73-257: adaptors,
timestep embedders, RDTBlock x 3, final layer, written by
tests/golden/make_rdt_golden.py) at a reduced size with the seeded
parameters of tests/golden/rdt_small.py.  Each test runs the oracle in pure
fp32 (rb=False) on the same parameters and inputs.  A composition mistake
(token order, even/odd alternation, a dropped position embedding, a wrong
adaptor depth or gamma, the final slice) moves the outputs by O(1), far
outside the fp32 reordering noise the tolerances allow.
"""
import math
import os

import numpy as np
import pytest

from golden import rdt_small as RS
from oracle import oracle as O
from oracle import rdt as OR

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "rdt_small.npz")


@pytest.fixture(scope="module")
def fx():
    return np.load(FIX)


@pytest.fixture(scope="module")
def params():
    return RS.make_params()


@pytest.fixture(scope="module")
def inputs():
    return RS.make_inputs()


def close(got, ref, rel=2e-5, what=""):
    """fp32 vs fp32 after different summation orders: mean relative error
    (sum|d| / sum|ref|) and max-abs relative to the largest reference value."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} vs {ref.shape}"
    scale = max(float(np.abs(ref).max()), 1e-30)
    mr = float(np.abs(got - ref).sum() / max(np.abs(ref).sum(), 1e-30))
    ma = float(np.abs(got - ref).max()) / scale
    assert mr <= rel and ma <= 10 * rel, f"{what}: mean-rel {mr:.2e}, max-abs/scale {ma:.2e}"


def lang_trunc(inputs, b):
    return inputs["lang_tok"][b:b + 1, :RS.LANG_LEN[b]]


def test_fixture_shapes(fx):
    c = RS.CFG
    assert fx["b0_t0/out"].shape == (c.horizon, c.action_dim)
    assert fx["b1_t0/cond_1"].shape == (c.img_len, c.hidden)
    assert fx["b1_t0/cond_0"].shape == (RS.LANG_LEN[1], c.hidden)
    assert list(fx["t_index"]) == [999, 599, 200]


def test_adaptors_match_reference(fx, params, inputs):
    """MlpAdaptor depth 2 for language / image, 3 for the state adaptor
    (rdt1b.cpp:56-85), on the action input cat(x_t, ones) (rdt1b.cpp:286-302)."""
    for b in range(2):
        close(OR.mlp_adaptor(params, "lang_adaptor", lang_trunc(inputs, b)[0], 2, rb=False),
              fx[f"b{b}_t0/lang_c"], what=f"lang adaptor b{b}")
        close(OR.mlp_adaptor(params, "img_adaptor", inputs["img_tok"][b], 2, rb=False),
              fx[f"b{b}_t0/img_c"], what=f"img adaptor b{b}")
        x_t = inputs["noisy"][b]
        act_in = np.concatenate([x_t, np.ones_like(x_t)], axis=-1)
        close(OR.mlp_adaptor(params, "state_adaptor", act_in, 3, rb=False),
              fx[f"b{b}_t0/x_seq"][1:], what=f"action tokens b{b}")


def test_state_token_cpp_form(fx, params, inputs):
    """The C++ state token state_adaptor(cat(state, zeros)) (rdt1b.cpp:202-229)
    through the reference's Mlp3x, and that it differs from the Python
    model's all-ones form (test_rdt1b_alignment.py:204-208)."""
    for b in range(2):
        got = OR.state_token(params, inputs["state"][b:b + 1], RS.CFG, rb=False)[0]
        close(got, fx[f"b{b}/state_tok_zeros"], what=f"state token b{b}")
        assert np.abs(got - fx[f"b{b}_t0/x_seq"][0]).max() > 1e-2


def test_timestep_embedders_match_reference(fx, params):
    for ti in range(len(RS.T_VALUES)):
        t_int = O.timestep_index(float(fx["t_values"][ti]), RS.CFG.num_train_timesteps)
        assert t_int == int(fx["t_index"][ti])
        close(OR.timestep_embed(params, "t_embedder", t_int, RS.CFG, rb=False)[0],
              fx[f"b0_t{ti}/t_emb"][0], what=f"t_embedder t={t_int}")
    close(OR.timestep_embed(params, "freq_embedder", RS.CFG.ctrl_freq, RS.CFG, rb=False)[0],
          fx["b0_t0/freq_emb"][0], what="freq_embedder")


def test_condition_tokens_and_alternation(fx, params, inputs):
    """Position embeddings on the condition (rdt1b.cpp:342-349) and the
    even -> language, odd -> image alternation (dit_block.cu:369)."""
    for b in range(2):
        lang_c = fx[f"b{b}_t0/lang_c"][None]
        img_c = fx[f"b{b}_t0/img_c"][None]
        lang, img = OR.condition_tokens(params, lang_c, img_c, RS.CFG, rb=False)
        for i in range(RS.CFG.layers):
            close((lang if i % 2 == 0 else img)[0], fx[f"b{b}_t0/cond_{i}"], what=f"cond of block {i}")


def test_token_assembly_matches_reference(fx, params):
    """x = [t_emb, freq_emb, state, actions] + x_pos_embed (rdt1b.cpp:319-340)
    is the input of block 0."""
    for ti in range(len(RS.T_VALUES)):
        x_seq = fx["b0_t0/x_seq"]
        x = np.concatenate([fx[f"b0_t{ti}/t_emb"][0][None], fx["b0_t0/freq_emb"][0][None], x_seq], 0)
        close(x + params["x_pos_embed"][0], fx[f"b0_t{ti}/xin_0"], what="block-0 input")


@pytest.mark.parametrize("blk", [0, 1, 2])
def test_block_matches_reference(fx, params, blk):
    """RDTBlock::forward (dit_block.cu:349-387) with the cross K/V of
    cross_kv (dit_block.cu:288-308) on the reference's own block inputs."""
    for b in range(2):
        for ti in range(len(RS.T_VALUES)):
            x_in = fx[f"b{b}_t{ti}/xin_{blk}"][None]
            cond = fx[f"b{b}_t0/cond_{blk}"][None]
            ck, cv = OR.cross_kv(params, blk, cond, RS.CFG, rb=False)
            got = OR.rdt_block(params, blk, x_in, ck, cv, None, RS.CFG, rb=False)
            close(got[0], fx[f"b{b}_t{ti}/xout_{blk}"], what=f"block {blk} b{b} t{ti}")


def test_block_masked_padding_equals_truncation(fx, params):
    """Language padded to lang_max with noise rows and a valid length gives
    the truncated result (the reference truncates, rdt1b.cpp:426)."""
    b = 1
    L = RS.LANG_LEN[b]
    cond = fx[f"b{b}_t0/cond_0"][None]
    pad = np.concatenate([cond, 3.0 * O.randn(7, (1, RS.CFG.lang_max - L, RS.CFG.hidden))], 1)
    ck, cv = OR.cross_kv(params, 0, pad, RS.CFG, rb=False)
    got = OR.rdt_block(params, 0, fx[f"b{b}_t0/xin_0"][None], ck, cv, np.array([L], np.int32), RS.CFG,
                       rb=False)
    close(got[0], fx[f"b{b}_t0/xout_0"], what="padded language block")


def _encode(params, inputs):
    """Adaptor outputs of the padded batch and the per-layer caches."""
    lang_c = OR.mlp_adaptor(params, "lang_adaptor", inputs["lang_tok"], 2, rb=False)
    img_c = OR.mlp_adaptor(params, "img_adaptor", inputs["img_tok"], 2, rb=False)
    return OR.encode_caches(params, lang_c, img_c, RS.CFG, rb=False)


def test_denoise_step_matches_reference(fx, params, inputs):
    """RDT1BModel::denoise_step (rdt1b.cpp:254-369) at batch 2 with ragged
    language (valid lengths 11 and 7 of 16 padded tokens) against the
    reference forward of each batch element, state token taken from the
    reference's own x_seq."""
    caches = _encode(params, inputs)
    state_tok = np.stack([fx[f"b{b}_t0/x_seq"][0] for b in range(2)])
    for ti, t in enumerate(RS.T_VALUES):
        v = OR.denoise_step(params, inputs["noisy"], float(t), state_tok, caches, inputs["lang_len"],
                            RS.CFG, rb=False)
        for b in range(2):
            close(v[b], fx[f"b{b}_t{ti}/out"], what=f"denoise b{b} t={t}")


def test_sample_matches_reference(fx, params, inputs):
    """FlowMatchingSampler::sample (flow_matching.cpp:25-93), 3 Euler steps."""
    caches = _encode(params, inputs)
    state_tok = np.stack([fx[f"b{b}_t0/x_seq"][0] for b in range(2)])
    x = OR.sample(params, inputs["noisy"], state_tok, caches, inputs["lang_len"], RS.CFG, rb=False)
    for b in range(2):
        np.testing.assert_array_equal(inputs["noisy"][b], fx[f"b{b}/sample_x0"])
        close(x[b], fx[f"b{b}/sample"], what=f"sample b{b}")


def test_sample_constant_velocity_closed_form(params, inputs):
    """With the final layer's fc2 weight zero the velocity is its bias c for
    every step, and the Euler sum of dt over t = 1 -> 0 is -1: x_N = x_0 - c."""
    p = dict(params)
    p["final_layer.ffn_final.fc2.weight"] = np.zeros_like(p["final_layer.ffn_final.fc2.weight"])
    c = p["final_layer.ffn_final.fc2.bias"]
    caches = _encode(p, inputs)
    st = np.zeros((2, RS.CFG.hidden), np.float32)
    x = OR.sample(p, inputs["noisy"], st, caches, inputs["lang_len"], RS.CFG, rb=False)
    np.testing.assert_allclose(x, inputs["noisy"] - c, rtol=0, atol=2e-6)


def test_block_zero_branches_is_identity(params):
    """Every branch ends in a projection: with those weights and biases zero
    the block returns its residual input bit for bit."""
    p = dict(params)
    for n in ("attn.proj", "cross_attn.proj", "ffn.fc2"):
        p[f"blocks.1.{n}.weight"] = np.zeros_like(p[f"blocks.1.{n}.weight"])
        p[f"blocks.1.{n}.bias"] = np.zeros_like(p[f"blocks.1.{n}.bias"])
    x = O.randn(11, (1, RS.CFG.seq, RS.CFG.hidden))
    cond = O.randn(12, (1, RS.CFG.img_len, RS.CFG.hidden))
    ck, cv = OR.cross_kv(p, 1, cond, RS.CFG, rb=False)
    np.testing.assert_array_equal(OR.rdt_block(p, 1, x, ck, cv, None, RS.CFG, rb=False), x)


def test_denoise_batch_invariance(params, inputs):
    """Batch element b of a batch-2 step equals the batch-1 step of element b."""
    caches = _encode(params, inputs)
    st = O.randn(5, (2, RS.CFG.hidden))
    v2 = OR.denoise_step(params, inputs["noisy"], 0.6, st, caches, inputs["lang_len"], RS.CFG, rb=False)
    for b in range(2):
        cb = [(k[b:b + 1], v[b:b + 1]) for k, v in caches]
        v1 = OR.denoise_step(params, inputs["noisy"][b:b + 1], 0.6, st[b:b + 1], cb, inputs["lang_len"][b:b + 1],
                             RS.CFG, rb=False)
        close(v1[0], v2[b], rel=1e-6, what=f"batch slot {b}")


# ---- sincos table and timestep index --------------------------------------

def test_sincos_table_matches_reference_rows(fx):
    """build_sincos_table (dit_block.cu:58-72): [cos, sin] halves, frequency
    denominator `half` -- the reference's sincos_emb rows."""
    steps = fx["sincos_steps"]
    for dim in (32, 256):
        tab = O.sincos_table(1000, dim)
        got = tab[steps]
        ref = fx[f"sincos_{dim}"]
        angle = steps[:, None].astype(np.float64)
        tol = 2e-6 + 2e-7 * angle
        assert np.all(np.abs(got - ref) <= tol), f"dim {dim}: {np.abs(got - ref).max():.2e}"


def test_sincos_table_closed_form_fp64():
    """Against cos/sin of t * 10000^(-i/half) evaluated in fp64; the float32
    angle carries a relative error of a few ulps, so the bound grows with t."""
    for dim in (32, 256):
        half = dim // 2
        tab = O.sincos_table(1000, dim).astype(np.float64)
        t = np.arange(1000, dtype=np.float64)[:, None]
        freq = np.exp(-math.log(10000.0) * np.arange(half) / half)[None]
        ang = t * freq
        tol = 1e-6 + 4e-7 * ang
        assert np.all(np.abs(tab[:, :half] - np.cos(ang)) <= tol)
        assert np.all(np.abs(tab[:, half:] - np.sin(ang)) <= tol)
        # the dead dit_block.cpp variant (denominator half - 1) differs
        freq_alt = np.exp(-math.log(10000.0) * np.arange(half) / (half - 1))[None]
        assert np.abs(tab[:, :half] - np.cos(t * freq_alt)).max() > 1e-2


def _half_cases():
    """float32 t whose product t * 999f is exactly k + 0.5 (searched among
    the float32 neighbours of (k + 0.5) / 999)."""
    out = []
    for k in range(999):
        c = np.float32((k + 0.5) / 999.0)
        cands = [c]
        up = dn = c
        for _ in range(4):
            up = np.nextafter(up, np.float32(2.0), dtype=np.float32)
            dn = np.nextafter(dn, np.float32(-1.0), dtype=np.float32)
            cands += [up, dn]
        for t in cands:
            if float(np.float32(t) * np.float32(999.0)) == k + 0.5:
                out.append((float(t), k))
                break
    return out


def test_timestep_index_rounds_half_away_from_zero():
    """t_int = std::round(t * 999) clamped to [0, 999] (rdt1b.cpp:312-313):
    halves round away from zero (so k + 0.5 -> k + 1 also for even k, where
    round-half-to-even would give k)."""
    cases = _half_cases()
    assert len(cases) >= 20
    assert any(k % 2 == 0 for _, k in cases)
    for t, k in cases:
        assert O.timestep_index(t, 1000) == k + 1, (t, k)
    # the schedule of the 5-step loop and the clamp
    for t, want in [(1.0, 999), (0.8, 799), (0.6, 599), (0.4, 400), (0.2, 200), (0.0, 0),
                    (-0.3, 0), (1.7, 999)]:
        assert O.timestep_index(t, 1000) == want, t
    # generic values: floor(x + 0.5) of the float32 product
    for t in np.linspace(0.0, 1.0, 4001, dtype=np.float32):
        x = float(np.float32(t) * np.float32(999.0))
        assert O.timestep_index(float(t), 1000) == int(math.floor(x + 0.5))
