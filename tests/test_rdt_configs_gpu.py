"""GPU parity of the RDT-1B runtime at the benchmarked configurations the
other model tests do not reach: one full-width block against the pure-fp32
oracle, batch 16 and int8 batch 32 (the library-path
GEMMs at M = 1072 / 2144), the "MLP 4x" block-stack variant, and full-depth
batch-slot consistency at batch 16.

Oracle: oracle/rdt.py (pinned against the reference's PyTorch RDT by
tests/test_oracle_rdt.py).  rb=False is the pure-fp32 restatement; rb=True
rounds to bf16 exactly where the GPU stores bf16.
"""
import numpy as np
import pytest
import torch

from _util import mean_rel
from oracle import oracle as O
from oracle import rdt as OR
from servoflow_amd import rdt as R
from test_rdt_gpu import (DEV, assert_within_floor, build, make_condition, oracle_cfg, oracle_noise_floor,
                          rb_of, set_cond, small_cfg)

pytestmark = pytest.mark.gpu


# ---- one full-width block against the pure-fp32 oracle ------------------------

@pytest.mark.parametrize("blk", [0, 1], ids=["language", "image"])
def test_block_vs_fp32_oracle(blk):
    """RDTBlock::forward (dit_block.cu:349-387) at full width: block 0
    attends to 1024 padded language keys (valid length 700), block 1 to the
    4374 image keys.  The fp32 residual after the block is compared with the
    pure-fp32 oracle (rb=False: fp32 activations, fp32 K/V cache) at the
    max-abs <= 2e-2 and mean-rel <= 1e-3.

    At batch 1 the runtime stores the FFN's inputs (the norm3 output and
    the GELU hidden) in fp16, three more significant bits than bf16 at the
    same bytes; every other activation is bf16.  With those two in bf16 as
    well the block sat at 1.3e-3 from fp32 (they are the two largest of the
    block's bf16 storage errors), above the bar.  The GPU is also held to the
    oracle with the same storage points (rb_of)."""
    print(f"block {blk} vs fp32 oracle", flush=True)
    c = R.default_config(layers=2, batch=1)
    m = build(c)
    lang, ll, img, state = make_condition(c, lang_len=[700])
    set_cond(m, lang, ll, img, state)
    S = c.horizon + 3
    x = O.randn(77 + blk, (1, S, c.hidden))
    xd = torch.from_numpy(x).to(DEV)
    m.run_blocks(xd, first=blk, count=1)
    got = xd.cpu().numpy()
    p = m.state_dict()
    oc = oracle_cfg(c)
    lang32, img32 = OR.condition_tokens(p, lang, img, oc, rb=False)
    ck, cv = OR.cross_kv(p, blk, lang32 if blk == 0 else img32, oc, rb=False)
    ref32 = OR.rdt_block(p, blk, x, ck, cv, ll if blk == 0 else None, oc, rb=False)
    langb, imgb = OR.condition_tokens(p, lang, img, oc, rb=rb_of(c))
    ckb, cvb = OR.cross_kv(p, blk, langb if blk == 0 else imgb, oc, rb=rb_of(c))
    refb = OR.rdt_block(p, blk, x, ckb, cvb, ll if blk == 0 else None, oc, rb=rb_of(c))
    mx = float(np.abs(got - ref32).max())
    mr = mean_rel(got, ref32)
    mr_delta = mean_rel(got - x, ref32 - x)
    mr_model = mean_rel(refb, ref32)
    mr_b = mean_rel(got, refb)
    print(f"block {blk}: vs fp32 max-abs {mx:.3e} mean-rel {mr:.3e} (branch sum {mr_delta:.3e}); "
          f"bf16-storage oracle vs fp32 {mr_model:.3e}; GPU vs bf16-storage oracle {mr_b:.3e}")
    assert np.isfinite(got).all()
    assert mx <= 2e-2
    assert mr <= 1e-3
    assert mr_b <= 1e-3


# ---- batch 16 and int8 batch 32: the library-path regime ----------------------

@pytest.mark.parametrize("batch,int8,blk", [(16, 0, 0), (16, 0, 1), (32, 1, 0), (32, 1, 1), (32, 2, 0), (32, 2, 1)],
                         ids=["b16-language", "b16-image", "int8_b32-language", "int8_b32-image",
                              "int8direct_b32-language", "int8direct_b32-image"])
def test_block_vs_fp32_oracle_large_batch(batch, int8, blk):
    """RDTBlock::forward (dit_block.cu:349-387) at batch 16 (bf16 weights)
    and batch 32 (int8 weights): 1072 / 2144 rows per projection, the
    library-path GEMMs.  The fp32 residual after one full-width block is
    held to the north-star bar against the pure-fp32 oracle (rb=False):
    max-abs <= 2e-2 and mean-rel <= 1e-3.  Block 0 attends to language keys
    with ragged valid lengths, block 1 to image keys (reduced condition
    lengths: the precision question sits in the storage points of the
    1072 / 2144-row projections, not in the key count).

    Above 160 rows the runtime multiplies fp16 activations by fp16 copies
    of the weights and keeps the products in fp16 (the oracle's CPU model
    of that storage put the block at 5.6-7.9e-4 from fp32; with the bf16
    inputs and bf16 products used before, 1.6-1.8e-3).  int8 = 2 multiplies
    the int8 codes directly instead (no copies; the same fp16 storage
    points).  The GPU is also held to the oracle with the same storage
    points (rb_of) at the same bar."""
    print(f"block {blk} batch {batch} int8 {int8} vs fp32 oracle", flush=True)
    c = small_cfg(layers=2, batch=batch, int8_weights=int8)
    m = build(c)
    lang_len = np.random.default_rng(batch + blk).integers(8, c.lang_max + 1, size=batch).astype(np.int32)
    lang, ll, img, state = make_condition(c, lang_len=lang_len)
    set_cond(m, lang, ll, img, state)
    S = c.horizon + 3
    x = O.randn(177 + blk, (batch, S, c.hidden))
    xd = torch.from_numpy(x).to(DEV)
    m.run_blocks(xd, first=blk, count=1)
    got = xd.cpu().numpy()
    p = m.state_dict()
    m.close()
    oc = oracle_cfg(c)
    cond32 = OR.condition_tokens(p, lang, img, oc, rb=False)[blk]
    ck, cv = OR.cross_kv(p, blk, cond32, oc, rb=False)
    ref32 = OR.rdt_block(p, blk, x, ck, cv, ll if blk == 0 else None, oc, rb=False)
    condb = OR.condition_tokens(p, lang, img, oc, rb=rb_of(c))[blk]
    ckb, cvb = OR.cross_kv(p, blk, condb, oc, rb=rb_of(c))
    refb = OR.rdt_block(p, blk, x, ckb, cvb, ll if blk == 0 else None, oc, rb=rb_of(c))
    mx, mr = float(np.abs(got - ref32).max()), mean_rel(got, ref32)
    mr_model, mr_b = mean_rel(refb, ref32), mean_rel(got, refb)
    print(f"block {blk} B={batch} int8={int8}: vs fp32 max-abs {mx:.3e} mean-rel {mr:.3e}; "
          f"storage model vs fp32 {mr_model:.3e}; GPU vs storage model {mr_b:.3e}", flush=True)
    assert np.isfinite(got).all()
    assert mx <= 2e-2
    assert mr <= 1e-3
    assert mr_b <= 1e-3


@pytest.mark.parametrize("batch,int8", [(16, 0), (32, 1)], ids=["b16", "int8_b32"])
def test_denoise_step_large_batch(batch, int8):
    """Config 4 at batch 16 and config 5 (int8 weights) at batch 32: every
    block GEMM has M = 67 * B > 160 rows, the hipBLASLt product + epilogue
    path (int8 codes widened exactly).  Two layers, reduced condition
    lengths, one step against the oracle at the bf16 noise floor."""
    print(f"denoise step batch={batch} int8={int8}", flush=True)
    c = small_cfg(layers=2, batch=batch, int8_weights=int8)
    m = build(c)
    lang_len = np.random.default_rng(batch).integers(8, c.lang_max + 1, size=batch).astype(np.int32)
    lang, ll, img, state = make_condition(c, lang_len=lang_len)
    set_cond(m, lang, ll, img, state)
    x_t = O.randn(99, (batch, c.horizon, c.action_dim))
    got = m.denoise_step(torch.from_numpy(x_t).to(DEV), 0.8).cpu().numpy()
    p = m.state_dict()
    oc = oracle_cfg(c)
    caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))
    ref, floor = oracle_noise_floor(lambda: OR.denoise_step(p, x_t, 0.8, state, caches, ll, oc, rb=rb_of(c)))
    print(f"batch {batch} int8 {int8}: mean-rel {mean_rel(got, ref):.3e} floor {floor:.3e}")
    assert_within_floor(got, ref, floor, f"denoise step B={batch} int8={int8}")


@pytest.mark.parametrize("batch,int8", [(16, 0), (32, 1), (32, 2)], ids=["b16", "int8_b32", "int8direct_b32"])
def test_loop_large_batch_graph_and_oracle(batch, int8):
    """The 5-step hipGraph loop at batch 16 / int8 batch 32: graph replays
    equal the eager loop bit for bit, and batch slots 0 and B-1 match the
    oracle's loop at the bf16 noise floor."""
    print(f"loop batch={batch} int8={int8}", flush=True)
    c = small_cfg(layers=2, batch=batch, int8_weights=int8)
    m = build(c)
    lang_len = np.random.default_rng(batch + 1).integers(8, c.lang_max + 1, size=batch).astype(np.int32)
    lang, ll, img, state = make_condition(c, lang_len=lang_len)
    set_cond(m, lang, ll, img, state)
    x0 = O.randn(17, (batch, c.horizon, c.action_dim))
    xe = torch.from_numpy(x0).to(DEV)
    m.sample(xe, use_graph=False)
    eager = xe.cpu().numpy()
    for _ in range(2):
        xg = torch.from_numpy(x0).to(DEV)
        m.sample(xg, use_graph=True)
        assert np.array_equal(xg.cpu().numpy(), eager)
    p = m.state_dict()
    oc = oracle_cfg(c)
    for b in (0, batch - 1):
        caches = OR.encode_caches(p, lang[b:b + 1], img[b:b + 1], oc, rb=rb_of(c))
        ref, floor = oracle_noise_floor(
            lambda: OR.sample(p, x0[b:b + 1], state[b:b + 1], caches, ll[b:b + 1], oc, rb=rb_of(c)))
        print(f"loop B={batch} slot {b}: mean-rel {mean_rel(eager[b:b + 1], ref):.3e} floor {floor:.3e}")
        assert_within_floor(eager[b:b + 1], ref, floor, f"loop B={batch} slot {b}")


@pytest.mark.parametrize("batch,int8", [(3, 0), (3, 1), (3, 2), (1, 0)])
def test_weight_writes_reach_the_fp16_copies(batch, int8):
    """The runtime multiplies fp16 copies of weights -- above 160 rows every
    projection's, at batch 1 with bf16 weights the FFN matrices' -- rebuilt
    before a pass only when the parameters may have changed.  A write
    through sf_rdt_param_data after a pass (param_write), and a write
    through a pointer taken before a pass followed by sf_rdt_params_changed,
    both reach the next graph replay: its result matches the oracle on the
    new weights (a stale copy would give the old weights' result)."""
    import ctypes
    c = small_cfg(layers=2, batch=batch, int8_weights=int8)
    m = build(c)
    lang, ll, img, state = make_condition(c)
    set_cond(m, lang, ll, img, state)
    x0 = O.randn(41, (c.batch, c.horizon, c.action_dim))

    def loop():
        x = torch.from_numpy(x0).to(DEV)
        m.sample(x, use_graph=True)
        return x.cpu().numpy()

    base = loop()
    oc = oracle_cfg(c)
    for how in ("param_write", "raw_pointer"):
        name = "blocks.1.ffn.fc2.weight"
        idx = R.lib().sf_rdt_find_param(m.h, name.encode())
        p0 = m.state_dict()
        if int8:
            # new codes, same row scales: negate every code of the matrix
            q = np.empty(p0[name].shape, np.int8)
            ptr = R.lib().sf_rdt_param_data(m.h, idx)
            R._memcpy_d2h(q, ptr)
            newv = (-q.astype(np.int16)).clip(-127, 127).astype(np.int8)
        else:
            newv = O.bf16_round(-p0[name])
            newv = (newv.view(np.uint32) >> 16).astype(np.uint16)
        if how == "param_write":
            loop()                     # a pass first: the copies are current
            m.param_write(idx, newv.reshape(-1))
        else:
            ptr = R.lib().sf_rdt_param_data(m.h, idx)   # pointer taken before the pass
            loop()
            R._hipmemcpy(ptr, np.ascontiguousarray(newv).ctypes.data, newv.nbytes, 1)
            m.params_changed()
        got = loop()
        p = m.state_dict()
        assert not np.array_equal(p[name], p0[name])
        caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))
        ref, floor = oracle_noise_floor(lambda: OR.sample(p, x0, state, caches, ll, oc, rb=rb_of(c)))
        print(f"{how} int8={int8}: mean-rel {mean_rel(got, ref):.3e} floor {floor:.3e}", flush=True)
        assert_within_floor(got, ref, floor, f"loop after {how}")
        assert not np.array_equal(got, base)
        base = got


def test_run_blocks_int8_large_batch_block_range():
    """sf_rdt_run_blocks on an int8 model at batch 32 (2144 rows, the
    library path) over blocks 1..2 of 3: the runtime widens the int8 codes
    of exactly the blocks it runs (a stale or missing copy would multiply by
    another block's weights); against the oracle's two-block stack."""
    print("run_blocks int8 batch 32 blocks 1..2", flush=True)
    c = small_cfg(layers=3, batch=32, int8_weights=1)
    m = build(c)
    lang, ll, img, state = make_condition(c)
    set_cond(m, lang, ll, img, state)
    x = O.randn(9, (c.batch, c.horizon + 3, c.hidden))
    xd = torch.from_numpy(x).to(DEV)
    m.run_blocks(xd, first=1, count=2)
    got = xd.cpu().numpy()
    p = m.state_dict()
    oc = oracle_cfg(c)
    caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))

    def stack():
        r = x
        for i in (1, 2):
            r = OR.rdt_block(p, i, r, caches[i][0], caches[i][1], ll if i % 2 == 0 else None, oc, rb_of(c))
        return r

    ref, floor = oracle_noise_floor(stack)
    mx, mr, scale = float(np.abs(got - ref).max()), mean_rel(got, ref), max(1.0, float(np.abs(ref).max()))
    print(f"int8 b32 blocks 1..2: max-abs {mx:.3e} (|ref| <= {scale:.2f}) mean-rel {mr:.3e} floor {floor:.3e}")
    # measured max-abs 2.8e-3 on 4.4M residual elements up to ~6.5 in
    # magnitude, mean-rel 1.09x the floor: 2x margins (another block's
    # weights would put mean-rel near 1)
    assert np.isfinite(got).all()
    assert mx <= 6e-3 and mr <= 2 * floor


@pytest.mark.parametrize("int8", [0, 1])
def test_odd_shapes_denoise_step(int8):
    """A configuration off the RDT-1B grid: hidden 1024 (16 heads), 3
    blocks, batch 3 (201 rows per projection: the library path), 77
    language and 129 image condition tokens.  B*H = 48 leaves the
    query-block grid's last head group padded; the language blocks (0, 2)
    project their K/V as one GEMM, the single image block per call; lengths
    off every multiple of 16.  Denoise step against the oracle."""
    print(f"odd shapes int8={int8}", flush=True)
    c = small_cfg(hidden=1024, heads=16, layers=3, batch=3, lang_max=77, img_len=129, int8_weights=int8)
    m = build(c)
    lang, ll, img, state = make_condition(c, lang_len=[5, 40, 77])
    set_cond(m, lang, ll, img, state)
    x_t = O.randn(98, (c.batch, c.horizon, c.action_dim))
    v = m.denoise_step(torch.from_numpy(x_t).to(DEV), 0.6)
    got = v.cpu().numpy()
    p = m.state_dict()
    oc = oracle_cfg(c)
    caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))
    for i in range(c.layers):
        for wv in (0, 1):
            assert mean_rel(m.cache_numpy(i, wv), caches[i][wv]) < 2e-3, (i, wv)
    ref, floor = oracle_noise_floor(lambda: OR.denoise_step(p, x_t, 0.6, state, caches, ll, oc, rb=rb_of(c)))
    print(f"odd shapes int8={int8}: mean-rel {mean_rel(got, ref):.3e} floor {floor:.3e}")
    assert_within_floor(got, ref, floor, f"odd shapes int8={int8}")


# ---- config 3 as written: the MLP 4x block ------------------------------------

def test_mlp4x_block_stack():
    """The benchmarked block-stack configuration names an MLP 4x block (fc1 2048 -> 8192, fc2
    8192 -> 2048); the reference's RDT-1B has 1x (config.h:60-61), so this
    is the synthetic variant.  Two full-width blocks against the oracle."""
    print("mlp4x block stack", flush=True)
    c = small_cfg(layers=2, batch=1, mlp_ratio=4)
    m = build(c)
    shapes = {nm: sh for nm, _, sh in m.params()}
    assert shapes["blocks.0.ffn.fc1.weight"] == (4 * c.hidden, c.hidden)
    assert shapes["blocks.0.ffn.fc2.weight"] == (c.hidden, 4 * c.hidden)
    lang, ll, img, state = make_condition(c)
    set_cond(m, lang, ll, img, state)
    x = O.randn(5, (1, c.horizon + 3, c.hidden))
    xd = torch.from_numpy(x).to(DEV)
    m.run_blocks(xd)
    got = xd.cpu().numpy()
    p = m.state_dict()
    oc = oracle_cfg(c)
    caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))

    def stack():
        r = x
        for i in range(c.layers):
            r = OR.rdt_block(p, i, r, caches[i][0], caches[i][1], ll if i % 2 == 0 else None, oc, rb_of(c))
        return r

    ref, floor = oracle_noise_floor(stack)
    print(f"mlp4x: mean-rel {mean_rel(got, ref):.3e} floor {floor:.3e}")
    assert_within_floor(got, ref, floor, "MLP 4x two-block stack")


# ---- full depth: batch slots against batch-1 runs -----------------------------

def test_full_depth_batch16_slots_match_batch1():
    """28 layers, full condition lengths, 5-step graph loop at batch 16:
    slots 0, 7 and 15 against batch-1 models given the same slot's
    condition and noise.  The two runs take different GEMM paths (hipBLASLt
    in fp16 at M = 1072 vs split-K at M = 67) and storage types, so they
    differ by rounding: measured 1.4-1.6e-3 mean-rel on the action update
    after 28 x 5 block applications, bound 3e-3 (about 2x)."""
    print("full depth batch 16 vs batch 1", flush=True)
    c16 = R.default_config(batch=16)
    c1 = R.default_config(batch=1)
    m16 = build(c16)
    lang_len = np.random.default_rng(3).integers(32, 1025, size=16).astype(np.int32)
    lang, ll, img, state = make_condition(c16, lang_len=lang_len)
    set_cond(m16, lang, ll, img, state)
    x0 = O.randn(21, (16, c16.horizon, c16.action_dim))
    x16 = torch.from_numpy(x0).to(DEV)
    m16.sample(x16, use_graph=True)
    a16 = x16.cpu().numpy()
    del m16
    torch.cuda.synchronize()
    m1 = build(c1)
    for b in (0, 7, 15):
        set_cond(m1, lang[b:b + 1], ll[b:b + 1], img[b:b + 1], state[b:b + 1])
        x1 = torch.from_numpy(x0[b:b + 1].copy()).to(DEV)
        m1.sample(x1, use_graph=True)
        a1 = x1.cpu().numpy()
        mr = mean_rel(a16[b:b + 1] - x0[b:b + 1], a1 - x0[b:b + 1])
        print(f"slot {b}: mean-rel of the action update {mr:.3e}, max-abs {np.abs(a16[b:b + 1] - a1).max():.3e}")
        assert np.isfinite(a1).all()
        assert mr <= 3e-3, (b, mr)


def _full_size_condition():
    c = R.default_config(batch=32)
    lang_len = np.random.default_rng(32).integers(32, c.lang_max + 1, size=32).astype(np.int32)
    return make_condition(c, lang_len=lang_len)


def _full_size_int8_b32_loop(int8_weights, cond):
    """Config 5 at full size (28 layers, hidden 2048, int8 weights, batch 32,
    ragged language rows, 4374 image keys), the 5-step loop from seeded
    noise: checks graph == eager (twice), finiteness and that every slot
    moved; returns (x0, the eager result)."""
    c = R.default_config(batch=32, int8_weights=int8_weights)
    m = build(c)
    set_cond(m, *cond)
    x0 = O.randn(23, (32, c.horizon, c.action_dim))
    xe = torch.from_numpy(x0).to(DEV)
    m.sample(xe, use_graph=False)
    eager = xe.cpu().numpy()
    assert np.isfinite(eager).all()
    moved = np.abs(eager - x0).reshape(32, -1).max(axis=1)
    assert (moved > 0).all(), moved
    for rep in range(2):
        xg = torch.from_numpy(x0).to(DEV)
        m.sample(xg, use_graph=True)
        assert np.array_equal(xg.cpu().numpy(), eager), rep
    m.close()
    print(f"int8 b32 full size (int8_weights {int8_weights}): finite, graph == eager, "
          f"min per-slot move {moved.min():.3e}", flush=True)
    return x0, eager


def test_full_size_int8_batch32_graph_loop():
    """Config 5 at full size: 28 layers, hidden 2048, int8 weights, batch
    32, full condition lengths (ragged language rows, 4374 image keys), the
    5-step loop.  Properties that do not need the oracle at this size: the
    graph replays equal the eager loop bit for bit (twice), every action
    stays finite, and each batch slot moved from its noise."""
    print("full-size int8 batch 32 loop", flush=True)
    _full_size_int8_b32_loop(1, _full_size_condition())


def test_full_size_int8_batch32_direct_matches_copies():
    """The same full-size loop with int8_weights = 2 (every block matrix's
    codes read directly, no fp16 copies): graph == eager, finite, and each
    slot's action update within 1.5e-3 mean-rel of the int8_weights = 1
    loop (fp16 copies of the same codes: the same storage points, other
    summation orders; measured 4.4e-4 for the worst slot)."""
    print("full-size int8 batch 32 loop, codes read directly vs fp16 copies", flush=True)
    cond = _full_size_condition()
    x0, ref = _full_size_int8_b32_loop(1, cond)
    _, got = _full_size_int8_b32_loop(2, cond)
    for b in range(32):
        mr = mean_rel(got[b] - x0[b], ref[b] - x0[b])
        assert mr <= 1.5e-3, (b, mr)
    print(f"direct vs copies: worst slot mean-rel "
          f"{max(mean_rel(got[b] - x0[b], ref[b] - x0[b]) for b in range(32)):.3e}", flush=True)


# ---- V beyond the fp16 range: the layer switches to the exact P.V form --------

def test_large_v_runs_exact_form_and_stays_finite():
    """The fast P.V form converts V to fp16; a cached V element of
    magnitude >= 65504 would turn its output column inf/NaN there.  The
    runtime measures each layer's max |V| when the condition is set and runs
    such a layer in the exact bf16 form: the loop stays finite and matches
    the oracle (which takes any finite V), the other layer keeps the fp16
    form, and restoring the weights returns both to it with the earlier
    result reproduced bit for bit."""
    c = small_cfg(layers=2, batch=1)
    m = build(c)
    lang, ll, img, state = make_condition(c)
    set_cond(m, lang, ll, img, state)
    assert (m.pv_exact(0), m.pv_exact(1)) == (0, 0)
    x0 = O.randn(31, (1, c.horizon, c.action_dim))

    def run():
        x = torch.from_numpy(x0).to(DEV)
        m.sample(x, use_graph=True)
        return x.cpu().numpy()

    base = run()
    idx = R.lib().sf_rdt_find_param(m.h, b"blocks.1.cross_attn.kv.bias")
    col = c.hidden + 5                      # V section, head 0, dim 5
    old = m.state_dict()["blocks.1.cross_attn.kv.bias"][col:col + 1].copy()
    m.param_write(idx, np.array([70000.0], np.float32), offset=col)
    set_cond(m, lang, ll, img, state)
    assert (m.pv_exact(0), m.pv_exact(1)) == (0, 1)
    assert float(np.abs(m.cache_numpy(1, 1)).max()) >= 65504.0
    got = run()
    assert np.isfinite(got).all()
    xe = torch.from_numpy(x0).to(DEV)
    m.sample(xe, use_graph=False)
    assert np.array_equal(xe.cpu().numpy(), got)
    p = m.state_dict()
    oc = oracle_cfg(c)
    caches = OR.encode_caches(p, lang, img, oc, rb=rb_of(c))
    ref, floor = oracle_noise_floor(lambda: OR.sample(p, x0, state, caches, ll, oc, rb=rb_of(c)))
    print(f"large V: mean-rel {mean_rel(got, ref):.3e} floor {floor:.3e}")
    assert_within_floor(got, ref, floor, "loop with |V| >= 65504 in layer 1")
    m.param_write(idx, old, offset=col)
    set_cond(m, lang, ll, img, state)
    assert (m.pv_exact(0), m.pv_exact(1)) == (0, 0)
    assert np.array_equal(run(), base)
