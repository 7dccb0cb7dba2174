#!/usr/bin/env python3
"""Benchmark of the RDT-1B denoise loop and its attention hot path on one MI355X.

Prints ONE JSON line (the driver's contract).

Headline (`value`, the denoise-loop configuration at batch 1): latency of one full
denoise loop -- 5 Euler steps of the 28-layer RDT-1B (hidden 2048, 32 heads,
67 tokens, FFN 1x) with the condition K/V projected once per inference and
cached -- replayed as one hipGraph.  One bench "step" is one such inference
(graph replay, input copy-in and result copy-out included); inputs are
synthetic and resident in HBM; weights are random-init (std 0.02, RMSNorm
gamma = 1).  Timing uses HIP events on the stream the graph runs on.

`roofline` is the metric's second half: the image cross-attention op the loop
runs (67 queries x 4374 cached keys, 32 heads x 64, bf16, batch 1), algorithmic
bytes (K and V once, Q in, O out) over its measured duration against the 8 TB/s
HBM peak.  `extra` reports the other configs: cross-attention batch 8 and
language keys with valid lengths (config 2), the block stack (config 3), the
loop at batch 16 (config 4) and the int8-weight loop at batch 32 (config 5),
and the one-time condition encode, plus the MFMA utilisation the north star
asks for: the self-attention op and the block projections (`GEMM_SHAPES`:
batch 1 split-K, batch 16/32 and the condition projection on the library
path) as algorithmic TFLOP/s over the 2.5 PFLOP/s dense bf16 peak, and for
the batch-1 (weight-streaming) shapes their HBM rate.

`cpu_baseline` is the CPU oracle (oracle/, the fp32 restatement of the
reference's RDTBlock / denoise_step / naive attention) timed on the host
cores: one full 28-layer denoise step, scaled by 5 to a loop.  `extra`
also carries the oracle's attention ops of configs 1 and 2 on the host
(`cpu_self_b1_ms`, `cpu_cross_img_b1_ms`) beside their GPU times.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "RDT-1B denoise-loop latency ms (bs=1) + cross-attn HBM GB/s vs roofline"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
# HBM bytes per roofline op measured with rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE
# (x2.0 / x1.0, scales read off a 256 MiB copy kernel) on `bench.py
# --profile-roofline`: ring kernel 18650.9 KiB fetched (38.20 MB read) +
# 5123.1 KiB written, merge 2182.0 KiB fetched + 268.0 KiB written
# (profiles/cross_attention_image_roofline.md).  Re-measured whenever the
# attention kernels change.
TRAFFIC_B1_IMAGE_BYTES = 48186266
TRAFFIC_B8_IMAGE_BYTES = 291492659   # same profile, batch-8 op (no key split)


def attn_bytes(B, H, Sq, Sk_valid_total, D=64, eb=2):
    """Algorithmic HBM bytes of one attention op: K and V once, Q in, O out."""
    return 2 * H * Sk_valid_total * D * eb + 2 * B * H * Sq * D * eb


def attn_flops(H, Sq, Sk_valid_total, D=64):
    return 4 * H * Sq * Sk_valid_total * D


def _events():
    import torch

    return torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)


def time_graph(fn, steps, warmup, reps=20):
    """Captures `reps` back-to-back calls of fn in one HIP graph and times
    `steps` replays with HIP events on the capturing stream; ms per call."""
    import torch

    fn()
    torch.cuda.synchronize()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(s):
        with torch.cuda.graph(g, stream=s):
            for _ in range(reps):
                fn()
    torch.cuda.current_stream().wait_stream(s)
    stream = torch.cuda.current_stream()
    for _ in range(warmup):
        g.replay()
    torch.cuda.synchronize()
    start, stop = _events()
    start.record(stream)
    for _ in range(steps):
        g.replay()
    stop.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / (steps * reps)


# Working set of the graph-timed attention ops: K and V are cycled through
# enough distinct copies that one graph's calls touch at least this many
# bytes, twice the 256 MB memory-side cache (MALL), so every call streams its
# K/V from HBM as the denoise loop does (each layer's cache is read once per
# step, ~0.6 GB per step at batch 1).  Re-reading one K/V set call after call
# would serve part of it from the MALL instead.
COLD_SET_BYTES = 512 << 20


def bench_attention(B, Sk, steps, warmup, valid=None, Sq=67, H=32, exact_pv=False, reps=20, v16=None):
    """Graph-timed cross-attention op (exact_pv: the bf16 (hi, lo) P.V form
    instead of the default fp16 one): `reps` calls per graph, call i reading
    K/V copy i % n_sets (COLD_SET_BYTES).  v16 (default: the cross-attention
    calls, Sk > 128, on the fp16 form): V given in fp16, as the model runtime
    holds its cached V for that form (sf_attn_desc.v_f16); the self-attention
    (Sk <= 128) reads bf16 V from its projection."""
    import numpy as np
    import torch

    from servoflow_amd.attention import attention, make_desc, workspace_bytes

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(1234 + B + Sk)
    kv_bytes = 2 * B * H * Sk * 64 * 2
    n_sets = int(min(reps, max(1, -(-COLD_SET_BYTES // kv_bytes))))
    q = torch.randn(B, H, Sq, 64, device=dev, generator=g).to(torch.bfloat16)
    ks = [torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16) for _ in range(n_sets)]
    if v16 is None:
        v16 = Sk > 128 and not exact_pv
    vdt = torch.float16 if v16 else torch.bfloat16
    vs = [torch.randn(B, H, Sk, 64, device=dev, generator=g).to(torch.bfloat16).to(vdt) for _ in range(n_sets)]
    # output straight into [B, Sq, H*D], the layout the block's projection reads
    out = torch.empty(B, Sq, H, 64, device=dev, dtype=torch.bfloat16).permute(0, 2, 1, 3)
    vl = None
    if valid is not None:
        vl = torch.from_numpy(np.asarray(valid, np.int32)).to(dev)
    desc = make_desc(q, ks[0], vs[0], out, valid_len=vl)
    ws = torch.zeros(max(workspace_bytes(desc), 16), dtype=torch.uint8, device=dev)
    calls = [0]

    def fn():
        i = calls[0] % n_sets
        calls[0] += 1
        attention(q, ks[i], vs[i], out=out, valid_len=vl, workspace=ws, exact_pv=exact_pv)

    ms = time_graph(fn, steps, warmup, reps=reps)
    sk_total = B * Sk if valid is None else int(np.sum(valid))
    nbytes = attn_bytes(B, H, Sq, sk_total)
    res = {"us": ms * 1e3, "bytes": nbytes, "GBps": nbytes / (ms * 1e-3) / 1e9,
           "TFLOPs": attn_flops(H, Sq, sk_total) / (ms * 1e-3) / 1e12,
           "frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, "kv_sets": n_sets}
    del ks, vs
    torch.cuda.empty_cache()
    return res


def bench_gemm(M, N, K, steps, warmup, int8=False, epilogue="plain", a16=False, w16=False):
    """Graph-timed block projection C[M,N] = A[M,K] W[N,K]^T + bias through
    sf_gemm with a caller workspace (split-K kernel + reduce for M <= 160;
    above, hipBLASLt writes the bf16 C with its bias epilogue, int8 codes
    widened first and their row scales as its alpha vector; the shape is
    prepared first, as the model runtime does).  The graph's calls cycle through distinct weight
    copies totalling >= COLD_SET_BYTES (at most 64 calls), so weights stream
    from HBM as in the loop, where each is read once per step.  epilogue:
    "plain" (bf16 out) or "addnorm" (fp32 residual += product, then RMSNorm
    to bf16).  a16: fp16 activations and an fp16 C -- with int8 weights
    above 160 rows the direct int8 kernel (no 16-bit weight copy), or with
    w16 hipBLASLt on fp16 copies of the weights (the int8_weights = 1
    runtime's product).  Returns
    time, MFMA rate against the dense bf16 peak and the weight-streaming HBM
    rate."""
    import ctypes

    import torch

    from servoflow_amd import abi, kernels

    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(M + N + K)
    wbytes = N * K * (1 if int8 else 2)
    n_sets = int(min(64, max(1, -(-COLD_SET_BYTES // wbytes))))
    a = torch.randn(M, K, device=dev, generator=g).to(torch.float16 if a16 else torch.bfloat16)
    if int8:
        ws_ = [torch.randint(-127, 128, (N, K), device=dev, generator=g, dtype=torch.int32).to(torch.int8)
               for _ in range(n_sets)]
        scale = torch.rand(N, device=dev, generator=g) * 1e-3
    else:
        ws_ = [(torch.randn(N, K, device=dev, generator=g) * 0.02).to(torch.bfloat16) for _ in range(n_sets)]
        scale = None
    bias = torch.randn(N, device=dev, generator=g) * 0.02
    d = kernels._desc(a, ws_[0], bias, abi.SF_ACT_NONE, scale)
    wsp = torch.empty(max(int(abi.lib().sf_gemm_workspace_bytes(ctypes.byref(d))), 16),
                      dtype=torch.uint8, device=dev)
    if epilogue == "addnorm":
        res = torch.randn(M, N, device=dev, generator=g)
        gamma = torch.ones(N, device=dev)
        out = torch.empty(M, N, dtype=torch.bfloat16, device=dev)
        d.epilogue = abi.SF_EPI_ADD_NORM
        d.C, d.ldc, d.c_dtype = res.data_ptr(), res.stride(0), abi.SF_F32
        d.eps = 1e-6
        d.norm_gamma, d.norm_out = gamma.data_ptr(), out.data_ptr()
        d.norm_ldo, d.norm_dtype = out.stride(0), abi.SF_BF16
    else:
        out = torch.empty(M, N, dtype=torch.float16 if a16 else torch.bfloat16, device=dev)
        d.epilogue = abi.SF_EPI_PLAIN
        d.C, d.ldc, d.c_dtype = out.data_ptr(), out.stride(0), abi.SF_F16 if a16 else abi.SF_BF16
    d.workspace, d.workspace_bytes = wsp.data_ptr(), wsp.numel()
    copies = [c for i in range(0, n_sets, 8) for c in kernels.weights_to_f16(ws_[i:i + 8])] if w16 else []
    if w16:
        d.w_codes16, d.w16_f16 = copies[0].data_ptr(), 1
    abi.check(abi.lib().sf_gemm_prepare(ctypes.byref(d)), "sf_gemm_prepare")
    descs = []
    for i, w in enumerate(ws_):
        di = abi.GemmDesc()
        ctypes.pointer(di)[0] = d
        di.W = w.data_ptr()
        if w16:
            di.w_codes16 = copies[i].data_ptr()
        descs.append(di)
    calls = [0]

    def fn():
        di = descs[calls[0] % n_sets]
        calls[0] += 1
        abi.check(abi.lib().sf_gemm(ctypes.byref(di), torch.cuda.current_stream(dev).cuda_stream), "sf_gemm")

    ms = time_graph(fn, steps, warmup, reps=max(20, n_sets))
    del ws_, copies
    torch.cuda.empty_cache()
    flops = 2.0 * M * N * K
    nbytes = wbytes + M * K * 2 + M * N * 2
    return {"us": ms * 1e3, "TFLOPs": flops / (ms * 1e-3) / 1e12,
            "mfma_frac": flops / (ms * 1e-3) / 1e12 / MFMA_BF16_PEAK_TFLOPS,
            "GBps": nbytes / (ms * 1e-3) / 1e9, "hbm_frac": nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS,
            "w_sets": n_sets}


# Projection shapes of the block (M = batch * 67 tokens): the 2048-wide
# projections (proj, cross-q, cross-proj, fc1, fc2), the fused QKV, and the
# one-time condition K/V projection of the image tokens (M = 4374 per batch).
GEMM_SHAPES = (
    ("proj_b1", 67, 2048, 2048, False),
    ("proj_int8_b1", 67, 2048, 2048, True),
    ("qkv_b1", 67, 6144, 2048, False),
    ("proj_b16", 1072, 2048, 2048, False),
    ("qkv_b16", 1072, 6144, 2048, False),
    ("proj_int8_b32", 2144, 2048, 2048, True),
    ("proj_int8_direct_b32", 2144, 2048, 2048, 2),   # fp16 activations, int8 read directly
    ("kv_img_b1", 4374, 4096, 2048, False),
)


def make_model(B, int8=False, seed=1234, mlp_ratio=1, lens_out=None):
    """RDT-1B (28 layers) with random weights and a synthetic condition:
    language N(0,1) with valid lengths ~ U{32..1024}, image N(0,1) 4374 tokens,
    state token N(0,1).  int8: 0 bf16 weights, 1 int8 (fp16 copies above
    160 rows), 2 int8 read directly (sf_rdt_config.int8_weights).  Returns
    (model, encode_ms); lens_out (a list) receives the drawn language
    lengths."""
    import numpy as np
    import torch

    from servoflow_amd import rdt as R

    cfg = R.default_config(batch=B, int8_weights=int(int8), mlp_ratio=mlp_ratio)
    m = R.RdtModel(cfg)
    m.init_random(seed, 0.02)
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(seed + B)
    lang = torch.randn(B, cfg.lang_max, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    img = torch.randn(B, cfg.img_len, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    state = torch.randn(B, cfg.hidden, device=dev, generator=g).to(torch.bfloat16)
    rng = np.random.default_rng(seed + B)
    lens = rng.integers(32, 1025, size=B).astype(np.int32)
    if lens_out is not None:
        lens_out.extend(int(x) for x in lens)
    ll = torch.from_numpy(lens).to(dev)
    if B == 1:   # the caller's language tensor holds L = lens[0] rows (the reference's [1, L, 4096])
        m.set_lang_rows(int(lens[0]))
    m.set_condition(lang, ll, img, state)          # warm-up (first launch of each kernel)
    torch.cuda.synchronize()
    start, stop = _events()
    start.record()
    m.set_condition(lang, ll, img, state)
    stop.record()
    torch.cuda.synchronize()
    del lang, img
    return m, start.elapsed_time(stop)


def bench_loop(m, steps, warmup):
    """ms per graph-replayed 5-step denoise loop (copy-in/out included)."""
    import torch

    cfg = m.cfg
    dev = torch.device("cuda:0")
    x0 = torch.randn(cfg.batch, cfg.horizon, cfg.action_dim, device=dev)
    x = x0.clone()
    m.sample(x, use_graph=True)          # capture + first replay
    for _ in range(warmup):
        x.copy_(x0)
        m.sample(x, use_graph=True)
    torch.cuda.synchronize()
    start, stop = _events()
    start.record()
    for _ in range(steps):
        m.sample(x, use_graph=True)
    stop.record()
    torch.cuda.synchronize()
    if not torch.isfinite(x).all():
        raise RuntimeError("non-finite sampler output")
    return start.elapsed_time(stop) / steps


def bench_infer(m, steps):
    """sf_rdt_infer (InferenceEngine::infer) at the model's batch: raw
    tokens in (T5 language 1024 x 4096, SigLIP image 4374 x 1152, state),
    the action chunk out in host memory, stream synchronised.  A new frame id
    on every call re-encodes the condition (adaptors + every layer's K/V
    projection) before the 5-step graph loop; the same frame id reuses it.
    Returns (ms per call with a new frame, ms per call with the cached
    condition), host wall clock around the synchronous call."""
    import numpy as np
    import torch

    cfg = m.cfg
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev)
    g.manual_seed(77)
    B = cfg.batch
    lt = torch.randn(B, cfg.lang_max, cfg.lang_token_dim, device=dev, generator=g).to(torch.bfloat16)
    it = torch.randn(B, cfg.img_len, cfg.img_token_dim, device=dev, generator=g).to(torch.bfloat16)
    st = torch.randn(B, cfg.state_dim, device=dev, generator=g).to(torch.bfloat16)
    lens = np.random.default_rng(5).integers(32, 1025, size=B).astype(np.int32)
    ll = torch.from_numpy(lens).to(dev)
    if B == 1:
        m.set_lang_rows(int(lens[0]))
    m.infer(1, lt, ll, it, st, noise_seed=3)          # capture / warm-up
    m.infer(2, lt, ll, it, st, noise_seed=3)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(steps):
        _, enc = m.infer(100 + i, lt, ll, it, st, noise_seed=3 + i)
        assert enc
    new_ms = (time.perf_counter() - t0) * 1e3 / steps
    t0 = time.perf_counter()
    for i in range(steps):
        out, enc = m.infer(100 + steps - 1, lt, ll, it, st, noise_seed=3 + i)
        assert not enc
    cached_ms = (time.perf_counter() - t0) * 1e3 / steps
    if not np.isfinite(out).all():
        raise RuntimeError("non-finite action chunk")
    return new_ms, cached_ms


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def bench_blocks(m, steps):
    """Config 3: the 28-block stack, one denoise step's worth, eager launches."""
    import torch

    cfg = m.cfg
    x = torch.randn(cfg.batch, cfg.horizon + 3, cfg.hidden, device="cuda:0")
    m.run_blocks(x)
    torch.cuda.synchronize()
    start, stop = _events()
    start.record()
    for _ in range(steps):
        m.run_blocks(x)
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / steps


def gemm_picks(B, int8):
    """Which hipBLASLt algorithm the model's block projections run at batch
    B (sf_gemm_algo_pick; call after make_model, which prepares every
    shape): the QKV product (fp16 rows + bias), a 2048-wide projection into
    the residual add + norm (fp16 product) and fc1 (fp16 C with GELU +
    bias).  Each: index in hipBLASLt's heuristic list / candidates, and
    whether it was timed."""
    import ctypes

    from servoflow_amd import abi

    M = 67 * B
    res = {}
    for name, N, addnorm, act in (("qkv", 6144, False, abi.SF_ACT_NONE), ("proj", 2048, True, abi.SF_ACT_NONE),
                                  ("fc1", 2048, False, abi.SF_ACT_GELU_TANH)):
        d = abi.GemmDesc()
        d.M, d.N, d.K, d.lda, d.ldw = M, N, 2048, 2048, 2048
        d.a_dtype, d.w_dtype, d.w16_f16 = abi.SF_F16, abi.SF_I8 if int8 else abi.SF_BF16, 1
        d.bias, d.act = 256, act   # any non-null bias: the kind, not the data, is looked up
        if addnorm:
            d.epilogue, d.round_product, d.c_dtype, d.ldc = abi.SF_EPI_ADD_NORM, 1, abi.SF_F32, N
        else:
            d.epilogue, d.c_dtype, d.ldc = abi.SF_EPI_PLAIN, abi.SF_F16, N
        pick, ncand, timed = ctypes.c_int32(), ctypes.c_int32(), ctypes.c_int32()
        st = abi.lib().sf_gemm_algo_pick(ctypes.byref(d), ctypes.byref(pick), ctypes.byref(ncand), ctypes.byref(timed))
        res[name] = f"{pick.value}/{ncand.value} {'timed' if timed.value else 'heuristic'}" if st == 0 else "n/a"
    return res


def cpu_baseline(budget_s=25.0, lang_len=517):
    """The oracle's fp32 RDT-1B denoise step (28 layers, batch 1, image keys
    4374, language 1024 padded keys with valid length lang_len -- the
    headline's drawn L) on the host cores.
    Weights are N(0, 0.02); one layer's weights are shared by all 28 layers
    (the timing does not depend on the values) and the condition caches are
    random.  One step is timed and scaled by 5 to the loop."""
    import numpy as np

    from oracle import oracle as O
    from oracle import rdt as OR

    c = OR.RdtConfig()
    D = c.hidden
    seeds = iter(range(1, 1000))

    def mat(N, K):
        return O.bf16_round(O.randn(next(seeds), (N, K), 0.02))

    def vec(N):
        return O.randn(next(seeds), (N,), 0.02)

    p = {}
    shared = {
        "attn.qkv.weight": mat(3 * D, D), "attn.qkv.bias": vec(3 * D),
        "attn.proj.weight": mat(D, D), "attn.proj.bias": vec(D),
        "cross_attn.q.weight": mat(D, D), "cross_attn.q.bias": vec(D),
        "cross_attn.proj.weight": mat(D, D), "cross_attn.proj.bias": vec(D),
        "ffn.fc1.weight": mat(D, D), "ffn.fc1.bias": vec(D),
        "ffn.fc2.weight": mat(D, D), "ffn.fc2.bias": vec(D),
    }
    ones_d, ones_64 = np.ones(D, np.float32), np.ones(64, np.float32)
    for i in range(c.layers):
        pre = f"blocks.{i}."
        for k, v in shared.items():
            p[pre + k] = v
        for nm in ("norm1", "norm2", "norm3"):
            p[pre + nm + ".weight"] = ones_d
        for nm in ("attn.q_norm", "attn.k_norm", "cross_attn.q_norm", "cross_attn.k_norm"):
            p[pre + nm + ".weight"] = ones_64
    for a, k in (("state_adaptor.0", 2 * c.state_dim), ("state_adaptor.2", D), ("state_adaptor.4", D),
                 ("t_embedder.mlp.0", c.freq_dim), ("t_embedder.mlp.2", D),
                 ("freq_embedder.mlp.0", c.freq_dim), ("freq_embedder.mlp.2", D),
                 ("final_layer.ffn_final.fc1", D)):
        p[a + ".weight"], p[a + ".bias"] = mat(D, k), vec(D)
    p["final_layer.ffn_final.fc2.weight"] = mat(c.action_dim, D)
    p["final_layer.ffn_final.fc2.bias"] = vec(c.action_dim)
    p["final_layer.norm_final.weight"] = ones_d
    p["x_pos_embed"] = O.randn(900, (1, c.seq, D), 0.02)
    lang_k = O.bf16_round(O.randn(901, (1, c.heads, c.lang_max, 64)))
    img_k = O.bf16_round(O.randn(902, (1, c.heads, c.img_len, 64)))
    caches = [(lang_k, lang_k) if i % 2 == 0 else (img_k, img_k) for i in range(c.layers)]
    state = O.randn(903, (1, D))
    x_t = O.randn(904, (1, c.horizon, c.action_dim))
    ll = np.array([lang_len], np.int32)
    times = []
    t_end = time.perf_counter() + budget_s
    while not times or (time.perf_counter() < t_end and len(times) < 3):
        t0 = time.perf_counter()
        OR.denoise_step(p, x_t, 1.0, state, caches, ll, c, rb=False)
        times.append(time.perf_counter() - t0)
    step_s = float(np.median(times))
    cores = int(os.environ.get("OMP_NUM_THREADS", os.cpu_count() or 1))
    return {
        "value": round(step_s * c.num_steps * 1e3, 1),
        "unit": "ms",
        "cores": cores,
        "cpu_model": cpu_model(),
        "host_cpus": os.cpu_count(),
        "kind": "port",
        "sample": f"{len(times)} timed fp32 oracle denoise step(s) (28 layers, batch 1, lang 1024 "
                  f"keys with valid length {lang_len}, image 4374 keys), median {step_s * 1e3:.0f} ms, x5 steps",
    }


def cpu_attention_ops():
    """The attention ops of configs 1 and 2 on the host cores: the oracle's
    fp32 restatement of naive_attention_kernel (attention.cu:90-139), median
    of 3 runs each -- the self-attention op (1 x 32 heads x 67 x 67 x 64,
    fp32) and the batch-1 image cross-attention op (67 queries x 4374 keys)."""
    import numpy as np

    from oracle import oracle as O

    def med(fn):
        ts = []
        for _ in range(3):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return float(np.median(ts)) * 1e3

    q = O.randn(31, (1, 32, 67, 64))
    k, v = O.randn(32, (1, 32, 67, 64)), O.randn(33, (1, 32, 67, 64))
    self_ms = med(lambda: O.attention_f32(q, k, v))
    k, v = O.bf16_round(O.randn(34, (1, 32, 4374, 64))), O.bf16_round(O.randn(35, (1, 32, 4374, 64)))
    cross_ms = med(lambda: O.attention_f32(q, k, v))
    return {"cpu_self_b1_ms": round(self_ms, 3), "cpu_cross_img_b1_ms": round(cross_ms, 3)}


def profile_roofline(iters=50):
    """Runs only what the roofline profiles measure, through the same
    graph-timed function the bench line uses (bench_attention: 20 calls per
    graph, HIP events on the capturing stream): the batch-1 image
    cross-attention op (attn_ring_kernel + attn_merge_kernel) and the
    batch-8 one (attn_ring_kernel alone: no key split), then a plain 256 MiB
    device-to-device copy `iters` times -- the calibration kernel whose
    FETCH_SIZE / WRITE_SIZE per dispatch give the counters' scale (256 MiB
    read, 256 MiB written)."""
    import torch

    for B in (1, 8):
        r = bench_attention(B, 4374, steps=5, warmup=1)
        print(f"profile: cross-attention {B}x32x67x4374x64, graph-timed {r['us']:.2f} us per op "
              f"(under the profiler)", flush=True)
    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {iters} copies of 256 MiB done", flush=True)


def profile_mfma():
    """Runs only what the MFMA-utilisation profile measures, through the same
    graph-timed functions the bench line uses: the batch-1 self-attention op
    (attn_short_kernel, 1x32x67x67x64) and the block projections of
    GEMM_SHAPES (split-K kernel + reduce at M = 67, hipBLASLt with its bias
    epilogue above)."""
    r = bench_attention(1, 67, steps=5, warmup=1)
    print(f"profile: self-attention 1x32x67x67x64, graph-timed {r['us']:.2f} us per op", flush=True)
    for name, M, N, K, int8 in GEMM_SHAPES:
        r = bench_gemm(M, N, K, steps=5, warmup=1, int8=bool(int8), a16=int8 == 2)
        print(f"profile: gemm {name} {M}x{N}x{K}{' int8' if int8 else ''}, graph-timed "
              f"{r['us']:.2f} us per call", flush=True)


def profile_int8_b32(iters=3):
    """Runs only what the int8 large-batch traffic profile measures: the
    2144 x 2048 x 2048 projection (int8 batch 32) with fp16 activations and
    an fp16 C through the graph-timed bench_gemm -- the direct int8 kernel,
    then hipBLASLt on fp16 copies of the codes -- and a plain 256 MiB
    device-to-device copy `iters` times (the counters' calibration)."""
    import torch

    for w16 in (False, True):
        r = bench_gemm(2144, 2048, 2048, steps=3, warmup=1, int8=True, a16=True, w16=w16)
        print(f"profile: int8 gemm 2144x2048x2048 {'hipBLASLt on fp16 copies' if w16 else 'direct'}, "
              f"graph-timed {r['us']:.2f} us per call", flush=True)
    dev = torch.device("cuda:0")
    src = torch.empty(256 << 20, dtype=torch.uint8, device=dev).fill_(1)
    dst = torch.empty_like(src)
    for _ in range(iters):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(f"profile: {iters} copies of 256 MiB done", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50, help="timed denoise-loop inferences")
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--quick", action="store_true", help="headline and roofline only")
    ap.add_argument("--profile-roofline", action="store_true",
                    help="run only the roofline op and the copy calibration kernel (for rocprofv3)")
    ap.add_argument("--profile-mfma", action="store_true",
                    help="run only the self-attention op and the projection GEMMs (for rocprofv3 --pmc)")
    ap.add_argument("--profile-int8", action="store_true",
                    help="run only the int8 batch-32 projection, direct and on fp16 copies (for rocprofv3 --pmc)")
    ap.add_argument("--profile-loop", choices=["b16", "b32int8", "b32int8direct"],
                    help="build one large-batch model and replay its loop 3 times (for rocprofv3)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU; --gpus {args.gpus} is not supported "
              "(every GPU box here has one MI355X).", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    torch.cuda.init()
    if args.profile_roofline:
        profile_roofline()
        return
    if args.profile_mfma:
        profile_mfma()
        return
    if args.profile_int8:
        profile_int8_b32()
        return
    if args.profile_loop:
        B, int8 = {"b16": (16, 0), "b32int8": (32, 1), "b32int8direct": (32, 2)}[args.profile_loop]
        m, _ = make_model(B, int8=int8)
        ms = bench_loop(m, 3, 1)
        print(f"profile: loop batch {B}{' int8' if int8 else ''}: {ms:.3f} ms", flush=True)
        m.close()
        return
    extra = {}
    # ---- headline: batch-1 loop (config 4)
    lens1 = []
    m1, enc1 = make_model(1, lens_out=lens1)
    L1 = lens1[0]
    loop1 = bench_loop(m1, args.steps, args.warmup)
    extra["encode_condition_b1_ms"] = round(enc1, 3)
    if not args.quick:
        extra["block_stack_b1_ms"] = round(bench_blocks(m1, 5), 3)
        new_ms, cached_ms = bench_infer(m1, 10)
        extra["infer_b1_new_frame_ms"] = round(new_ms, 3)
        extra["infer_b1_cached_frame_ms"] = round(cached_ms, 3)
    m1.close()
    del m1
    torch.cuda.empty_cache()
    if not args.quick:
        # int8 weights at batch 1 (config 5's weights at the headline batch),
        # timed next to the bf16 loop: after the sustained GEMM runs below
        # the latency-bound batch-1 loop reads ~10% slower
        m8, enc8 = make_model(1, int8=True)
        extra["loop_int8_b1_ms"] = round(bench_loop(m8, max(10, args.steps // 2), args.warmup), 3)
        extra["encode_int8_b1_ms"] = round(enc8, 3)
        m8.close()
        del m8
        torch.cuda.empty_cache()
    # ---- roofline: the loop's image cross-attention op (config 2, batch 1)
    att_steps = max(10, args.steps // 2)
    img1 = bench_attention(1, 4374, att_steps, args.warmup)
    extra["cross_img_b1_us"] = round(img1["us"], 3)
    if not args.quick:
        img8 = bench_attention(8, 4374, att_steps, args.warmup)
        rng = np.random.default_rng(7)
        lv8 = rng.integers(32, 1025, size=8)
        lang8 = bench_attention(8, 1024, att_steps, args.warmup, valid=lv8)
        lang1 = bench_attention(1, 1024, att_steps, args.warmup, valid=[517])
        self1 = bench_attention(1, 67, att_steps, args.warmup)
        img16 = bench_attention(16, 4374, att_steps, args.warmup)
        img1x = bench_attention(1, 4374, att_steps, args.warmup, exact_pv=True)
        img8x = bench_attention(8, 4374, att_steps, args.warmup, exact_pv=True)
        extra.update({
            "cross_img_b8_us": round(img8["us"], 3),
            "cross_img_b8_GBps": round(img8["GBps"], 1),
            "cross_img_b8_frac": round(img8["frac"], 4),
            "cross_img_b8_traffic": TRAFFIC_B8_IMAGE_BYTES,
            "cross_img_b16_us": round(img16["us"], 3),
            "cross_img_b16_frac": round(img16["frac"], 4),
            "cross_img_b1_exact_pv_us": round(img1x["us"], 3),
            "cross_img_b8_exact_pv_us": round(img8x["us"], 3),
            "cross_img_b8_exact_pv_frac": round(img8x["frac"], 4),
            "cross_lang_b8_us": round(lang8["us"], 3),
            "cross_lang_b8_GBps": round(lang8["GBps"], 1),
            "cross_lang_b1_L517_us": round(lang1["us"], 3),
            "self_b1_us": round(self1["us"], 3),
            "self_b1_TFLOPs": round(self1["TFLOPs"], 2),
            "self_b1_mfma_frac": round(self1["TFLOPs"] / MFMA_BF16_PEAK_TFLOPS, 5),
        })
        for name, M, N, K, int8 in GEMM_SHAPES:
            r = bench_gemm(M, N, K, att_steps, args.warmup, int8=bool(int8), a16=int8 == 2)
            extra[f"gemm_{name}_us"] = round(r["us"], 3)
            extra[f"gemm_{name}_TFLOPs"] = round(r["TFLOPs"], 1)
            extra[f"gemm_{name}_mfma_frac"] = round(r["mfma_frac"], 4)
            if M <= 160:   # weight streaming: the HBM rate is the bound that matters
                extra[f"gemm_{name}_GBps"] = round(r["GBps"], 1)
                extra[f"gemm_{name}_hbm_frac"] = round(r["hbm_frac"], 4)
        for B, int8, key in ((16, 0, "loop_b16_ms"), (32, 1, "loop_int8_b32_ms"),
                             (32, 2, "loop_int8_direct_b32_ms"), (32, 0, "loop_b32_bf16_ms")):
            m, enc = make_model(B, int8=int8)
            extra[key] = round(bench_loop(m, max(3, args.steps // 10), 2), 3)
            extra[key.replace("loop", "encode")] = round(enc, 3)
            if int8 < 2:   # int8_weights = 2: the block products run the direct int8 kernel
                extra[key.replace("loop", "gemm_picks").replace("_ms", "")] = gemm_picks(B, bool(int8))
            m.close()
            del m
            torch.cuda.empty_cache()
        # config 3 as written: the 28-block stack with MLP 4x (2048 -> 8192 -> 2048)
        m4, _ = make_model(1, mlp_ratio=4)
        extra["block_stack_mlp4x_b1_ms"] = round(bench_blocks(m4, 5), 3)
        m4.close()
        del m4
        torch.cuda.empty_cache()
    cpu = None if args.no_cpu else cpu_baseline(lang_len=L1)
    if cpu is not None:
        extra.update(cpu_attention_ops())
    line = {
        "metric": METRIC,
        "value": round(loop1, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(loop1, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "config 4: RDT-1B denoise loop, 5 Euler steps, batch 1, 28 layers, "
                               "hidden 2048, 32 heads, 67 tokens, language condition of "
                               f"L = {L1} token rows (drawn from U{{32..1024}} with a fixed seed; "
                               "padded to 1024, only the L rows encoded and read) / image 4374 "
                               "keys cached once, one hipGraph replay "
                               "per step, random-init weights; the once-per-inference condition "
                               "encode is not in value (extra.encode_condition_b1_ms; a whole "
                               "control step with a new camera frame, encode + loop + host copy: "
                               "extra.infer_b1_new_frame_ms)", "lang_rows": L1},
        "roofline": {
            "bound": "hbm",
            "achieved": round(img1["GBps"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(img1["frac"], 4),
            "traffic": TRAFFIC_B1_IMAGE_BYTES,
            "traffic_source": "rocprofv3 --pmc FETCH_SIZE/WRITE_SIZE on bench.py --profile-roofline, "
                              "profiles/cross_attention_image_roofline.md",
            "kernel": "cross-attention op (attn_ring_kernel, fp16 P.V form, + attn_merge_kernel), 1x32x67x4374x64, "
                      "bf16 Q/K and the fp16 V the runtime caches for that form, "
                      f"{img1['bytes']} algorithmic bytes per launch, {img1['us']:.2f} us",
        },
        "cpu_baseline": cpu,
        "extra": extra,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
