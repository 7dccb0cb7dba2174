"""Writes tests/golden/rdt_small.npz: reference outputs of the RDT-1B model
composition at a reduced size, computed by the reference's own PyTorch
definition of the model.

Run from the repository root, in the build container only (the reference
tree does not exist on the GPU box, and nothing there runs this script):

    python tests/golden/make_rdt_golden.py

It imports `RDT1BRef`, `load_weights` and `sincos_emb` from the reference's
tests/alignment/test_rdt1b_alignment.py (lines 73-257: RmsNorm, sincos_emb,
TimestepEmbedder, Mlp2x, Mlp3x, FFN, SelfAttn, CrossAttn, RDTBlock,
FinalLayer, RDT, RDT1BRef, load_weights) and runs them in float32 on the CPU
with the seeded parameters and inputs of rdt_small.py, loaded through the
reference's own `load_weights` key mapping.  Forward hooks record the
reference's intermediate values; only data is written.

Recorded per batch element b (language truncated to LANG_LEN[b] tokens, the
reference's mechanism for a shorter condition) and per t in T_VALUES:
  lang_c, img_c      adaptor outputs (Mlp2x, rdt1b.cpp:56-85, 185, 199)
  x_seq              state_adaptor(cat([state, noisy], 1), ones): the
                     Python model's state token (row 0) and action tokens
  state_tok_zeros    state_adaptor(cat(state, zeros)): the C++ state token
                     (rdt1b.cpp:202-229) through the reference's Mlp3x
  t_emb, freq_emb    TimestepEmbedder outputs
  cond_i, xin_i, xout_i   each block's condition input (after the position
                     embedding add), residual input and output
  out                final_layer(x)[:, -T:]
and a 3-step Euler loop x <- x + (t_{i+1} - t_i) v(x, t_i) over
t_i = 1 - i/3 (flow_matching.cpp:10-17, 77-78; t_int = round(t * 999) as
rdt1b.cpp:312-313) whose velocity is the reference model's forward, plus
rows of sincos_emb for dims 32 and 256.

The Python model gives the state token an all-ones action mask
(test_rdt1b_alignment.py:204-208); the C++ encode_condition gives it zeros
(rdt1b.cpp:202-229).  Both tokens are recorded; the oracle's denoise step
takes the state token as an input, so the fixture's forward passes pin the
composition independently of that choice.
"""
import importlib.util
import math
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import rdt_small as RS  # noqa: E402

REF_FILE = "/root/reference/tests/alignment/test_rdt1b_alignment.py"


def load_reference():
    spec = importlib.util.spec_from_file_location("rdt1b_alignment_ref", REF_FILE)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def t_index(t):
    """std::round(float(t) * 999) clamped (rdt1b.cpp:312-313)."""
    x = float(np.float32(t) * np.float32(RS.CFG.num_train_timesteps - 1))
    v = math.floor(abs(x) + 0.5) * (1 if x >= 0 else -1)
    return max(0, min(int(v), RS.CFG.num_train_timesteps - 1))


def main():
    R = load_reference()
    torch.manual_seed(0)
    params = RS.make_params()
    inp = RS.make_inputs()
    model = R.RDT1BRef(RS.REF_CFG).float().eval()
    R.load_weights(model, {k: torch.from_numpy(v) for k, v in params.items()}, torch.float32)

    rec = {}
    hooks = []

    def keep(name):
        def fn(_m, _a, out):
            rec[name] = out.detach().clone()
        return fn

    def keep_in(name):
        def fn(_m, args):
            rec["xin_" + name] = args[0].detach().clone()
            rec["cond_" + name] = args[1].detach().clone()
        return fn

    hooks.append(model.lang_adaptor.register_forward_hook(keep("lang_c")))
    hooks.append(model.img_adaptor.register_forward_hook(keep("img_c")))
    hooks.append(model.state_adaptor.register_forward_hook(keep("x_seq")))
    hooks.append(model.model.t_embedder.register_forward_hook(keep("t_emb")))
    hooks.append(model.model.freq_embedder.register_forward_hook(keep("freq_emb")))
    for i, blk in enumerate(model.model.blocks):
        hooks.append(blk.register_forward_pre_hook(keep_in(str(i))))
        hooks.append(blk.register_forward_hook(keep("xout_" + str(i))))

    out = {}
    T = RS.CFG.horizon
    with torch.no_grad():
        for b, L in enumerate(RS.LANG_LEN):
            lang = torch.from_numpy(inp["lang_tok"][b:b + 1, :L].copy())
            img = torch.from_numpy(inp["img_tok"][b:b + 1].copy())
            state = torch.from_numpy(inp["state"][b:b + 1, None, :].copy())
            noisy = torch.from_numpy(inp["noisy"][b:b + 1].copy())
            freq = torch.tensor([RS.CFG.ctrl_freq])
            for ti, t in enumerate(RS.T_VALUES):
                rec.clear()
                y = model(lang, img, state, noisy, torch.tensor([t_index(t)]), freq)
                tag = f"b{b}_t{ti}"
                out[f"{tag}/out"] = y[0].numpy()
                for k, v in rec.items():
                    # condition and adaptor values do not depend on t
                    if ti == 0 or not (k.startswith("cond_") or k in ("lang_c", "img_c", "x_seq", "freq_emb")):
                        out[f"{tag}/{k}"] = v[0].numpy()
            # the C++ state token: state_adaptor(cat(state, zeros))
            st_in = torch.cat([state[:, 0], torch.zeros_like(state[:, 0])], dim=-1)
            out[f"b{b}/state_tok_zeros"] = model.state_adaptor(st_in)[0].numpy()
            # 3-step Euler loop with the reference forward as the velocity
            N = RS.CFG.num_steps
            ts = [np.float32(1.0) + np.float32(i) / np.float32(N) * np.float32(-1.0) for i in range(N + 1)]
            x = noisy.clone()
            for s in range(N):
                v = model(lang, img, state, x, torch.tensor([t_index(ts[s])]), freq)
                x = x + torch.tensor(float(np.float32(ts[s + 1] - ts[s]))) * v
            out[f"b{b}/sample"] = x[0].numpy()
            out[f"b{b}/sample_x0"] = noisy[0].numpy()
        for h in hooks:
            h.remove()
        steps = torch.tensor([0, 1, 25, 199, 500, 999])
        out["sincos_steps"] = steps.numpy().astype(np.int32)
        out["sincos_32"] = R.sincos_emb(steps, 32).numpy()
        out["sincos_256"] = R.sincos_emb(steps, 256).numpy()
    out["t_values"] = np.array(RS.T_VALUES, np.float32)
    out["t_index"] = np.array([t_index(t) for t in RS.T_VALUES], np.int32)
    dst = os.path.join(HERE, "rdt_small.npz")
    np.savez_compressed(dst, **{k: np.ascontiguousarray(v, np.float32 if v.dtype != np.int32 else np.int32)
                                for k, v in out.items()})
    print(f"wrote {dst}: {len(out)} arrays, {os.path.getsize(dst)} bytes")


if __name__ == "__main__":
    main()
