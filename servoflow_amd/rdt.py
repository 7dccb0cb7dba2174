"""ctypes front end for libsf_rdt.so (include/sf_rdt.h): the RDT-1B
denoise-loop runtime.  Plumbing for tests and the benchmark: torch supplies
device buffers and the stream; the model runs in the native library."""
from __future__ import annotations

import ctypes
import os

import numpy as np
import torch

from . import abi

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "lib", "libsf_rdt.so")


class RdtConfig(ctypes.Structure):
    """Mirror of `sf_rdt_config`."""

    _fields_ = [(n, ctypes.c_int32) for n in (
        "hidden", "layers", "heads", "action_dim", "horizon", "freq_dim", "state_dim",
        "lang_max", "img_len", "lang_token_dim", "img_token_dim", "num_train_timesteps",
        "ctrl_freq", "num_steps", "batch", "int8_weights")] + [("eps", ctypes.c_float),
                                                             ("mlp_ratio", ctypes.c_int32)]


class StEntry(ctypes.Structure):
    """Mirror of `sf_st_entry`."""

    _fields_ = [("name", ctypes.c_char * 256), ("dtype", ctypes.c_int32), ("ndim", ctypes.c_int32),
                ("shape", ctypes.c_int64 * 8), ("data_begin", ctypes.c_uint64), ("data_end", ctypes.c_uint64)]


SF_LOAD_PARTIAL = 1
_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    abi.lib()   # kernels first (libsf_rdt.so links against it)
    if not os.path.exists(LIB_PATH):
        raise FileNotFoundError(f"{LIB_PATH} is missing: build with __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    vp, i32, P = ctypes.c_void_p, ctypes.c_int32, ctypes.POINTER(RdtConfig)
    L.sf_rdt_config_default.argtypes = [P]
    L.sf_rdt_config_default.restype = None
    L.sf_rdt_create.argtypes = [P, ctypes.POINTER(vp)]
    L.sf_rdt_destroy.argtypes = [vp]
    L.sf_rdt_destroy.restype = None
    L.sf_rdt_init_random.argtypes = [vp, ctypes.c_uint64, ctypes.c_float, vp]
    L.sf_rdt_num_params.argtypes = [vp]
    L.sf_rdt_num_params.restype = i32
    L.sf_rdt_param_info.argtypes = [vp, i32, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(i32),
                                    ctypes.POINTER(i32), ctypes.c_int64 * 4]
    L.sf_rdt_param_data.argtypes = [vp, i32]
    L.sf_rdt_param_data.restype = vp
    L.sf_rdt_params_changed.argtypes = [vp]
    L.sf_rdt_param_scale.argtypes = [vp, i32]
    L.sf_rdt_param_scale.restype = vp
    L.sf_rdt_find_param.argtypes = [vp, ctypes.c_char_p]
    L.sf_rdt_find_param.restype = i32
    L.sf_rdt_cache_ptr.argtypes = [vp, i32, i32]
    L.sf_rdt_cache_ptr.restype = vp
    L.sf_rdt_pv_exact.argtypes = [vp, i32]
    L.sf_rdt_pv_exact.restype = i32
    L.sf_rdt_set_condition.argtypes = [vp, vp, vp, vp, vp, vp]
    L.sf_rdt_set_lang_rows.argtypes = [vp, i32]
    L.sf_rdt_encode_condition.argtypes = [vp, vp, vp, vp, vp, vp]
    L.sf_rdt_denoise_step.argtypes = [vp, vp, ctypes.c_float, vp, vp]
    L.sf_rdt_sample.argtypes = [vp, vp, i32, vp]
    L.sf_rdt_run_blocks.argtypes = [vp, vp, i32, i32, vp]
    L.sf_rdt_infer.argtypes = [vp, ctypes.c_uint64, vp, vp, vp, vp, ctypes.c_uint64, vp,
                               ctypes.POINTER(i32), vp]
    L.sf_safetensors_inspect.argtypes = [ctypes.c_char_p, ctypes.POINTER(StEntry), i32, ctypes.POINTER(i32)]
    L.sf_rdt_load_safetensors.argtypes = [vp, ctypes.c_char_p, i32, ctypes.POINTER(i32)]
    L.sf_rdt_last_error.argtypes = [vp]
    L.sf_rdt_last_error.restype = ctypes.c_char_p
    _lib = L
    return L


def default_config(**over) -> RdtConfig:
    c = RdtConfig()
    lib().sf_rdt_config_default(ctypes.byref(c))
    for k, v in over.items():
        setattr(c, k, v)
    return c


def inspect_safetensors(path):
    """[(name, sf_dtype, shape, data_begin, data_end)] of a safetensors file."""
    n = ctypes.c_int32()
    abi.check(lib().sf_safetensors_inspect(os.fsencode(path), None, 0, ctypes.byref(n)),
              "sf_safetensors_inspect")
    arr = (StEntry * max(n.value, 1))()
    abi.check(lib().sf_safetensors_inspect(os.fsencode(path), arr, n.value, ctypes.byref(n)),
              "sf_safetensors_inspect")
    return [(e.name.decode("utf-8"), e.dtype, tuple(e.shape[:e.ndim]), e.data_begin, e.data_end)
            for e in arr[:n.value]]


_hip = None


def _hipmemcpy(dst, src, nbytes, kind):
    global _hip
    if _hip is None:
        _hip = ctypes.CDLL("libamdhip64.so")
        _hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    torch.cuda.synchronize()
    st = _hip.hipMemcpy(dst, src, nbytes, kind)
    if st != 0:
        raise RuntimeError(f"hipMemcpy failed ({st})")


def _memcpy_d2h(dst_np, src_ptr):
    _hipmemcpy(dst_np.ctypes.data, src_ptr, dst_np.nbytes, 2)   # DeviceToHost
    return dst_np


class RdtModel:
    """Owns one sf_rdt instance on the current device."""

    def __init__(self, cfg: RdtConfig):
        self.cfg = cfg
        h = ctypes.c_void_p()
        abi.check(lib().sf_rdt_create(ctypes.byref(cfg), ctypes.byref(h)), "sf_rdt_create")
        self.h = h

    def close(self):
        if self.h:
            lib().sf_rdt_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    @staticmethod
    def _stream():
        return torch.cuda.current_stream().cuda_stream

    def init_random(self, seed=1234, std=0.02):
        abi.check(lib().sf_rdt_init_random(self.h, seed, std, self._stream()), "sf_rdt_init_random")

    def params(self):
        out = []
        for i in range(lib().sf_rdt_num_params(self.h)):
            name, dt, nd = ctypes.c_char_p(), ctypes.c_int32(), ctypes.c_int32()
            shape = (ctypes.c_int64 * 4)()
            abi.check(lib().sf_rdt_param_info(self.h, i, ctypes.byref(name), ctypes.byref(dt),
                                              ctypes.byref(nd), shape), "sf_rdt_param_info")
            out.append((name.value.decode(), dt.value, tuple(shape[:nd.value])))
        return out

    def param_numpy(self, idx, dtype, shape):
        """Parameter as fp32 numpy (int8 weights returned dequantised)."""
        n = int(np.prod(shape))
        ptr = lib().sf_rdt_param_data(self.h, idx)
        if dtype == abi.SF_F32:
            return _memcpy_d2h(np.empty(shape, np.float32), ptr)
        if dtype == abi.SF_BF16:
            raw = _memcpy_d2h(np.empty(n, np.uint16), ptr)
            return (raw.astype(np.uint32) << 16).view(np.float32).reshape(shape)
        q = _memcpy_d2h(np.empty(shape, np.int8), ptr)
        s = _memcpy_d2h(np.empty(shape[0], np.float32), lib().sf_rdt_param_scale(self.h, idx))
        return q.astype(np.float32) * s[:, None]

    def param_int8(self, idx):
        """(codes int8 [N, K], row scales fp32 [N]) of an int8 parameter."""
        _, dt, shape = self.params()[idx]
        assert dt == abi.SF_I8
        q = _memcpy_d2h(np.empty(shape, np.int8), lib().sf_rdt_param_data(self.h, idx))
        s = _memcpy_d2h(np.empty(shape[0], np.float32), lib().sf_rdt_param_scale(self.h, idx))
        return q, s

    def load_safetensors(self, path, partial=False):
        """Loads a checkpoint (sf_rdt_load_safetensors); returns the number of
        parameters written."""
        n = ctypes.c_int32()
        st = lib().sf_rdt_load_safetensors(self.h, os.fsencode(path), SF_LOAD_PARTIAL if partial else 0,
                                           ctypes.byref(n))
        if st != abi.SF_OK:
            raise abi.SfError(st, "sf_rdt_load_safetensors: " + lib().sf_rdt_last_error(self.h).decode())
        return n.value

    def param_write(self, idx, values, offset=0):
        """Writes `values` (numpy, the parameter's element type) into parameter
        idx starting at element `offset` (host -> device copy)."""
        _, dt, shape = self.params()[idx]
        esize = {abi.SF_F32: 4, abi.SF_BF16: 2, abi.SF_I8: 1}[dt]
        v = np.ascontiguousarray(values)
        assert v.itemsize == esize and offset + v.size <= int(np.prod(shape))
        _hipmemcpy(lib().sf_rdt_param_data(self.h, idx) + offset * esize, v.ctypes.data, v.nbytes, 1)

    def params_changed(self):
        """sf_rdt_params_changed: parameters were written through pointers
        obtained earlier; the weight copies are rebuilt before the next pass."""
        abi.check(lib().sf_rdt_params_changed(self.h), "sf_rdt_params_changed")

    def set_lang_rows(self, rows):
        """The language condition's token count L (sf_rdt_set_lang_rows): the
        cross-attention reads at most L keys, and at batch 1 the language
        adaptor and K/V projections run over L rows, from the next condition
        set."""
        abi.check(lib().sf_rdt_set_lang_rows(self.h, int(rows)), "sf_rdt_set_lang_rows")

    def pv_exact(self, layer):
        """sf_rdt_pv_exact: 1 when block `layer`'s cross-attention runs the
        exact bf16 P.V form for the current condition, 0 for the fp16 form."""
        r = lib().sf_rdt_pv_exact(self.h, layer)
        if r < 0:
            raise abi.SfError(abi.SF_EINVAL, "sf_rdt_pv_exact")
        return r

    def state_dict(self):
        return {nm: self.param_numpy(i, dt, sh) for i, (nm, dt, sh) in enumerate(self.params())}

    def cache_numpy(self, layer, which_v):
        """Block `layer`'s K (which_v 0) or V cache as fp32 [B, H, S, 64]: K
        is bf16; V is fp16 for a layer on the fp16 P.V form, else bf16."""
        c = self.cfg
        sc = c.lang_max if layer % 2 == 0 else c.img_len
        f16 = which_v and self.pv_exact(layer) == 0
        raw = _memcpy_d2h(np.empty(c.batch * c.heads * sc * 64, np.uint16),
                          lib().sf_rdt_cache_ptr(self.h, layer, which_v))
        if f16:
            return raw.view(np.float16).astype(np.float32).reshape(c.batch, c.heads, sc, 64)
        return (raw.astype(np.uint32) << 16).view(np.float32).reshape(c.batch, c.heads, sc, 64)

    def set_condition(self, lang_c, lang_len, img_c, state_tok):
        abi.check(lib().sf_rdt_set_condition(self.h, lang_c.data_ptr(), lang_len.data_ptr(),
                                             img_c.data_ptr(), state_tok.data_ptr(), self._stream()),
                  "sf_rdt_set_condition")

    def encode_condition(self, lang_tokens, lang_len, img_tokens, state):
        abi.check(lib().sf_rdt_encode_condition(self.h, lang_tokens.data_ptr(), lang_len.data_ptr(),
                                                img_tokens.data_ptr(), state.data_ptr(),
                                                self._stream()), "sf_rdt_encode_condition")

    def run_blocks(self, x, first=0, count=None):
        count = self.cfg.layers - first if count is None else count
        abi.check(lib().sf_rdt_run_blocks(self.h, x.data_ptr(), first, count, self._stream()),
                  "sf_rdt_run_blocks")
        return x

    def denoise_step(self, x_t, t, out=None):
        if out is None:
            out = torch.empty_like(x_t)
        abi.check(lib().sf_rdt_denoise_step(self.h, x_t.data_ptr(), float(t), out.data_ptr(),
                                            self._stream()), "sf_rdt_denoise_step")
        return out

    def infer(self, frame_id, lang_tokens, lang_len, img_tokens, state, noise_seed=0):
        """sf_rdt_infer: returns (action chunk [B, T, A] as a host fp32 numpy
        array, whether this call encoded the condition)."""
        import numpy as np

        c = self.cfg
        out = np.empty((c.batch, c.horizon, c.action_dim), np.float32)
        enc = ctypes.c_int32(-1)
        abi.check(lib().sf_rdt_infer(self.h, int(frame_id), lang_tokens.data_ptr(), lang_len.data_ptr(),
                                     img_tokens.data_ptr(), state.data_ptr(), int(noise_seed),
                                     out.ctypes.data, ctypes.byref(enc), self._stream()), "sf_rdt_infer")
        return out, bool(enc.value)

    def sample(self, x, use_graph=True):
        abi.check(lib().sf_rdt_sample(self.h, x.data_ptr(), 1 if use_graph else 0, self._stream()),
                  "sf_rdt_sample")
        return x
