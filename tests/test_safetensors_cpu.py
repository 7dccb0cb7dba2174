"""The safetensors header reader of libsf_rdt.so (sf_safetensors_inspect,
restating SafeTensorsLoader::parse_header / inspect,
src/loader/safetensors.cpp:75-114) against files written by the
`safetensors` package -- the format's reference implementation, an
independent producer -- plus malformed files.  Host only (no GPU)."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors import safe_open
from safetensors.torch import save_file

from servoflow_amd import abi
from servoflow_amd import rdt as R

CODES = {torch.float32: abi.SF_F32, torch.float16: abi.SF_F16, torch.bfloat16: abi.SF_BF16,
         torch.int8: abi.SF_I8, torch.int32: abi.SF_I32}


def test_inspect_matches_the_reference_writer(tmp_path):
    tensors = {
        "model.blocks.0.attn.qkv.weight": torch.randn(96, 32).to(torch.bfloat16),
        "lang_adaptor.0.bias": torch.randn(32),
        "x_pos_embed": torch.randn(1, 7, 32).to(torch.float16),
        "ema_model.foo": torch.zeros(3, dtype=torch.int8),
        "weird \"name\" é中": torch.arange(5, dtype=torch.int32),
        "scalar": torch.tensor(1.5),
    }
    path = str(tmp_path / "m.safetensors")
    save_file(tensors, path, metadata={"format": "pt", "note": 'a "quoted" value'})
    got = {e[0]: e for e in R.inspect_safetensors(path)}
    assert set(got) == set(tensors)
    raw = open(path, "rb").read()
    hlen = struct.unpack("<Q", raw[:8])[0]
    with safe_open(path, framework="pt") as f:
        for name, t in tensors.items():
            nm, dt, shape, b, e = got[name]
            assert dt == CODES[t.dtype], name
            assert shape == tuple(t.shape), name
            assert e - b == t.numel() * t.element_size(), name
            # the bytes at [b, e) are the tensor's bytes
            ref = f.get_tensor(name)
            assert raw[b:e] == ref.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes(), name
            assert b >= 8 + hlen


@pytest.mark.parametrize("content", [
    b"",                                                     # empty
    b"\x10\x00\x00\x00\x00\x00\x00\x00{}",                     # header length past the end
    struct.pack("<Q", 5) + b"{\"a\":",                         # truncated JSON
    struct.pack("<Q", 2) + b"[]",                              # not an object
    struct.pack("<Q", 40) + json.dumps({"t": {"dtype": "F32", "shape": [2]}}).encode().ljust(40),
])
def test_malformed_files_are_rejected(tmp_path, content):
    path = tmp_path / "bad.safetensors"
    path.write_bytes(content)
    with pytest.raises(abi.SfError):
        R.inspect_safetensors(str(path))


def test_missing_file_is_an_error(tmp_path):
    with pytest.raises(abi.SfError):
        R.inspect_safetensors(str(tmp_path / "nope.safetensors"))


@pytest.mark.parametrize("depth,ok", [(10, True), (63, True), (200, False), (100000, False)])
def test_metadata_nesting_depth_is_bounded(tmp_path, depth, ok):
    """Nested metadata is skipped recursively; past 64 levels the header is
    rejected instead of recursing without bound."""
    meta = "[" * depth + "]" * depth
    hdr = ('{"__metadata__": ' + meta + ', "t": {"dtype": "F32", "shape": [2], "data_offsets": [0, 8]}}').encode()
    path = tmp_path / "nest.safetensors"
    path.write_bytes(struct.pack("<Q", len(hdr)) + hdr + b"\0" * 8)
    if ok:
        assert [e[0] for e in R.inspect_safetensors(str(path))] == ["t"]
    else:
        with pytest.raises(abi.SfError):
            R.inspect_safetensors(str(path))
