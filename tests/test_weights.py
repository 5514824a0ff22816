"""The weight path without a GPU: mt_st_* against files the safetensors library writes
(dtype, shape, bytes, header order) and the refusals of SafeTensors.swift:19-44 (short
file, header past the end, header not an object, malformed entry, data past the end,
missing tensor); WeightArena planning (Weights.swift:24-79): 256-byte placement in call
order, concatenation along the first axis, padded weights, dtype checks."""
import json
import os
import struct

import numpy as np
import pytest
import torch
from safetensors.torch import save_file

import mingtts as mt


def _write(path, tensors, metadata=None):
    save_file(tensors, str(path), metadata=metadata)
    return str(path)


def _raw(t: torch.Tensor) -> bytes:
    return t.contiguous().view(torch.uint8).numpy().tobytes()


def test_entries_match_the_writer(tmp_path):
    g = torch.Generator().manual_seed(0)
    ts = {"a.weight": torch.randn(5, 8, generator=g).bfloat16(), "b": torch.randn(3, generator=g).half(),
          "c.scale": torch.randn(2, 3, 4, generator=g), "d.idx": torch.arange(6, dtype=torch.int64)}
    p = _write(tmp_path / "m.safetensors", ts, {"format": "pt"})
    st = mt.SafeTensors(p)
    assert set(st.entries) == set(ts)
    codes = {torch.bfloat16: mt.BF16, torch.float16: mt.F16, torch.float32: mt.F32, torch.int64: -1}
    for name, t in ts.items():
        dt, shape, nbytes = st.entries[name]
        assert dt == codes[t.dtype] and shape == tuple(t.shape) and nbytes == t.numel() * t.element_size()
        assert st.raw(name) == _raw(t)
    st.close()


def _header_file(path, header: bytes, data: bytes = b"", length=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header) if length is None else length) + header + data)
    return str(path)


@pytest.mark.parametrize("case,needle", [
    ("short", "file too small"),
    ("length", "exceeds file"),
    ("array", "not a JSON object"),
    ("garbage", "not a JSON object"),
    ("no_offsets", "malformed entry x"),
    ("bad_shape", "malformed entry x"),
    ("reversed", "malformed entry x"),
    ("truncated", "download incomplete?"),
])
def test_refusals(tmp_path, case, needle):
    p = tmp_path / f"{case}.safetensors"
    good = {"x": {"dtype": "BF16", "shape": [2, 2], "data_offsets": [0, 8]}}
    if case == "short":
        p.write_bytes(b"\x01\x02")
    elif case == "length":
        _header_file(p, json.dumps(good).encode(), b"\0" * 8, length=10 ** 6)
    elif case == "array":
        _header_file(p, b"[1, 2]", b"")
    elif case == "garbage":
        _header_file(p, b"{\"x\": {\"dtype\": }", b"")
    elif case == "no_offsets":
        _header_file(p, json.dumps({"x": {"dtype": "BF16", "shape": [2]}}).encode())
    elif case == "bad_shape":
        _header_file(p, json.dumps({"x": {"dtype": "BF16", "shape": [2.5], "data_offsets": [0, 4]}}).encode(), b"\0" * 4)
    elif case == "reversed":
        _header_file(p, json.dumps({"x": {"dtype": "BF16", "shape": [2], "data_offsets": [4, 0]}}).encode(), b"\0" * 4)
    elif case == "truncated":
        _header_file(p, json.dumps(good).encode(), b"\0" * 6)   # 8 bytes needed
    with pytest.raises(mt.MingTTSError) as e:
        mt.SafeTensors(str(p))
    assert e.value.code == mt.EINVAL and needle in str(e.value), str(e.value)


def test_header_escapes_and_metadata(tmp_path):
    """A name with JSON escapes and a __metadata__ object are read as the format defines."""
    hdr = json.dumps({"__metadata__": {"k": "v\\n"}, "q\"uoteé": {"dtype": "F16", "shape": [2],
                                                                       "data_offsets": [0, 4]}})
    p = _header_file(tmp_path / "esc.safetensors", hdr.encode(), b"\x00\x3c\x00\xc0")
    st = mt.SafeTensors(p)
    assert list(st.entries) == ["q\"uoteé"]
    assert np.frombuffer(st.raw("q\"uoteé"), np.float16).tolist() == [1.0, -2.0]
    with pytest.raises(mt.MingTTSError) as e:
        st.entry("nope")
    assert "missing tensor nope" in str(e.value)


def test_arena_plan(tmp_path):
    g = torch.Generator().manual_seed(1)
    ts = {"l.q.weight": torch.randn(8, 16, generator=g).bfloat16(), "l.k.weight": torch.randn(2, 16, generator=g).bfloat16(),
          "l.v.weight": torch.randn(2, 16, generator=g).bfloat16(), "l.o.weight": torch.randn(16, 8, generator=g).bfloat16(),
          "l.o.bias": torch.randn(16, generator=g).bfloat16(), "e.weight": torch.randn(4, 10, generator=g).bfloat16(),
          "f32": torch.randn(4, generator=g)}
    st = mt.SafeTensors(_write(tmp_path / "a.safetensors", ts))
    arena = mt.WeightArena(st)
    qkv = arena.tensor("l.q.weight", "l.k.weight", "l.v.weight")
    o = arena.linear("l.o", 16, 8, bias=True)
    pad = arena.padded_linear("e", 4, 16, 10)
    assert (qkv.offset, qkv.count) == (0, 12 * 16)
    assert (o.w.offset, o.w.count) == (512, 128)        # 384 bytes -> next 256 boundary
    assert (o.bias.offset, o.bias.count) == (768, 16)
    assert pad.w.offset == 1024 and arena.nbytes == 1024 + 256
    with pytest.raises(mt.MingTTSError) as e:
        arena.tensor("f32")
    assert "expected BF16" in str(e.value)
    with pytest.raises(mt.MingTTSError) as e:
        arena.padded_linear("e", 4, 8, 12)
    assert "is not BF16 [4, 12]" in str(e.value)
    with pytest.raises(mt.MingTTSError) as e:
        arena.linear("l.o", 16, 16, bias=False)
    assert "expected 16x16" in str(e.value)
    arena.close()
    st.close()


def test_arena_refuses_a_shape_larger_than_its_byte_range(tmp_path):
    """A header whose shape claims more bytes than its data_offsets span is refused by the
    arena (the copies would read past the tensor, and past the mapping for the last one)."""
    hdr = {"e.weight": {"dtype": "BF16", "shape": [4, 8], "data_offsets": [0, 32]},   # needs 64
           "ok.weight": {"dtype": "BF16", "shape": [2, 4], "data_offsets": [32, 48]}}
    p = _header_file(tmp_path / "lie.safetensors", json.dumps(hdr).encode(), b"\0" * 48)
    st = mt.SafeTensors(p)
    arena = mt.WeightArena(st)
    with pytest.raises(mt.MingTTSError) as e:
        arena.padded_linear("e", 4, 16, 8)
    assert e.value.code == mt.EINVAL and "data_offsets span 32 bytes" in str(e.value)
    with pytest.raises(mt.MingTTSError) as e:
        arena.tensor("e.weight")
    assert "data_offsets span 32 bytes" in str(e.value)
    assert arena.tensor("ok.weight").count == 8      # a consistent entry still plans
    arena.close()
    st.close()
