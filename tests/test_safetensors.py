"""The native safetensors reader (include/popcorn_safetensors.h) and the weight
loader mirror (Gemma4WeightLoader.swift:14-120), on the CPU: archives written
by the `safetensors` package (an independent implementation of the format)
read back byte for byte, metadata, edge shapes, and malformed headers
refused with a message."""
import json
import struct

import numpy as np
import pytest

import popcorn_amd as pa
from popcorn_amd.safetensors import SafeTensors, WeightLoader

st_numpy = pytest.importorskip("safetensors.numpy")


def _write(path, tensors, metadata=None):
    st_numpy.save_file(tensors, str(path), metadata=metadata)
    return str(path)


def test_roundtrip_dtypes_and_metadata(tmp_path):
    rng = np.random.default_rng(0)
    tensors = {
        "a.f32": rng.standard_normal((3, 5)).astype(np.float32),
        "b.f16": rng.standard_normal((7,)).astype(np.float16),
        "c.u32": rng.integers(0, 2 ** 32, (4, 9), dtype=np.uint64).astype(np.uint32),
        "d.i64": rng.integers(-5, 5, (2, 2, 2)).astype(np.int64),
        "e.u8": rng.integers(0, 255, (11,)).astype(np.uint8),
        "f.i32": np.array(7, np.int32),          # rank 0
        "g.empty": np.zeros((0, 4), np.float32),  # no bytes
        "h.i16": rng.integers(-100, 100, (5,)).astype(np.int16),
        "i.f64": rng.standard_normal((2,)),
    }
    path = _write(tmp_path / "m.safetensors", tensors, {"format": "pt", "note": "ünïcode \"q\""})
    st = SafeTensors(path)
    assert sorted(st.names) == sorted(tensors)
    for name, arr in tensors.items():
        dt, shape = st.info(name)
        assert shape == list(arr.shape), name
        if arr.dtype == np.float64:
            assert dt == "F64" and st.dtype(name) is None
            with pytest.raises(pa.PopcornError) as e:
                st.read(name)
            assert e.value.code == pa.PopcornError.UNSUPPORTED_DATA_TYPE_COMBINATION
            continue
        got = st.read(name)
        assert got.dtype == arr.dtype and got.tobytes() == arr.tobytes(), name
    assert st.metadata("format") == "pt"
    assert st.metadata("note") == "ünïcode \"q\""
    with pytest.raises(pa.PopcornError):
        st.metadata("absent")
    with pytest.raises(pa.PopcornError) as e:
        st.read("nope")
    assert "no tensor named" in str(e.value)
    st.close()


def test_bf16_bits_survive(tmp_path):
    bits = np.array([0x3F80, 0xC000, 0x7F80, 0x0001, 0x8000], np.uint16)
    # the safetensors package writes BF16 from uint16 views via its dtype map
    header = {"w": {"dtype": "BF16", "shape": [5], "data_offsets": [0, 10]}}
    path = tmp_path / "bf.safetensors"
    _raw(path, header, bits.tobytes())
    st = SafeTensors(str(path))
    assert st.dtype("w") == "bf16"
    assert st.read("w").tolist() == bits.tolist()


def _raw(path, header, data, pad=0):
    h = json.dumps(header).encode() + b" " * pad
    path.write_bytes(struct.pack("<Q", len(h)) + h + data)


@pytest.mark.parametrize("case,header,data,msg", [
    ("short", None, b"\x01\x02", "shorter than"),
    ("len", {"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}, b"", "runs past the end"),
    ("json", "{not json", b"", "header JSON"),
    ("notobj", [1, 2], b"", "not a JSON object"),
    ("dtype", {"a": {"dtype": "Q7", "shape": [1], "data_offsets": [0, 1]}}, b"\x00", "unknown dtype"),
    ("count", {"a": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\x00" * 4, "bytes, not elements"),
    ("oob", {"a": {"dtype": "U8", "shape": [4], "data_offsets": [0, 4]}}, b"\x00" * 2, "outside the data buffer"),
    ("overlap", {"a": {"dtype": "U8", "shape": [2], "data_offsets": [0, 2]},
                 "b": {"dtype": "U8", "shape": [2], "data_offsets": [1, 3]}}, b"\x00" * 3, "hole or overlap"),
    ("hole", {"a": {"dtype": "U8", "shape": [1], "data_offsets": [1, 2]}}, b"\x00" * 2, "hole or overlap"),
    ("tail", {"a": {"dtype": "U8", "shape": [1], "data_offsets": [0, 1]}}, b"\x00" * 3, "no tensor covers"),
    ("shape", {"a": {"dtype": "U8", "shape": [-1], "data_offsets": [0, 1]}}, b"\x00", "non-negative integer"),
    ("meta", {"__metadata__": {"k": 1}}, b"", "must be strings"),
    ("fields", {"a": {"dtype": "U8", "shape": [1]}}, b"\x00", "needs dtype, shape and data_offsets"),
])
def test_malformed_archives_are_refused(tmp_path, case, header, data, msg):
    path = tmp_path / f"{case}.safetensors"
    if case == "short":
        path.write_bytes(data)
    elif case == "len":
        h = json.dumps(header).encode()
        path.write_bytes(struct.pack("<Q", len(h) + 100) + h)
    elif isinstance(header, str):
        h = header.encode()
        path.write_bytes(struct.pack("<Q", len(h)) + h + data)
    else:
        _raw(path, header, data)
    with pytest.raises(pa.PopcornError) as e:
        SafeTensors(str(path))
    assert e.value.code == pa.PopcornError.INVALID_ARGUMENT
    assert msg in e.value.message, e.value.message


def test_padded_header_and_missing_file(tmp_path):
    path = tmp_path / "pad.safetensors"
    _raw(path, {"a": {"dtype": "U8", "shape": [3], "data_offsets": [0, 3]}}, b"abc", pad=5)
    assert SafeTensors(str(path)).read("a").tobytes() == b"abc"
    with pytest.raises(pa.PopcornError):
        SafeTensors(str(tmp_path / "absent.safetensors"))


def test_weight_loader_prefix_and_quantized_detection(tmp_path):
    # Gemma4WeightLoader.swift:21-29 (prefix), :80-119 (quantized triplet)
    rng = np.random.default_rng(1)
    packed = rng.integers(0, 2 ** 32, (16, 8), dtype=np.uint64).astype(np.uint32)
    tensors = {
        "model.language_model.layers.0.mlp.gate_proj.weight": packed,
        "model.language_model.layers.0.mlp.gate_proj.scales": np.ones((16, 1), np.float16),
        "model.language_model.layers.0.mlp.gate_proj.biases": np.zeros((16, 1), np.float16),
        "model.language_model.layers.0.self_attn.o_proj.weight": np.ones((4, 64), np.float32),
    }
    path = _write(tmp_path / "w.safetensors", tensors)
    st = SafeTensors(path)
    wl = WeightLoader(st, None)
    assert wl.language_model_prefix == "model.language_model"
    assert wl.layer_prefix(3) == "model.language_model.layers.3"
    # without a quantization config nothing is read as quantized
    assert wl._maybe_quantized(wl.layer_prefix(0) + ".mlp.gate_proj", None) is None
    with pytest.raises(pa.PopcornError):
        WeightLoader(SafeTensors(_write(tmp_path / "x.safetensors", {"other.weight": np.ones(2, np.float32)})))
