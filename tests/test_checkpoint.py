"""Safetensors reader and MLX-affine adapter: header rules and messages of the
reference reader (src/js/compute/native.zig:1772-1885), layer selection rules
(docs/core/quantized-inference.md:85-112). CPU only; loading onto the device
is covered in test_gpu_parity.py."""
import json
import struct

import numpy as np
import pytest

from affon_amd import checkpoint as C


def write_file(path, entries, *, metadata=None, header=None, data=None, raw_prefix=None):
    """entries: (name, dtype, shape, bytes). Offsets are laid out in order."""
    if header is None:
        header, blob, offset = {}, b"", 0
        for name, dtype, shape, payload in entries:
            header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [offset, offset + len(payload)]}
            blob += payload
            offset += len(payload)
        if metadata is not None:
            header["__metadata__"] = metadata
        data = blob
    text = json.dumps(header).encode() if not isinstance(header, bytes) else header
    with open(path, "wb") as f:
        f.write(raw_prefix if raw_prefix is not None else struct.pack("<Q", len(text)))
        f.write(text)
        f.write(data or b"")
    return path


def test_inspect_lists_every_dtype(tmp_path):
    p = write_file(tmp_path / "a.safetensors", [
        ("w", "U32", [2, 3], np.arange(6, dtype=np.uint32).tobytes()),
        ("s", "BF16", [2, 1], np.zeros(2, np.uint16).tobytes()),
        ("d", "F64", [1], np.zeros(1, np.float64).tobytes()),
        ("i", "I64", [0], b""),
        ("f", "F32", [], np.zeros(1, np.float32).tobytes()),
    ], metadata={"format": "mlx"})
    assert C.inspect(str(p)) == {"w": {"shape": [2, 3], "dtype": "U32"}, "s": {"shape": [2, 1], "dtype": "BF16"},
                                 "d": {"shape": [1], "dtype": "F64"}, "i": {"shape": [0], "dtype": "I64"},
                                 "f": {"shape": [], "dtype": "F32"}}


@pytest.mark.parametrize("header,data,message", [
    ({"w": {"dtype": "F16", "shape": [1], "data_offsets": [0, 2]}}, b"\0\0", "has unsupported dtype"),
    ({"w": {"shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4, "metadata is missing dtype"),
    ({"w": {"dtype": 3, "shape": [1], "data_offsets": [0, 4]}}, b"\0" * 4, "dtype must be a string"),
    ({"w": {"dtype": "F32", "data_offsets": [0, 4]}}, b"\0" * 4, "metadata is missing shape"),
    ({"w": {"dtype": "F32", "shape": 1, "data_offsets": [0, 4]}}, b"\0" * 4, "shape must be an array"),
    ({"w": {"dtype": "F32", "shape": [-1], "data_offsets": [0, 4]}}, b"\0" * 4,
     "shape must contain non-negative integers"),
    ({"w": {"dtype": "F32", "shape": [1]}}, b"\0" * 4, "metadata is missing offsets"),
    ({"w": {"dtype": "F32", "shape": [1], "data_offsets": [0]}}, b"\0" * 4, "expects two offsets"),
    ({"w": {"dtype": "F32", "shape": [1], "data_offsets": [0, -4]}}, b"\0" * 4,
     "offsets must be non-negative integers"),
    ({"w": {"dtype": "F32", "shape": [1], "data_offsets": [0, 8]}}, b"\0" * 4, "offsets exceed file size"),
    ({"w": {"dtype": "F32", "shape": [1], "data_offsets": [4, 0]}}, b"\0" * 4, "offsets exceed file size"),
    ({"w": {"dtype": "F32", "shape": [2], "data_offsets": [0, 4]}}, b"\0" * 4, "tensor byte length mismatch"),
    ({"w": [1, 2]}, b"", "metadata must be an object"),
    ({"__metadata__": {"a": 1}}, b"", "__metadata__ values must be strings"),
    ([1, 2], b"", "header must be an object"),
])
def test_header_rules(tmp_path, header, data, message):
    p = write_file(tmp_path / "bad.safetensors", None, header=header, data=data)
    with pytest.raises(C.CheckpointError, match=message):
        C.inspect(str(p))


def test_file_level_rules(tmp_path):
    with pytest.raises(C.CheckpointError, match="failed to open file"):
        C.inspect(str(tmp_path / "missing.safetensors"))
    small = tmp_path / "small"
    small.write_bytes(b"\1\2\3")
    with pytest.raises(C.CheckpointError, match="file is too small"):
        C.inspect(str(small))
    p = write_file(tmp_path / "big.safetensors", None, header=b"{}", raw_prefix=struct.pack("<Q", 1 << 30))
    with pytest.raises(C.CheckpointError, match="has an invalid header"):
        C.inspect(str(p))
    p = write_file(tmp_path / "json.safetensors", None, header=b"{not json")
    with pytest.raises(C.CheckpointError, match="has invalid metadata"):
        C.inspect(str(p))


def test_name_selection_rules(tmp_path):
    p = str(write_file(tmp_path / "a.safetensors", [("w", "F32", [1], b"\0" * 4)]))
    with pytest.raises(TypeError, match="names must be an array"):
        C.load(None, p, "w")
    with pytest.raises(TypeError, match="names must be strings"):
        C.load(None, p, [1])
    with pytest.raises(C.CheckpointError, match="Duplicate checkpoint name"):
        C.load(None, p, ["w", "w"])
    with pytest.raises(C.CheckpointError, match="Missing requested checkpoint tensor"):
        C.load(None, p, ["w", "x"])


def mlx_header(layers, bits, group, pdtype="BF16"):
    header = {}
    for prefix, out, inp in layers:
        header[prefix + ".weight"] = {"dtype": "U32", "shape": [out, inp * bits // 32]}
        header[prefix + ".scales"] = {"dtype": pdtype, "shape": [out, inp // group]}
        header[prefix + ".biases"] = {"dtype": pdtype, "shape": [out, inp // group]}
    return header


def test_layer_selection():
    header = mlx_header([("model.q_proj", 64, 256), ("model.k_proj", 32, 256)], 4, 64)
    header["model.embed.weight"] = {"dtype": "U32", "shape": [10, 8]}       # U32 without parameters: not a layer
    header["model.norm.weight"] = {"dtype": "BF16", "shape": [256]}
    specs = C.quantized_layer_specs(header, 4, 64)
    assert [(s.prefix, s.out_features, s.in_features, s.param_dtype) for s in specs] == [
        ("model.q_proj", 64, 256, "BF16"), ("model.k_proj", 32, 256, "BF16")]
    with pytest.raises(C.CheckpointError, match="needs .weight, .scales and .biases"):
        C.quantized_layer_specs(header, 4, 64, ["model.embed"])
    with pytest.raises(C.CheckpointError, match="shapes do not match"):
        C.quantized_layer_specs(header, 8, 64)   # the same words read as 8-bit codes: wrong parameter shape
    bad = mlx_header([("p", 8, 128)], 4, 64)
    bad["p.biases"]["dtype"] = "F32"
    with pytest.raises(C.CheckpointError, match="share one dtype"):
        C.quantized_layer_specs(bad, 4, 64)


def test_quantization_config(tmp_path):
    cfg = tmp_path / "config.json"
    cfg.write_text(json.dumps({"model_type": "llama", "quantization": {"group_size": 64, "bits": 4}}))
    assert C.quantization_config(str(cfg)) == (4, 64)
    assert C.quantization_config({"quantization": {"bits": 8, "group_size": 32}}) == (8, 32)
    with pytest.raises(C.CheckpointError, match="no quantization"):
        C.quantization_config({"model_type": "llama"})
    with pytest.raises(TypeError, match="bits must be 2, 4, or 8"):
        C.quantization_config({"quantization": {"bits": 3, "group_size": 32}})
