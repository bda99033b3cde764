"""CPU tests of the checkpoint reader (SafeTensors.cs, Qwen36Weights.cs). The safetensors cases
mirror tests/DeepInfer.Tests/SafeTensorsTests.cs fixture for fixture (same header JSON, bytes,
offsets and expected outcome); format compatibility is pinned against files written by the
`safetensors` package itself (0.8.0 here). No GPU call is made."""
import json
import os
import struct

import numpy as np
import pytest

import deepinfer_hip as dh
from tests import ckpt_util as cu


def fixture(tmp_path, dtype, shape, offsets, values, duplicate=False, name="st"):
    """SafeTensorsTests.Fixture: {"test": entry} (+ "overlap": same entry), compact JSON."""
    entry = {"dtype": dtype, "shape": list(shape), "data_offsets": list(offsets)}
    header = {"test": entry}
    if duplicate:
        header["overlap"] = entry
    return cu.write_raw(tmp_path / name, json.dumps(header, separators=(",", ":")).encode(), bytes(values))


# ---- SafeTensorsTests.cs:10-20
def test_packed_unsigned_weights_read_without_float_conversion(tmp_path):
    data = bytes([1, 2, 3, 4, 255, 254, 253, 252])
    path = fixture(tmp_path, "U32", [1, 1, 1, 1, 2], [0, 8], data)
    with dh.SafeTensors(path) as f:
        t = f.get("test", 1, 1, 1, 1, 2)
        out = np.zeros(8, dtype=np.uint8)
        f.read_into(t, out)
        assert out.tobytes() == data
        with pytest.raises(dh.InvalidDataError):
            f.read_into(t, np.zeros(7, dtype=np.uint8))
        with pytest.raises(dh.InvalidDataError):
            f.read_float(t)


# ---- SafeTensorsTests.cs:21-30
def test_bfloat16_values_and_shape_are_validated(tmp_path):
    path = fixture(tmp_path, "BF16", [2, 2], [0, 8], [0, 0x3f, 0, 0x40, 0x80, 0x3f, 0x80, 0xbf])
    with dh.SafeTensors(path) as f:
        t = f.get("test", 2, 2)
        assert f.read_float(t).tolist() == [.5, 2.0, 1.0, -1.0]
        assert f.read_bfloat16(t).tolist() == [0x3f00, 0x4000, 0x3f80, 0xbf80]
        with pytest.raises(dh.InvalidDataError):
            f.get("test", 4)
        with pytest.raises(dh.InvalidDataError):
            f.get("missing", 2, 2)


# ---- SafeTensorsTests.cs:31-37
@pytest.mark.parametrize("start,end", [(0, 10), (-1, 7), (4, 12)])
def test_invalid_offsets_are_rejected(tmp_path, start, end):
    path = fixture(tmp_path, "BF16", [2, 2], [start, end], bytes(8))
    with pytest.raises(dh.InvalidDataError):
        dh.SafeTensors(path)


# ---- SafeTensorsTests.cs:38-44
def test_unsupported_dtype_and_overlapping_tensors_are_rejected(tmp_path):
    with pytest.raises(dh.NotSupportedError, match="Unsupported safetensors dtype 'F16'"):
        dh.SafeTensors(fixture(tmp_path, "F16", [2, 2], [0, 8], bytes(8), name="a"))
    with pytest.raises(dh.InvalidDataError, match="Overlapping tensors"):
        dh.SafeTensors(fixture(tmp_path, "BF16", [2, 2], [0, 8], bytes(8), duplicate=True, name="b"))


# ---- SafeTensorsTests.cs:45-51
def test_truncated_header_and_non_finite_values_are_rejected(tmp_path):
    path = fixture(tmp_path, "F32", [1], [0, 4], struct.pack("<f", float("nan")))
    with dh.SafeTensors(path) as f:
        with pytest.raises(dh.InvalidDataError, match="Non-finite"):
            f.read_float(f.get("test", 1))
    with open(path, "wb") as fh:
        fh.write(struct.pack("<Q", 2 ** 64 - 1))
    with pytest.raises(dh.InvalidDataError, match="header length"):
        dh.SafeTensors(path)


# ---- header rules beyond the reference's fixtures (SafeTensors.cs:18-43)
@pytest.mark.parametrize("header,kind,match", [
    (b"{}", None, None),                                                     # empty is valid
    (b"{ ", dh.InvalidDataError, "Invalid JSON"),
    (b'{"a":{"dtype":"U32","shape":[1],"data_offsets":[0,4]}} x', dh.InvalidDataError, "trailing"),
    (b'[]', dh.InvalidDataError, "not an object"),
    (b'{"a":{"dtype":"U32","shape":[],"data_offsets":[0,0]}}', dh.InvalidDataError, "shape"),
    (b'{"a":{"dtype":"U32","shape":[0],"data_offsets":[0,0]}}', dh.InvalidDataError, "shape"),
    (b'{"a":{"dtype":"U32","shape":[1,1,1,1,1,1,1,1,1],"data_offsets":[0,4]}}', dh.InvalidDataError, "shape"),
    (b'{"a":{"dtype":"U32","shape":[1.0],"data_offsets":[0,4]}}', dh.InvalidDataError, "shape"),
    (b'{"a":{"dtype":"U32","shape":[2147483648],"data_offsets":[0,4]}}', dh.InvalidDataError, "shape"),
    (b'{"a":{"dtype":"U32","shape":[1],"data_offsets":[0]}}', dh.InvalidDataError, "offsets"),
    (b'{"a":{"dtype":"U32","shape":[1]}}', dh.InvalidDataError, "entry"),
    (b'{"a":{"dtype":"U32","shape":[1],"data_offsets":[0,4]},"a":{"dtype":"U32","shape":[1],"data_offsets":[4,8]}}',
     dh.InvalidDataError, "Duplicate tensor name"),
    (b'{"a":{"dtype":"I8","shape":[1],"data_offsets":[0,1]}}', dh.NotSupportedError, "I8"),
])
def test_header_rules(tmp_path, header, kind, match):
    path = cu.write_raw(tmp_path / "h", header, bytes(8))
    if kind is None:
        with dh.SafeTensors(path) as f:
            assert f.tensors == {}
    else:
        with pytest.raises(kind, match=match):
            dh.SafeTensors(path)


def test_header_length_bounds(tmp_path):
    p = tmp_path / "short"
    p.write_bytes(b"\x01\x00\x00\x00\x00\x00\x00\x00{")   # length 1 < 2
    with pytest.raises(dh.InvalidDataError):
        dh.SafeTensors(p)
    p.write_bytes(struct.pack("<Q", 40) + b"{}")            # longer than the file
    with pytest.raises(dh.InvalidDataError):
        dh.SafeTensors(p)
    p.write_bytes(b"\x00" * 4)                             # no length at all
    with pytest.raises(dh.InvalidDataError):
        dh.SafeTensors(p)
    p.write_bytes(struct.pack("<Q", 16777217) + b" " * 16777217)
    with pytest.raises(dh.InvalidDataError):
        dh.SafeTensors(p)


def test_metadata_escapes_and_padding(tmp_path):
    """__metadata__ is skipped; names go through JSON escapes (\\u, surrogate pairs); the
    header may carry trailing spaces (the format pads it to 8 bytes)."""
    hdr = ('{"__metadata__":{"format":"pt"},"caf\\u00e9\\ud83d\\ude00":{"dtype":"F32","shape":[2],'
           '"data_offsets":[0,8]}}    ').encode()
    path = cu.write_raw(tmp_path / "m", hdr, struct.pack("<2f", 1.5, -2.0))
    with dh.SafeTensors(path) as f:
        assert list(f.tensors) == ["café\U0001F600"]
        assert f.read_float(f.get("café\U0001F600", 2)).tolist() == [1.5, -2.0]


def test_nesting_limit(tmp_path):
    deep = b'{"__metadata__":' + b"[" * 70 + b"]" * 70 + b"}"
    with pytest.raises(dh.InvalidDataError, match="deep"):
        dh.SafeTensors(cu.write_raw(tmp_path / "d", deep, b""))


def test_files_written_by_the_safetensors_package(tmp_path):
    """Byte-exact reads of U32 / F32 / BF16 tensors written by safetensors.torch.save_file."""
    import torch
    from safetensors.torch import save_file
    rng = np.random.default_rng(3)
    packed = rng.integers(0, 2 ** 32, size=(3, 5, 16), dtype=np.uint64).astype(np.uint32)
    f32 = rng.normal(size=(7,)).astype(np.float32)
    bf = torch.tensor(rng.normal(size=(4, 6)), dtype=torch.bfloat16)
    path = tmp_path / "pkg.safetensors"
    save_file({"w": torch.from_numpy(packed.view(np.int32)).view(torch.uint32), "v": torch.from_numpy(f32),
               "s": bf}, str(path), metadata={"format": "mlx"})
    with dh.SafeTensors(path) as f:
        t = f.tensors
        assert (t["w"].dtype, t["v"].dtype, t["s"].dtype) == ("U32", "F32", "BF16")
        assert t["w"].shape == (3, 5, 16)
        out = np.zeros(packed.shape, dtype=np.uint32)
        f.read_into(f.get("w", 3, 5, 16), out)
        assert np.array_equal(out, packed)
        assert np.array_equal(f.read_float(f.get("v", 7)), f32)
        assert np.array_equal(f.read_bfloat16(f.get("s", 4, 6)), bf.view(torch.int16).numpy().view(np.uint16).ravel())
        assert np.array_equal(f.read_float(f.get("s", 4, 6)), bf.float().numpy().ravel())


def test_disposed_reader_raises(tmp_path):
    f = dh.SafeTensors(fixture(tmp_path, "U32", [2], [0, 8], bytes(8)))
    t = f.get("test", 2)
    f.dispose()
    with pytest.raises(dh.ObjectDisposedError):
        f.read_float(t)


# ---- checkpoint directory (Qwen36Weights.cs:27-65, 82)
def test_checkpoint_config_and_vectors(tmp_path):
    norm = np.linspace(-1, 1, 2048).astype(np.float32)
    cu.write_checkpoint(tmp_path, {"language_model.model.norm.weight": ("F32", (2048,), norm.tobytes())},
                        bits=5, eps=1e-6, theta=1e7)
    with dh.Checkpoint(tmp_path) as c:
        assert (c.weight_bits, c.epsilon, c.rope_theta) == (5, np.float32(1e-6), np.float32(1e7))
        assert np.array_equal(c.vector("language_model.model.norm.weight", 2048), norm)
        with pytest.raises(dh.InvalidDataError, match="shape mismatch"):
            c.vector("language_model.model.norm.weight", 1024)
        with pytest.raises(dh.InvalidDataError, match="Missing tensor shard"):
            c.vector("language_model.model.layers.0.input_layernorm.weight", 2048)


@pytest.mark.parametrize("edit,kind,match", [
    (lambda cfg: cfg.update(model_type="qwen3_moe"), dh.NotSupportedError, "geometry"),
    (lambda cfg: cfg["text_config"].update(num_experts=128), dh.NotSupportedError, "geometry"),
    (lambda cfg: cfg["text_config"].update(norm_topk_prob=False), dh.NotSupportedError, "geometry"),
    (lambda cfg: cfg["text_config"].update(max_position_embeddings=131072), dh.NotSupportedError, "context"),
    (lambda cfg: cfg["text_config"]["rope_parameters"].update(rope_type="yarn"), dh.NotSupportedError, "RoPE"),
    (lambda cfg: cfg["text_config"]["rope_parameters"].update(partial_rotary_factor=0.5), dh.NotSupportedError, "RoPE"),
    (lambda cfg: cfg["text_config"].update(rms_norm_eps=0), dh.InvalidDataError, "normalization"),
    (lambda cfg: cfg["text_config"]["rope_parameters"].update(rope_theta=1), dh.InvalidDataError, "normalization"),
    (lambda cfg: cfg["quantization"].update(bits=4), dh.NotSupportedError, "affine"),
    (lambda cfg: cfg["quantization"].update(group_size=32), dh.NotSupportedError, "affine"),
    (lambda cfg: cfg["quantization"].update(mode="mxfp4"), dh.NotSupportedError, "affine"),
])
def test_checkpoint_config_rules(tmp_path, edit, kind, match):
    cu.write_checkpoint(tmp_path, {}, edit=edit)
    with pytest.raises(kind, match=match):
        dh.Checkpoint(tmp_path)


def test_checkpoint_unsafe_shard_path_and_non_finite_vector(tmp_path):
    bad = np.array([1.0, np.inf], dtype=np.float32)
    cu.write_checkpoint(tmp_path, {"v": ("F32", (2,), bad.tobytes())},
                        extra_map={"escape": "../model.safetensors", "nested": "sub/model.safetensors"})
    with dh.Checkpoint(tmp_path) as c:
        with pytest.raises(dh.InvalidDataError, match="Non-finite"):
            c.vector("v", 2)
        with pytest.raises(dh.InvalidDataError, match="Unsafe shard path"):
            c.vector("escape", 2)
        with pytest.raises(dh.InvalidDataError, match="Unsafe shard path"):
            c.vector("nested", 2)


def test_checkpoint_missing_index(tmp_path):
    cu.write_checkpoint(tmp_path, {})
    os.remove(tmp_path / "model.safetensors.index.json")
    with pytest.raises(dh.InvalidDataError, match="index"):
        dh.Checkpoint(tmp_path)
