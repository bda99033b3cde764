"""Test helpers that write safetensors files and MLX-layout checkpoint directories (plain
format writers; the reader under test is the library's)."""
import json
import os
import struct


def write_raw(path, header: bytes, data: bytes):
    """u64 little-endian header length, header bytes, data section."""
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(header)))
        f.write(header)
        f.write(data)
    return path


def write_safetensors(path, tensors: dict):
    """tensors: name -> (dtype, shape, raw bytes), laid out in insertion order."""
    header, off, blobs = {}, 0, []
    for name, (dtype, shape, raw) in tensors.items():
        header[name] = {"dtype": dtype, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        off += len(raw)
        blobs.append(raw)
    h = json.dumps(header, separators=(",", ":")).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)
    return path


def qwen36_config(bits=8, eps=1e-6, theta=1e7):
    """config.json fields Qwen36Weights checks (Qwen36Weights.cs:27-53)."""
    return {
        "model_type": "qwen3_5_moe",
        "text_config": {
            "hidden_size": 2048, "num_hidden_layers": 40, "num_experts": 256, "num_experts_per_tok": 8,
            "moe_intermediate_size": 512, "vocab_size": 248320, "num_attention_heads": 16,
            "num_key_value_heads": 2, "head_dim": 256, "full_attention_interval": 4,
            "linear_num_value_heads": 32, "linear_num_key_heads": 16, "linear_key_head_dim": 128,
            "linear_value_head_dim": 128, "linear_conv_kernel_dim": 4, "norm_topk_prob": True,
            "max_position_embeddings": 262144, "rms_norm_eps": eps,
            "rope_parameters": {"rope_theta": theta, "partial_rotary_factor": 0.25, "rope_type": "default"},
        },
        "quantization": {"group_size": 64, "bits": bits, "mode": "affine"},
    }


def write_checkpoint(directory, tensors: dict, bits=8, eps=1e-6, theta=1e7, edit=None, extra_map=None,
                     shards=1, quant_overrides=None):
    """config.json + model.safetensors.index.json + `shards` shard files holding `tensors`
    (name -> (dtype, shape, raw bytes)) split round-robin by name."""
    os.makedirs(directory, exist_ok=True)
    cfg = qwen36_config(bits, eps, theta)
    if quant_overrides:
        cfg["quantization"].update(quant_overrides)
    if edit:
        edit(cfg)
    with open(os.path.join(directory, "config.json"), "w") as f:
        json.dump(cfg, f)
    names = list(tensors)
    parts = [dict() for _ in range(shards)]
    weight_map = {}
    for i, n in enumerate(names):
        parts[i % shards][n] = tensors[n]
        weight_map[n] = f"model-{i % shards + 1:05d}-of-{shards:05d}.safetensors"
    for k in range(shards):
        write_safetensors(os.path.join(directory, f"model-{k + 1:05d}-of-{shards:05d}.safetensors"), parts[k])
    if extra_map:
        weight_map.update(extra_map)
    with open(os.path.join(directory, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": weight_map}, f)
    return directory


def matrix_tensors(prefix, packed, scales, biases):
    """PREFIX.{weight,scales,biases} entries from uint32 / uint16-bit arrays."""
    return {
        prefix + ".weight": ("U32", packed.shape, packed.tobytes()),
        prefix + ".scales": ("BF16", scales.shape, scales.tobytes()),
        prefix + ".biases": ("BF16", biases.shape, biases.tobytes()),
    }
