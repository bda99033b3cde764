"""GPU tests of checkpoint loading (Qwen36Weights.Matrix / the MoE layer of
Qwen36Weights.cs:66-99): tensor bytes land in device memory unchanged, validation happens
before anything is allocated, and a decode step on a loaded layer is bit-identical to the
same step on the layer uploaded directly."""
import ctypes

import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from tests import ckpt_util as cu
from oracle import oracle as orc
from tests.test_gpu_hotpath import _moe_layer, _upload_layer, dev_bf16

pytestmark = pytest.mark.gpu


def device_bytes(m: dh.QuantMatrix, index: int) -> bytes:
    """Raw device buffer contents through the library's staging copy."""
    L = dh.load()
    n = m.buffer_bytes(index)
    p = L.dih_quant_matrix_buffer(m.handle, index)
    assert p
    data = ctypes.string_at(p, n)
    err = ctypes.create_string_buffer(256)
    assert L.dih_quant_matrix_commit(m.handle, err, 256) == 0, err.value
    return data


def tensors_of(prefix, q: orc.QMatrix):
    lead = () if q.experts == 1 else (q.experts,)
    return cu.matrix_tensors(prefix,
                             q.packed.reshape(lead + (q.rows, q.columns * q.bits // 32)),
                             q.scales.reshape(lead + (q.rows, q.columns // 64)),
                             q.biases.reshape(lead + (q.rows, q.columns // 64)))


def test_matrices_load_byte_exact_across_shards(device, tmp_path):
    rng = np.random.default_rng(11)
    a = orc.random_matrix(rng, 3, 130, 256, 8)
    b = orc.random_matrix(rng, 1, 64, 192, 5)
    t = {}
    t.update(tensors_of("m8", a))
    t.update(tensors_of("m5", b))
    cu.write_checkpoint(tmp_path, t, bits=5, shards=3)   # PREFIX.weight/.scales/.biases split over shards
    with dh.Checkpoint(tmp_path) as ck:
        m8 = ck.matrix(device, "m8", 130, 256, experts=3, bits=8)
        m5 = ck.matrix(device, "m5", 64, 192)            # bits 0 -> the checkpoint's 5
        try:
            assert (m5.bits, m8.bits) == (5, 8)
            for m, q in ((m8, a), (m5, b)):
                assert device_bytes(m, 0) == q.packed.tobytes()
                assert device_bytes(m, 1) == q.scales.tobytes()
                assert device_bytes(m, 2) == q.biases.tobytes()
        finally:
            m8.dispose()
            m5.dispose()


def test_matrix_validation(device, tmp_path):
    rng = np.random.default_rng(12)
    q = orc.random_matrix(rng, 1, 32, 128, 8)
    t = tensors_of("ok", q)
    bad = tensors_of("f32scales", q)
    bad["f32scales.scales"] = ("F32", (32, 2), np.zeros((32, 2), np.float32).tobytes())
    t.update(bad)
    cu.write_checkpoint(tmp_path, t, bits=8, quant_overrides={"ok": {"bits": 5, "group_size": 64}})
    with dh.Checkpoint(tmp_path) as ck:
        with pytest.raises(dh.NotSupportedError, match="quantization override"):
            ck.matrix(device, "ok", 32, 128)
        with pytest.raises(dh.NotSupportedError, match="U32 packed weights"):
            ck.matrix(device, "f32scales", 32, 128)
        with pytest.raises(dh.InvalidDataError, match="shape mismatch"):
            ck.matrix(device, "ok", 32, 192, bits=5)
        with pytest.raises(dh.InvalidDataError, match="Missing tensor shard"):
            ck.matrix(device, "absent", 32, 128)


@pytest.mark.parametrize("bits", [8])
def test_loaded_moe_layer_decodes_identically(device, tmp_path, bits):
    """Full config-2 layer written in the checkpoint layout, loaded by dih_checkpoint_moe_layer,
    then one decode step each on the loaded and the directly uploaded layer: identical
    residuals, ids and logits."""
    rng = np.random.default_rng(13)
    E, H, I = 256, 2048, 512
    L = _moe_layer(rng, E, H, I, bits)
    p = "language_model.model.layers.3."
    names = ["mlp.gate", "mlp.switch_mlp.gate_proj", "mlp.switch_mlp.up_proj", "mlp.switch_mlp.down_proj",
             "mlp.shared_expert.gate_proj", "mlp.shared_expert.up_proj", "mlp.shared_expert.down_proj",
             "mlp.shared_expert_gate"]
    mats = [L.router, L.gate, L.up, L.down, L.shared_gate, L.shared_up, L.shared_down, L.shared_route]
    t = {}
    for n, q in zip(names, mats):
        t.update(tensors_of(p + n, q))
    cu.write_checkpoint(tmp_path, t, bits=bits, shards=2)
    del t
    q, ref_layer = _upload_layer(device, L)
    with dh.Checkpoint(tmp_path) as ck:
        layer, owned = ck.moe_layer(device, 3)
    try:
        x = dev_bf16(orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32)))
        r0 = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        outs = []
        for lay in (ref_layer, layer):
            res = dev_bf16(r0)
            lg = torch.zeros(E, dtype=torch.float32, device="cuda")
            ids = torch.zeros(8, dtype=torch.int32, device="cuda")
            dh.moe_decode(device, lay, x, res, trace=dh.make_trace(logits=lg, ids=ids))
            torch.cuda.synchronize()
            outs.append((res.cpu().numpy(), lg.cpu().numpy(), ids.cpu().numpy()))
        for a, b in zip(*outs):
            assert np.array_equal(a, b)
    finally:
        for m in q + owned:
            if m is not None:
                m.dispose()
