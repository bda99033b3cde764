"""dih_moe_decode_noalloc against dih_moe_decode_norm: the same kernels on buffers carved
from the library's fixed per-GPU scratch array instead of the context's grow-only scratch.
Outputs (residual, normed row, router logits, ids, probs, per-slot down outputs) must be
bit-identical to the allocating entry point's on the same inputs, for two calls in a row,
the second on a smaller layer, and the integer routing must match the oracle's rule."""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc

pytestmark = pytest.mark.gpu


def _upload(device, host):
    m = device.allocate(host.experts, host.rows, host.columns, host.bits)
    m.upload(0, host.packed)
    m.upload(1, host.scales)
    m.upload(2, host.biases)
    return m


def _layer(device, rng, E, H, I, bits):
    hosts = [orc.random_matrix(rng, 1, E, H, 8, scale_lo=1.25e-4, scale_hi=5e-4)]
    hosts += [orc.random_matrix(rng, e, r, c, bits) for e, r, c in
              ((E, I, H), (E, I, H), (E, H, I), (1, I, H), (1, I, H), (1, H, I))]
    hosts.append(orc.random_matrix(rng, 1, 1, H, 8))
    mats = [_upload(device, h) for h in hosts]
    return mats, dh.make_layer(*mats)


def _bf16(rng, n):
    return torch.from_numpy(orc.f32_to_bf16_bits(rng.normal(size=n).astype(np.float32)).view(np.int16)).cuda()


def _step(device, fn, layer, E, H, x, res0, f32_residual, norm_w):
    res = res0.clone()
    lg = torch.zeros(E, dtype=torch.float32, device="cuda")
    ids = torch.zeros(8, dtype=torch.int32, device="cuda")
    probs = torch.zeros(8, dtype=torch.float32, device="cuda")
    rout = torch.zeros((9, H), dtype=torch.float32, device="cuda")
    normed = torch.zeros(H, dtype=torch.float32, device="cuda")
    merge = None
    if f32_residual or norm_w is not None:
        merge = dh.make_merge(residual_f32=f32_residual, norm_weight=norm_w, epsilon=1e-6,
                              normed=normed if norm_w is not None else None)
    fn(device, layer, x, res, trace=dh.make_trace(logits=lg, ids=ids, probs=probs, expert_out=rout), merge=merge)
    torch.cuda.synchronize()
    return [t.cpu().numpy() for t in (res, lg, ids, probs, rout, normed)]


@pytest.mark.parametrize("order", ["noalloc_first", "allocating_first"])
def test_noalloc_decode_matches_allocating_entry(device, order):
    rng = np.random.default_rng(17)
    cases = [  # (E, H, I, bits, f32 residual, fused norm): the second call is smaller
        (256, 2048, 512, 8, False, False),
        (64, 1024, 256, 5, True, True),
    ]
    for E, H, I, bits, f32_res, with_norm in cases:
        mats, layer = _layer(device, rng, E, H, I, bits)
        try:
            x = _bf16(rng, H)
            res0 = (torch.randn(H, device="cuda") if f32_res else _bf16(rng, H))
            norm_w = torch.rand(H, device="cuda") + 0.5 if with_norm else None
            fns = [dh.moe_decode_noalloc, dh.moe_decode]
            if order == "allocating_first":
                fns.reverse()
            outs = [_step(device, fn, layer, E, H, x, res0, f32_res, norm_w) for fn in fns]
            for a, b in zip(*outs):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8))
            lg, ids, probs = outs[0][1], outs[0][2], outs[0][3]
            oid, opr = orc.top8(lg)
            assert np.array_equal(ids, oid)
            assert np.max(np.abs(probs - opr)) <= 1e-6
            r = outs[0][0] if f32_res else orc.bf16_bits_to_f32(outs[0][0].view(np.uint16))
            assert np.all(np.isfinite(r))
        finally:
            for m in mats:
                m.dispose()


def test_noalloc_decode_rejects_invalid_arguments_before_launch(device):
    rng = np.random.default_rng(18)
    mats, layer = _layer(device, rng, 16, 256, 128, 8)
    try:
        res = torch.full((256,), 7, dtype=torch.int16, device="cuda")
        with pytest.raises(dh.ArgumentError):
            dh.moe_decode_noalloc(device, layer, None, res)
        bad = dh.make_layer(mats[0], mats[1], mats[2], mats[2], mats[4], mats[5], mats[6], mats[7])
        with pytest.raises(dh.ArgumentError):
            dh.moe_decode_noalloc(device, bad, _bf16(rng, 256), res)
        torch.cuda.synchronize()
        assert bool((res == 7).all())
    finally:
        for m in mats:
            m.dispose()
