"""Ordering of library work against the caller's torch stream.

A device-resident entry point called with stream NULL runs on the context's stream. That
stream is a blocking HIP stream, so it must start after every kernel the caller queued on
torch's default (null) stream and finish before anything queued there afterwards. Each
test holds the caller's stream busy with a GPU sleep, refills the input behind it, calls
the library and reads the output back with a torch kernel queued right after the call:
without the ordering the library reads the stale input (or the clone reads an unfinished
output), and the result differs from the oracle.
"""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

SLEEP_CYCLES = int(2e8)   # tens of milliseconds of GPU time queued ahead of the call


def _setup(device, rows=512, columns=2048, seed=7):
    rng = np.random.default_rng(seed)
    host = orc.random_matrix(rng, 1, rows, columns, 8)
    m = device.allocate(1, rows, columns, 8)
    m.upload(0, host.packed)
    m.upload(1, host.scales)
    m.upload(2, host.biases)
    x_new = rng.normal(size=columns).astype(np.float32)
    return host, m, x_new


def test_null_stream_fill_is_seen_by_a_null_stream_call(device):
    host, m, x_new = _setup(device)
    try:
        assert torch.cuda.current_stream().cuda_stream == 0
        src = torch.from_numpy(x_new).cuda()
        x = torch.zeros_like(src)
        y = torch.full((host.rows,), float("nan"), device="cuda")
        torch.cuda.synchronize()
        torch.cuda._sleep(SLEEP_CYCLES)        # caller's stream busy ...
        x.copy_(src)                           # ... then the input refilled behind it
        dh.qmv(device, m, x, y, x_dtype=dh.F32, y_dtype=dh.F32)
        out = y.clone()                        # read back on the caller's stream
        y.zero_()                              # and overwritten there afterwards
        torch.cuda.synchronize()
        want = orc.qmv_f64(host, x_new)
        assert orc.rel_err(out.cpu().numpy(), want) < 1e-5
        assert float(y.abs().max()) == 0.0
    finally:
        m.dispose()


def test_side_stream_call_runs_on_that_stream(device):
    host, m, x_new = _setup(device, seed=8)
    try:
        s = torch.cuda.Stream()
        src = torch.from_numpy(x_new).cuda()
        x = torch.zeros_like(src)
        y = torch.full((host.rows,), float("nan"), device="cuda")
        torch.cuda.synchronize()
        with torch.cuda.stream(s):
            torch.cuda._sleep(SLEEP_CYCLES)
            x.copy_(src)
            dh.qmv(device, m, x, y, x_dtype=dh.F32, y_dtype=dh.F32)   # current stream = s
            out = y.clone()
        s.synchronize()
        want = orc.qmv_f64(host, x_new)
        assert orc.rel_err(out.cpu().numpy(), want) < 1e-5
    finally:
        m.dispose()


def test_null_stream_fill_before_prefill_moe(device):
    """The multi-launch prefill entry (routing, grouping, GEMMs, merge) behind a busy
    caller stream: ids and residual must come from the refilled inputs."""
    rng = np.random.default_rng(9)
    T, E, H, I = 64, 16, 512, 128
    L = orc.MoeLayer(None, *(orc.random_matrix(rng, e, r, c, 8) for e, r, c in
                             ((E, I, H), (E, I, H), (E, H, I), (1, I, H), (1, I, H), (1, H, I), (1, 1, H))))
    qs = []
    for mm in (L.gate, L.up, L.down, L.shared_gate, L.shared_up, L.shared_down, L.shared_route):
        q = device.allocate(mm.experts, mm.rows, mm.columns, mm.bits)
        q.upload(0, mm.packed); q.upload(1, mm.scales); q.upload(2, mm.biases)
        qs.append(q)
    try:
        layer = dh.make_layer(None, *qs)
        xs = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        lg = orc.f32_to_bf16_bits(rng.normal(size=(T, E)).astype(np.float32))
        xsrc = torch.from_numpy(xs.view(np.int16)).cuda()
        lsrc = torch.from_numpy(lg.view(np.int16)).cuda()
        xd = torch.zeros_like(xsrc)
        ld = torch.zeros_like(lsrc)
        res = torch.full((T, H), 0x7fc0, dtype=torch.int16, device="cuda")   # bf16 NaN
        ids = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
        torch.cuda.synchronize()
        torch.cuda._sleep(SLEEP_CYCLES)
        xd.copy_(xsrc)
        ld.copy_(lsrc)
        res.zero_()
        dh.moe_prefill(device, layer, T, xd, ld, res, trace=dh.make_trace(ids=ids))
        got_ids = ids.clone()
        got_res = res.clone()
        torch.cuda.synchronize()
        oid, opr = orc.top8_bf16(lg)
        assert np.array_equal(got_ids.cpu().numpy(), oid)
        want = orc.moe_f64(L, orc.bf16_bits_to_f32(xs), oid, opr)
        got = orc.bf16_bits_to_f32(got_res.cpu().numpy().view(np.uint16)).astype(np.float64)
        scale = float(np.sqrt(np.mean(want * want)))
        assert np.max(np.abs(got - want) - np.abs(want) * 2.0 ** -8) / scale < 1e-2
    finally:
        for q in qs:
            q.dispose()
