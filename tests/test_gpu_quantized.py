"""GPU tests of the synchronous host-pointer ABI, mirroring the reference's
tests/DeepInfer.Tests/QuantizedTests.cs one test per reference test.

They call libdeepinfer_hip through the C ABI (ctypes) via the QuantizedHip mirror of
QuantizedMetal. Expected values come from the reference's own closed forms
(QuantizedTests.cs:136-165) accumulated in double, with the reference's tolerances.
"""
import numpy as np
import pytest

import deepinfer_hip as dh
from tests.refcases import populate, scalar_weights

pytestmark = pytest.mark.gpu


def _load(m_host, qm):
    qm.write(0, m_host.packed)
    qm.write(1, m_host.scales)
    qm.write(2, m_host.biases)


@pytest.mark.parametrize("bits,columns,batched", [
    (5, 512, True), (8, 512, False), (5, 2048, False), (8, 2048, True), (5, 4096, True),
    (8, 4096, False), (5, 64, True), (8, 64, False), (5, 192, False), (8, 192, True),
    (5, 256, True), (8, 256, False)])
def test_tiled_gemv_matches_independent_scalar_with_tail_rows_and_eight_experts(device, bits, columns, batched):
    """QuantizedTests.cs:49-70."""
    m = device.allocate(9, 129, columns, bits)
    try:
        _load(populate(9, 129, columns, bits, 3), m)
        ids = [8, 0, 6, 2, 5, 1, 7, 3]
        x = (np.sin(np.arange(columns * (8 if batched else 1), dtype=np.float32) * np.float32(.013)) * np.float32(.1)).astype(np.float32)
        out = np.zeros(129 * 8, dtype=np.float32)
        m.multiply_experts(x, out, ids, batched)
        w = scalar_weights(9, 129, columns, bits, 3).astype(np.float64)
        for slot in range(8):
            xs = x[(slot * columns if batched else 0):][:columns].astype(np.float64)
            expected = w[ids[slot]] @ xs
            assert np.max(np.abs(expected - out[slot * 129:(slot + 1) * 129])) <= 3e-4
    finally:
        m.dispose()


@pytest.mark.parametrize("bits,columns", [(5, 128), (8, 128), (5, 256), (8, 256)])
def test_fused_experts_match_scalar_swiglu_and_down_across_changed_inputs(bits, columns):
    """QuantizedTests.cs:71-117 (own device: the dispatch/submission counts are asserted)."""
    with dh.QuantizedHip() as device:
        gate = device.allocate(9, 192, columns, bits)
        up = device.allocate(9, 192, columns, bits)
        down = device.allocate(9, columns, 192, 8 if bits == 5 else 5)
        shared = device.allocate(1, columns, 64, 5)
        _load(populate(9, 192, columns, bits, 1), gate)
        _load(populate(9, 192, columns, bits, 2), up)
        _load(populate(9, columns, 192, 8 if bits == 5 else 5, 3), down)
        _load(populate(1, columns, 64, 5, 4), shared)
        ids = [8, 0, 6, 2, 5, 1, 7, 3]
        inp = (np.sin(np.arange(columns, dtype=np.float32) * np.float32(.13)) * np.float32(.1)).astype(np.float32)
        sin = (np.cos(np.arange(64, dtype=np.float32) * np.float32(.07)) * np.float32(.2)).astype(np.float32)
        out = np.zeros(columns * 8, dtype=np.float32)
        sout = np.zeros(columns, dtype=np.float32)
        wg = scalar_weights(9, 192, columns, bits, 1).astype(np.float64)
        wu = scalar_weights(9, 192, columns, bits, 2).astype(np.float64)
        wd = scalar_weights(9, columns, 192, 8 if bits == 5 else 5, 3).astype(np.float64)
        ws = scalar_weights(1, columns, 64, 5, 4).astype(np.float64)
        for _ in range(2):
            inp[0] += np.float32(.15)
            sin[0] -= np.float32(.2)
            ids.reverse()
            device.expert_mlp(gate, up, down, shared, inp, sin, ids, out, sout)
            for slot in range(8):
                g = wg[ids[slot]] @ inp.astype(np.float64)
                u = wu[ids[slot]] @ inp.astype(np.float64)
                act = g / (1 + np.exp(-g)) * u
                expected = wd[ids[slot]] @ act
                assert np.max(np.abs(expected - out[slot * columns:(slot + 1) * columns])) <= 3e-4
            assert np.max(np.abs(ws[0] @ sin.astype(np.float64) - sout)) <= 3e-4
        assert device.dispatches == 6 and device.submissions == 2


def test_invalid_fused_expert_call_does_not_submit_or_overwrite_outputs():
    """QuantizedTests.cs:118-135."""
    with dh.QuantizedHip() as d, dh.QuantizedHip() as other:
        gate = d.allocate(3, 64, 64, 5)
        up = d.allocate(3, 64, 64, 5)
        down = d.allocate(3, 64, 64, 8)
        shared = d.allocate(1, 64, 64, 5)
        foreign = other.allocate(3, 64, 64, 5)
        x = np.zeros(64, dtype=np.float32)
        y = np.full(128, -2, dtype=np.float32)
        sy = np.zeros(64, dtype=np.float32)
        with pytest.raises(dh.ArgumentOutOfRangeError):
            d.expert_mlp(gate, up, down, shared, x, x, [3, 0], y, sy)
        with pytest.raises(dh.ArgumentError):
            d.expert_mlp(gate, up, down, shared, np.zeros(63, dtype=np.float32), x, [1, 0], y, sy)
        with pytest.raises(dh.ArgumentError):
            d.expert_mlp(gate, foreign, down, shared, x, x, [1, 0], y, sy)
        with pytest.raises(dh.ArgumentError):
            d.expert_mlp(gate, gate, down, shared, x, x, [1, 0], y, sy)
        with pytest.raises(dh.ArgumentError):
            d.expert_mlp(gate, up, down, shared, x, x, [1, 0], y, y[:64])
        up.dispose()
        with pytest.raises(dh.ObjectDisposedError):
            d.expert_mlp(gate, up, down, shared, x, x, [1, 0], y, sy)
        assert d.submissions == 0
        assert np.all(y == -2)


@pytest.mark.parametrize("batching", [True, False])
def test_independent_mixed_gemvs_preserve_outputs_with_one_batch_wait(batching):
    """QuantizedTests.cs:166-209: zero codes, scale 1.0, bias (j+1)+(row index)*.25."""
    with dh.QuantizedHip(batch_submissions=batching) as device:
        a = device.allocate(1, 3, 64, 5)
        b = device.allocate(3, 7, 128, 8)
        c = device.allocate(2, 5, 64, 5)
        d = device.allocate(1, 4, 64, 8)
        mats = [a, b, c, d]
        for j, m in enumerate(mats):
            groups = m.columns // 64
            m.write(0, np.zeros(m.experts * m.rows * m.columns * m.bits // 8, dtype=np.uint8))
            n = m.experts * m.rows * groups
            m.write(1, np.full(n, 0x3F80, dtype=np.uint16))
            vals = ((j + 1) + (np.arange(n) // groups) * np.float32(.25)).astype(np.float32)
            m.write(2, (vals.view(np.uint32) >> 16).astype(np.uint16))
        inp = ((np.arange(64) - 20) * np.float32(.01)).astype(np.float32)
        bat = ((np.arange(256) - 100) * np.float32(.005)).astype(np.float32)
        jobs = [dh.QuantizedJob(a, inp, np.zeros(3, dtype=np.float32)),
                dh.QuantizedJob(b, bat, np.zeros(14, dtype=np.float32), [2, 0], True),
                dh.QuantizedJob(c, inp, np.zeros(10, dtype=np.float32), [1, 0]),
                dh.QuantizedJob(d, inp, np.zeros(4, dtype=np.float32))]
        for _ in range(2):
            inp[0] += np.float32(.25)
            bat[0] -= np.float32(.5)
            device.multiply_batch(jobs)
            for j, job in enumerate(jobs):
                m = job.matrix
                experts = job.experts or [0]
                for slot, e in enumerate(experts):
                    xs = job.input[(slot * m.columns if job.batched else 0):][:m.columns]
                    for row in range(m.rows):
                        expected = np.float32(((j + 1) + (e * m.rows + row) * .25)) * xs.astype(np.float64).sum()
                        assert abs(expected - job.output[slot * m.rows + row]) <= 2e-4
        assert device.dispatches == 8
        assert device.submissions == (2 if batching else 8)


def test_invalid_batch_has_no_partial_submission_or_output():
    """QuantizedTests.cs:210-227."""
    with dh.QuantizedHip() as device, dh.QuantizedHip() as other:
        a = device.allocate(1, 64, 64, 5)
        b = device.allocate(1, 64, 64, 5)
        foreign = other.allocate(1, 64, 64, 5)
        inp = np.zeros(64, dtype=np.float32)
        out = np.full(64, -3, dtype=np.float32)
        z = lambda n: np.zeros(n, dtype=np.float32)  # noqa: E731
        with pytest.raises(dh.ArgumentError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(a, inp, z(64))])
        with pytest.raises(dh.ArgumentError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(b, out, z(64))])
        with pytest.raises(dh.ArgumentError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(foreign, inp, z(64))])
        with pytest.raises(dh.ArgumentError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(b, inp, z(63))])
        with pytest.raises(dh.ArgumentOutOfRangeError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(b, inp, z(64), [1])])
        b.dispose()
        with pytest.raises(dh.ObjectDisposedError):
            device.multiply_batch([dh.QuantizedJob(a, inp, out), dh.QuantizedJob(b, inp, z(64))])
        assert device.submissions == 0
        assert np.all(out == -3)


@pytest.mark.parametrize("bits", [5, 8])
def test_selected_expert_gemv_matches_scalar_quantization(device, bits):
    """QuantizedTests.cs:228-256: scale 1.0, bias 0.5 => y = sum (q+.5)*x."""
    from oracle.oracle import QMatrix, pack_codes
    e = np.arange(3)[:, None, None]
    r = np.arange(7)[None, :, None]
    c = np.arange(128)[None, None, :]
    q = ((c * 7 + e * 3 + r) & ((1 << bits) - 1)).astype(np.uint32)
    host = QMatrix(pack_codes(q, bits), np.full(3 * 7 * 2, 0x3F80, np.uint16), np.full(3 * 7 * 2, 0x3F00, np.uint16),
                   3, 7, 128, bits)
    m = device.allocate(3, 7, 128, bits)
    try:
        _load(host, m)
        x = np.sin(np.arange(256, dtype=np.float32) * np.float32(.17)).astype(np.float32)
        y = np.zeros(14, dtype=np.float32)
        m.multiply_experts(x, y, [2, 0], batched=True)
        for slot, ex in enumerate([2, 0]):
            expected = ((q[ex].astype(np.float64) + .5) @ x[slot * 128:(slot + 1) * 128].astype(np.float64))
            assert np.max(np.abs(expected - y[slot * 7:(slot + 1) * 7])) <= .004
    finally:
        m.dispose()


def test_embedding_row_matches_scalar_dequant(device):
    """CopyRow / di_quant_embedding (quantized.mm:384-397) against ScalarWeight."""
    for bits in (5, 8):
        m = device.allocate(1, 5, 192, bits)
        try:
            _load(populate(1, 5, 192, bits, 2), m)
            out = np.zeros(192, dtype=np.float32)
            m.copy_row(3, out)
            assert np.array_equal(out, scalar_weights(1, 5, 192, bits, 2)[0, 3])
            with pytest.raises(dh.ArgumentError):
                m.copy_row(5, out)
        finally:
            m.dispose()


def test_residency_reporting(device):
    """ExplicitResidency... (QuantizedTests.cs:28-47): bytes reported only when resident,
    and released with the matrix."""
    with dh.QuantizedHip(residency=True, residency_refresh_milliseconds=20) as enabled, \
            dh.QuantizedHip(residency=False) as disabled:
        ordinary = disabled.allocate(1, 64, 64, 8)
        assert disabled.residency_bytes == 0
        matrix = enabled.allocate(1, 64, 64, 8)
        assert enabled.residency_bytes >= 4096
        enabled.prepare_residency()
        enabled.prepare_residency()
        _load(populate(1, 64, 64, 8, 3), matrix)
        _load(populate(1, 64, 64, 8, 3), ordinary)
        x = np.full(64, .125, dtype=np.float32)
        a = np.zeros(64, dtype=np.float32)
        b = np.zeros(64, dtype=np.float32)
        matrix.multiply_experts(x, a, [0], False)
        ordinary.multiply_experts(x, b, [0], False)
        assert np.array_equal(a, b)
        matrix.dispose()
        assert enabled.residency_bytes == 0
