"""GPU parity of dih_attention (BF16 prefill attention + partition combine) against
oracle.attention_f64, following the reference's own checks:

* prefill_attention_checks.mm: xorshift inputs (seed 0x6a51c9e7), bases 0..4098, query
  counts 1..128, query offsets, BF16 double oracle; |diff| <= 3e-5 and relative L2
  <= 1e-4 (:72, :76).
* bf16_attention_long_checks.mm: zero queries over values 1 / -2 give exactly .5 / -1
  (sigmoid(0) = .5) at every position up to the 262144-row cache (:13, :20).
* attention_batch_checks.mm: a chunk computed as 128-query calls equals one call over
  the whole chunk, outputs outside the chunk untouched (:28-38).
"""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

ABS_TOL, REL_L2 = 3e-5, 1e-4


def _bf16_dev(a):
    return torch.from_numpy(orc.f32_to_bf16_bits(np.asarray(a, np.float32)).view(np.int16)).cuda()


class Inputs:
    """q [storage, 4096], raw [storage, 8192] (x5), keys/values [cap, 512] bf16, drawn
    like prefill_attention_checks.mm:17-26."""

    def __init__(self, storage, cap, seed=0x6a51c9e7):
        (q,), s = orc.xorshift_values(seed, storage * 4096)
        (k, v), s = orc.xorshift_values(s, cap * 512, 2)
        (r,), s = orc.xorshift_values(s, storage * 8192)
        self.q = q.reshape(storage, 4096)
        self.kb = orc.f32_to_bf16_bits(k).reshape(cap, 512)
        self.vb = orc.f32_to_bf16_bits(v).reshape(cap, 512)
        self.k = orc.bf16_bits_to_f32(self.kb)
        self.v = orc.bf16_bits_to_f32(self.vb)
        self.raw = (r * 5).reshape(storage, 8192)
        self.dq = torch.from_numpy(self.q).cuda()
        self.dk = torch.from_numpy(self.kb.view(np.int16)).cuda()
        self.dv = torch.from_numpy(self.vb.view(np.int16)).cuda()
        self.draw = torch.from_numpy(self.raw).cuda()


def _check(got, want):
    got = np.asarray(got, np.float64)
    diff = np.abs(got - want)
    assert np.all(np.isfinite(got))
    worst = float(diff.max())
    rel = float(np.sqrt(np.sum(diff ** 2) / max(np.sum(want ** 2), 1e-30)))
    assert worst <= ABS_TOL and rel <= REL_L2, (worst, rel)


@pytest.fixture(scope="module")
def inputs():
    return Inputs(256, 8192)


@pytest.mark.parametrize("base,count,offset", [
    (0, 1, 0), (0, 3, 0), (0, 17, 0), (0, 128, 0), (31, 3, 128), (31, 65, 0), (1022, 5, 0),
    (1022, 32, 0), (2047, 128, 128), (4098, 1, 0), (4098, 128, 128)])
def test_attention_random_oracle(device, inputs, base, count, offset):
    """Random causal inputs at the library's own partition choice."""
    I = inputs
    position = base + offset
    part = dh.attention_partition(position, count)
    out = torch.full((256, 4096), float("nan"), device="cuda")
    dh.attention(device, I.dq[offset:], I.dk, I.dv, I.draw[offset:], out[offset:], position, count)
    torch.cuda.synchronize()
    got = out.cpu().numpy()
    want = orc.attention_f64(I.q[offset:offset + count], I.k, I.v, I.raw[offset:offset + count], position,
                             partition=part)
    _check(got[offset:offset + count], want)
    assert np.all(np.isnan(got[:offset])) and np.all(np.isnan(got[offset + count:]))


@pytest.mark.parametrize("count", [1, 5, 100])
@pytest.mark.parametrize("partition", [32, 128, 256, 1024, 2048, 4096, 8192])
def test_attention_partitions(device, inputs, partition, count):
    """Explicit rounding partitions (gpu_prefill.mm:486-489 allows 1024..32768; any multiple
    of 32 here): one decode token (the decode kernel's own rounding at 32, the scores pass
    up to 4096, the general kernel above), short and multi-tile chunks."""
    I = inputs
    position = 5000 - count
    out = torch.zeros((count, 4096), device="cuda")
    dh.attention(device, I.dq, I.dk, I.dv, I.draw, out, position, count, partition=partition)
    torch.cuda.synchronize()
    want = orc.attention_f64(I.q[:count], I.k, I.v, I.raw[:count], position, partition=partition)
    _check(out.cpu().numpy(), want)


@pytest.mark.parametrize("position,count,partition", [(9000, 64, 0), (20000, 1, 0), (6000, 16, 0), (4000, 1, 2048),
                                                      (3000, 100, 128), (3000, 100, 32)])
def test_attention_rounding_points(device, position, count, partition):
    """Inputs on which the rounding points show: queries scaled so that a few keys dominate
    each row and values around 1 (outputs O(1)). Moving where probabilities are rounded
    (another partition) moves 40-77 % of the outputs, a relative L2 change of 3.3e-5 to
    1.1e-4 against the reference's double oracle; the library must stay within 1e-5 of the
    oracle at its own partition (the default: 1024). Single outputs may differ by up to
    1.5e-4 here: with few dominant keys, one probability whose fp32 exponential lands on
    the other side of a bf16 rounding midpoint than the double one moves an output by
    p * 2^-8 / sum(p), which the reference's 3e-5 bound (on its diffuse inputs) never meets.
    (3000, 100, 128) and (3000, 100, 32) have several rounding partitions inside one
    block's keys."""
    n = position + count
    (q,), s = orc.xorshift_values(0x5eed1024, count * 4096)
    (k, v), s = orc.xorshift_values(s, n * 512, 2)
    (r,), s = orc.xorshift_values(s, count * 8192)
    q = (50.0 * q).reshape(count, 4096).astype(np.float32)
    kb = orc.f32_to_bf16_bits(k).reshape(n, 512)
    vb = orc.f32_to_bf16_bits((1.0 + v).astype(np.float32)).reshape(n, 512)
    raw = (r * 5).reshape(count, 8192)
    out = torch.zeros((count, 4096), device="cuda")
    dh.attention(device, torch.from_numpy(q).cuda(), torch.from_numpy(kb.view(np.int16)).cuda(),
                 torch.from_numpy(vb.view(np.int16)).cuda(), torch.from_numpy(raw).cuda(), out, position, count,
                 partition=partition)
    torch.cuda.synchronize()
    part = dh.attention_partition(position, count, partition)
    kf, vf = orc.bf16_bits_to_f32(kb), orc.bf16_bits_to_f32(vb)
    want = orc.attention_f64(q, kf, vf, raw, position, partition=part)
    got = out.cpu().numpy().astype(np.float64)

    def rel(a):
        return float(np.sqrt(np.sum((a - want) ** 2) / np.sum(want ** 2)))
    assert np.all(np.isfinite(got))
    assert float(np.max(np.abs(got - want))) <= 1.5e-4
    assert rel(got) <= 1e-5, rel(got)
    for other in {32, part // 2, 2 * part} - {part, 16}:
        alt = orc.attention_f64(q, kf, vf, raw, position, partition=other)
        assert rel(alt) > 3e-5, other


@pytest.mark.parametrize("count,partition", [(100, 128), (100, 0), (1, 0)])
def test_attention_partition_far_below_the_maximum(device, count, partition):
    """Rounding partitions whose maximum lies about 60 (natural units; ~87 in log2) below an
    earlier one's: KV head 0's queries all point along one vector and keys 10..13 along it
    with scores of 60, so that for heads 0-7 every later partition's probabilities are
    below 2^-64 of the running scale (the path that scales them down by an exact power of
    two instead of scaling the accumulators up). Outputs must stay finite and match."""
    position = 3000 - count
    n = position + count
    (q,), s = orc.xorshift_values(0x5eed60, count * 4096)
    (k, v), s = orc.xorshift_values(s, n * 512, 2)
    (r,), s = orc.xorshift_values(s, count * 8192)
    q = q.reshape(count, 16, 256).astype(np.float32)   # heads 8-15: diffuse attention
    qv = orc.round_bf16(50.0 * q[0, 0]).astype(np.float64)
    q[:, :8] = qv.astype(np.float32)
    q = q.reshape(count, 4096)
    k = k.reshape(n, 512)
    k[10:14, :256] = (qv * (60.0 * 16 / float(qv @ qv))).astype(np.float32)
    kb = orc.f32_to_bf16_bits(k.astype(np.float32))
    vb = orc.f32_to_bf16_bits((1.0 + v).astype(np.float32)).reshape(n, 512)
    raw = (r * 5).reshape(count, 8192)
    out = torch.zeros((count, 4096), device="cuda")
    dh.attention(device, torch.from_numpy(q).cuda(), torch.from_numpy(kb.view(np.int16)).cuda(),
                 torch.from_numpy(vb.view(np.int16)).cuda(), torch.from_numpy(raw).cuda(), out, position, count,
                 partition=partition)
    torch.cuda.synchronize()
    kf, vf = orc.bf16_bits_to_f32(kb), orc.bf16_bits_to_f32(vb)
    want = orc.attention_f64(q, kf, vf, raw, position, partition=dh.attention_partition(position, count, partition))
    _check(out.cpu().numpy(), want)


def test_attention_bf16_operands(device, inputs):
    """bf16 queries and gate in, bf16 out: the same math on bf16-valued inputs, output
    within one bf16 rounding of the f32 result."""
    I = inputs
    position, count = 700, 40
    qb = orc.round_bf16(I.q[:count])
    rb = orc.round_bf16(I.raw[:count])
    out = torch.zeros((count, 4096), dtype=torch.int16, device="cuda")
    dh.attention(device, _bf16_dev(qb), I.dk, I.dv, _bf16_dev(rb), out, position, count,
                 q_dtype=dh.BF16, gate_dtype=dh.BF16, out_dtype=dh.BF16)
    torch.cuda.synchronize()
    got = orc.bf16_bits_to_f32(out.cpu().numpy().view(np.uint16)).astype(np.float64)
    want = orc.attention_f64(qb, I.k, I.v, rb, position, partition=dh.attention_partition(position, count))
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + ABS_TOL)


@pytest.mark.parametrize("position", [0, 31, 32, 96, 127, 128, 129, 255, 1000, 8191])
def test_attention_decode_positions(device, inputs, position):
    """One decode token (the decode kernels: 128-key blocks of four 32-key tiles, after the
    scores pass for the default 1024-key rounding) at block and tile edges, where some of a
    block's tiles have no keys, and with cache rows past the position set to NaN (they must
    not be read into the result)."""
    I = inputs
    k = I.dk.clone()
    v = I.dv.clone()
    k[position + 1:] = 0x7fc0   # bf16 NaN
    v[position + 1:] = 0x7fc0
    for partition in (0, 32):
        out = torch.full((1, 4096), float("nan"), device="cuda")
        dh.attention(device, I.dq, k, v, I.draw, out, position, 1, partition=partition)
        torch.cuda.synchronize()
        want = orc.attention_f64(I.q[:1], I.k, I.v, I.raw[:1], position, partition=partition or 1024)
        _check(out.cpu().numpy(), want)


@pytest.mark.parametrize("position", [32767, 32768, 40000])
def test_attention_decode_long(device, position):
    """One decode token past 32K keys: 256, 257 and 313 block partials per head, the last
    two more than the wide combine loads in one round (its looped path)."""
    I = Inputs(1, position + 1)
    for partition in (0, 32):
        out = torch.full((1, 4096), float("nan"), device="cuda")
        dh.attention(device, I.dq, I.dk, I.dv, I.draw, out, position, 1, partition=partition)
        torch.cuda.synchronize()
        want = orc.attention_f64(I.q[:1], I.k, I.v, I.raw[:1], position, partition=partition or 1024)
        _check(out.cpu().numpy(), want)


def test_attention_decode_bf16(device, inputs):
    """The decode kernel with bf16 queries, gate and output."""
    I = inputs
    position = 3000
    qb = orc.round_bf16(I.q[:1])
    rb = orc.round_bf16(I.raw[:1])
    out = torch.zeros((1, 4096), dtype=torch.int16, device="cuda")
    dh.attention(device, _bf16_dev(qb), I.dk, I.dv, _bf16_dev(rb), out, position, 1,
                 q_dtype=dh.BF16, gate_dtype=dh.BF16, out_dtype=dh.BF16)
    torch.cuda.synchronize()
    got = orc.bf16_bits_to_f32(out.cpu().numpy().view(np.uint16)).astype(np.float64)
    want = orc.attention_f64(qb, I.k, I.v, rb, position, partition=1024)
    assert np.all(np.abs(got - want) <= 2.0 ** -8 * np.abs(want) + ABS_TOL)


def test_attention_matches_exact_softmax(device, inputs):
    """Against the plain double softmax of unrounded operands: the bf16 rounding of q and
    of the probabilities stays within a few bf16 ulps of the values' scale."""
    I = inputs
    position, count = 300, 24
    out = torch.zeros((count, 4096), device="cuda")
    dh.attention(device, I.dq, I.dk, I.dv, I.draw, out, position, count)
    torch.cuda.synchronize()
    exact = orc.attention_f64(I.q[:count], I.k, I.v, I.raw[:count], position, bf16_operands=False)
    assert np.max(np.abs(out.cpu().numpy() - exact)) < 1e-3


def test_attention_ignores_rows_past_the_chunk(device, inputs):
    """Cache rows after position+tokens-1 (not yet written in a real cache) never reach
    the output: NaN there changes nothing."""
    I = inputs
    position, count = 900, 50
    k = I.dk.clone()
    v = I.dv.clone()
    k[position + count:] = 0x7fc0   # bf16 NaN
    v[position + count:] = 0x7fc0
    a = torch.zeros((count, 4096), device="cuda")
    b = torch.zeros((count, 4096), device="cuda")
    dh.attention(device, I.dq, I.dk, I.dv, I.draw, a, position, count)
    dh.attention(device, I.dq, k, v, I.draw, b, position, count)
    torch.cuda.synchronize()
    assert torch.equal(a, b) and bool(torch.isfinite(a).all())


@pytest.mark.parametrize("end", [2048, 32768, 131072, 262144])
def test_attention_long_analytic(device, end):
    """bf16_attention_long_checks.mm: zero queries and gates, values 1 (KV head 0) and -2
    (KV head 1) -> .5 for heads 0-7 and -1 for heads 8-15, through the last cache row."""
    cap = 262144
    keys = torch.zeros((cap, 512), dtype=torch.int16, device="cuda")
    vals = torch.empty((cap, 512), dtype=torch.int16, device="cuda")
    vals[:, :256] = 0x3f80
    vals[:, 256:] = -16384          # 0xc000 = -2.0
    q = torch.zeros((128, 4096), device="cuda")
    raw = torch.zeros((128, 8192), device="cuda")
    out = torch.zeros((128, 4096), device="cuda")
    expected = np.concatenate([np.full(2048, .5), np.full(2048, -1.0)])
    for count in (1, 3, 128):
        out.zero_()
        dh.attention(device, q, keys, vals, raw, out, end - count, count)
        torch.cuda.synchronize()
        got = out[:count].cpu().numpy()
        assert np.all(np.abs(got - expected[None, :]) <= 3e-5), (end, count, np.max(np.abs(got - expected)))


@pytest.mark.parametrize("base", [0, 1022, 4097])
def test_attention_chunk_composition(device, base):
    """attention_batch_checks.mm: 128-query calls over a chunk equal one call over it
    (same partition), and nothing outside the chunk is written."""
    storage, offset, count, partition = 2064, 7, 1024, 1024
    I = Inputs(storage, 8192, seed=0x71f23c5)
    small = torch.full((storage, 4096), float("nan"), device="cuda")
    large = torch.full((storage, 4096), float("nan"), device="cuda")
    for start in range(0, count, 128):
        n = min(128, count - start)
        o = offset + start
        dh.attention(device, I.dq[o:], I.dk, I.dv, I.draw[o:], small[o:], base + start, n, partition=partition)
    dh.attention(device, I.dq[offset:], I.dk, I.dv, I.draw[offset:], large[offset:], base, count,
                 partition=partition)
    torch.cuda.synchronize()
    a = small.cpu().numpy()
    b = large.cpu().numpy()
    assert np.all(np.isnan(b[:offset])) and np.all(np.isnan(b[offset + count:]))
    assert np.all(np.isnan(a[:offset])) and np.all(np.isnan(a[offset + count:]))
    _check(a[offset:offset + count], b[offset:offset + count].astype(np.float64))


def test_attention_arguments_are_validated(device, inputs):
    I = inputs
    out = torch.full((4, 4096), 7.0, device="cuda")
    bad = [dict(position=-1, tokens=4), dict(position=0, tokens=0), dict(position=8190, tokens=4),
           dict(position=0, tokens=4, partition=100), dict(position=0, tokens=4, partition=-32),
           dict(position=0, tokens=4, q_dtype=2)]
    for kw in bad:
        with pytest.raises(dh.ArgumentError, match="Invalid attention arguments"):
            dh.attention(device, I.dq, I.dk, I.dv, I.draw, out, **kw)
    with pytest.raises(dh.ArgumentError):
        dh.attention(device, None, I.dk, I.dv, I.draw, out, 0, 4)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all())
