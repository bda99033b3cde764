"""GPU parity tests of the device-resident hot path against the CPU oracle.

Integer work (top-8 ids, grouping, argmax, bf16 dequantization) must be bit-exact.
Matmul outputs must satisfy max|gpu - oracle| / RMS(oracle) <= TOL (1e-2, the north-star
tolerance) against the fp64 oracle of the reference's dequantize-then-matmul; tighter
bounds are asserted where the arithmetic allows (noted per test).
"""
import ctypes

import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc
from tests import refcases

pytestmark = pytest.mark.gpu
TOL = 1e-2


def upload(device, host: orc.QMatrix):
    m = device.allocate(host.experts, host.rows, host.columns, host.bits)
    m.upload(0, host.packed)
    m.upload(1, host.scales)
    m.upload(2, host.biases)
    return m


def dev_bf16(bits_u16: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits_u16, dtype=np.uint16).view(np.int16)).cuda()


def host_bf16(t: torch.Tensor) -> np.ndarray:
    return orc.bf16_bits_to_f32(t.cpu().numpy().view(np.uint16))


def u32(t: torch.Tensor) -> np.ndarray:
    return t.cpu().numpy().view(np.uint32)


def assert_rounded(got, exact, err_scale):
    """A bf16 result must equal a value within TOL*err_scale of the fp64 answer, rounded to
    bf16: |got - exact| <= 2^-8*|exact| (one round-to-nearest-even step) + TOL*err_scale."""
    got = np.asarray(got, dtype=np.float64)
    exact = np.asarray(exact, dtype=np.float64)
    bound = np.abs(exact) * 2.0 ** -8 + TOL * err_scale
    worst = np.max(np.abs(got - exact) - bound)
    assert worst <= 0, worst


def rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a)))


# ------------------------------------------------------------------------------ qmv

@pytest.mark.parametrize("bits,rows,columns", [(8, 4096, 2048), (5, 4096, 2048), (8, 300, 512),
                                               (5, 129, 4096), (8, 97, 192), (5, 64, 64),
                                               (8, 5, 2048), (8, 4097, 2048)])
def test_qmv_bf16_matches_fp64_oracle(device, bits, rows, columns):
    """Config-1 shape (8-bit [4096x2048], x bf16 ~N(0,1), bf16 out) and tails/odd widths
    (8-bit rows of 2048 columns take the one-shot kernel: 5 rows is one partial block, 4097
    leaves one row in the last block)."""
    rng = np.random.default_rng(0)
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=columns).astype(np.float32))
        x = dev_bf16(xb)
        want = orc.qmv_f64(host, orc.bf16_bits_to_f32(xb))
        y32 = torch.zeros(rows, dtype=torch.float32, device="cuda")
        yb = torch.zeros(rows, dtype=torch.int16, device="cuda")
        dh.qmv(device, m, x, y32, y_dtype=dh.F32)
        dh.qmv(device, m, x, yb, y_dtype=dh.BF16)
        torch.cuda.synchronize()
        e32 = orc.rel_err(y32.cpu().numpy(), want)
        assert e32 < TOL and e32 < 1e-5, e32          # fp32 accumulation only
        # the bf16 output is the RNE rounding of that f32 result ...
        assert np.array_equal(yb.cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y32.cpu().numpy()))
        # ... hence within one bf16 rounding step of the fp64 answer
        assert_rounded(host_bf16(yb), want, rms(want))
    finally:
        m.dispose()


@pytest.mark.parametrize("bits,x_bf16", [(8, True), (8, False), (5, True)])
def test_qmv_long_launch_matches_fp64_oracle(device, bits, x_bf16):
    """Launches of more than 16,384 row groups take the long-run kernels: 8-bit rows of 2048
    columns with bf16 x the one-shot kernel (three rows a wave; 16,391 rows leave a ragged
    last block), the others the resident single-matrix kernel."""
    rng = np.random.default_rng(9)
    rows, columns = 16391, 2048
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xf = rng.normal(size=columns).astype(np.float32)
        if x_bf16:
            xb = orc.f32_to_bf16_bits(xf)
            x, xf, xd = dev_bf16(xb), orc.bf16_bits_to_f32(xb), dh.BF16
        else:
            x, xd = torch.from_numpy(xf).cuda(), dh.F32
        want = orc.qmv_f64(host, xf)
        y32 = torch.full((rows,), float("nan"), dtype=torch.float32, device="cuda")
        yb = torch.zeros(rows, dtype=torch.int16, device="cuda")
        dh.qmv(device, m, x, y32, x_dtype=xd, y_dtype=dh.F32)
        dh.qmv(device, m, x, yb, x_dtype=xd, y_dtype=dh.BF16)
        torch.cuda.synchronize()
        e32 = orc.rel_err(y32.cpu().numpy(), want)
        assert e32 < 1e-5, e32
        assert np.array_equal(yb.cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(y32.cpu().numpy()))
    finally:
        m.dispose()


def _dynamic_range_x(rng, n, profile):
    """bf16 activations for the f16 staging checks: 'span' gives every element a random
    binade in 2^-20..2^15, so every 32-column chunk spans the whole range; 'tiny' is
    N(0,1)*2^-20 (f16 subnormals unless the chunk is scaled up); 'huge' is N(0,1)*2^30."""
    if profile == "span":
        x = rng.choice([-1.0, 1.0], size=n) * np.exp2(rng.uniform(-20, 15, size=n))
    elif profile == "tiny":
        x = rng.normal(size=n) * 2.0 ** -20
    else:
        x = rng.normal(size=n) * 2.0 ** 30
    return orc.f32_to_bf16_bits(x.astype(np.float32))


@pytest.mark.parametrize("rows", [4096, 16391])
@pytest.mark.parametrize("profile", ["span", "tiny", "huge"])
def test_qmv_f16_staging_dynamic_range(device, profile, rows):
    """The 8-bit decode GEMV stages bf16 x as f16, each 32-column chunk scaled by the power
    of two that puts its largest magnitude in [2^14, 2^15). That is exact for every value
    within 2^29 of the chunk's largest, so the result stays at fp32-accumulation accuracy
    whatever the activations' scale (config-1 shape; 16,391 rows: the one-shot long-launch
    kernel, which stages per lane in registers)."""
    rng = np.random.default_rng(11)
    host = orc.random_matrix(rng, 1, rows, 2048, 8)
    m = upload(device, host)
    try:
        xb = _dynamic_range_x(rng, 2048, profile)
        y = torch.zeros(rows, dtype=torch.float32, device="cuda")
        dh.qmv(device, m, dev_bf16(xb), y, y_dtype=dh.F32)
        torch.cuda.synchronize()
        want = orc.qmv_f64(host, orc.bf16_bits_to_f32(xb))
        got = y.cpu().numpy()
        assert np.all(np.isfinite(got))
        err = orc.rel_err(got, want)
        assert err < 1e-5, err
    finally:
        m.dispose()


def test_qmv_experts_batched_and_bad_ids(device):
    rng = np.random.default_rng(1)
    host = orc.random_matrix(rng, 9, 129, 512, 8)
    m = upload(device, host)
    try:
        ids = np.array([8, 0, 6, 2, 5, 1, 7, 3], dtype=np.uint32)
        x = rng.normal(size=8 * 512).astype(np.float32)
        y = torch.zeros(8 * 129, dtype=torch.float32, device="cuda")
        dh.qmv(device, m, torch.from_numpy(x).cuda(), y, experts=torch.from_numpy(ids.view(np.int32)).cuda(),
               count=8, batched=True, x_dtype=dh.F32)
        torch.cuda.synchronize()
        want = orc.qmv_f64(host, x, ids, batched=True)
        assert orc.rel_err(y.cpu().numpy(), want) < 1e-5
        bad = torch.tensor([3, 9], dtype=torch.int32, device="cuda")
        y2 = torch.zeros(2 * 129, dtype=torch.float32, device="cuda")
        dh.qmv(device, m, torch.from_numpy(x).cuda(), y2, experts=bad, count=2, batched=True, x_dtype=dh.F32)
        torch.cuda.synchronize()
        out = y2.cpu().numpy()
        assert np.all(np.isfinite(out[:129])) and np.all(np.isnan(out[129:]))
    finally:
        m.dispose()


def test_dequant_bf16_is_bit_exact(device):
    """expanded_weights semantics: bf16 RNE of fp32(q*scale+bias), both bit widths."""
    rng = np.random.default_rng(2)
    for bits in (5, 8):
        host = orc.random_matrix(rng, 3, 77, 320, bits)
        m = upload(device, host)
        try:
            out = torch.zeros((77, 320), dtype=torch.int16, device="cuda")
            dh.dequant_bf16(device, m, 2, out)
            torch.cuda.synchronize()
            want = orc.f32_to_bf16_bits(host.dequant()[2])
            assert np.array_equal(out.cpu().numpy().view(np.uint16), want)
        finally:
            m.dispose()


# --------------------------------------------------------------------------- routing

def test_top8_known_answers(device):
    """graph_checks.mm:63-77 cases plus the routing KAT of QuantizedTests.cs:280-288."""
    cases = refcases.top8_cases()
    logits = torch.from_numpy(np.stack(cases)).cuda()
    ids = torch.zeros((5, 8), dtype=torch.int32, device="cuda")
    probs = torch.zeros((5, 8), dtype=torch.float32, device="cuda")
    dh.top8(device, logits, 5, 256, ids, probs, logits_dtype=dh.F32)
    torch.cuda.synchronize()
    for k, v in enumerate(cases):
        exp = refcases.stable_top8(v)
        assert np.array_equal(ids.cpu().numpy()[k], exp), k
        chosen = v[exp].astype(np.float64)
        p = np.exp(chosen - chosen[0])
        p /= p.sum()
        assert np.max(np.abs(probs.cpu().numpy()[k] - p)) <= 1e-6
    assert list(ids.cpu().numpy()[1]) == list(range(255, 247, -1))
    assert abs(probs.cpu().numpy()[1].sum() - 1) <= 1e-6


def test_top8_bf16_random_with_ties_matches_oracle(device):
    rng = np.random.default_rng(3)
    T = 2048
    lg = rng.normal(size=(T, 256)).astype(np.float32)
    lg[::7, 10:40] = 2.5          # many exact ties among the top values
    lb = orc.f32_to_bf16_bits(lg)
    ids = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
    probs = torch.zeros((T, 8), dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    dh.top8(device, dev_bf16(lb), T, 256, ids, probs, status=status)
    torch.cuda.synchronize()
    oid, opr = orc.top8_bf16(lb)
    assert np.array_equal(ids.cpu().numpy(), oid)
    assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
    assert int(status.item()) == 0


def test_top8_flags_non_finite(device):
    lg = np.zeros((2, 256), dtype=np.float32)
    lg[1, 17] = np.nan
    ids = torch.zeros((2, 8), dtype=torch.int32, device="cuda")
    probs = torch.zeros((2, 8), dtype=torch.float32, device="cuda")
    status = torch.zeros(1, dtype=torch.int32, device="cuda")
    dh.top8(device, torch.from_numpy(lg).cuda(), 2, 256, ids, probs, status=status, logits_dtype=dh.F32)
    torch.cuda.synchronize()
    assert int(status.item()) == 1
    assert list(ids.cpu().numpy()[0]) == list(range(8))


@pytest.mark.parametrize("count", [1, 3, 64, 65, 127, 128, 129, 512, 513, 2048, 2049, 4100])
@pytest.mark.parametrize("pattern", [0, 1, 2])
def test_build_groups_is_bit_exact(device, count, pattern):
    """Route lists, counts and their invariants (prefill_expert_checks.mm:26-52)."""
    ids = refcases.route_pattern(pattern, count)
    counts = torch.zeros(256, dtype=torch.int32, device="cuda")
    routes = torch.zeros(256 * count, dtype=torch.int32, device="cuda")
    dh.build_groups(device, torch.from_numpy(ids.view(np.int32)).cuda(), count, 256, counts, routes)
    torch.cuda.synchronize()
    oc, orr = orc.build_groups(ids, count, 256)
    gc, gr = u32(counts), u32(routes)
    assert np.array_equal(gc, oc)
    seen = np.zeros(count * 8, dtype=bool)
    flat = ids.reshape(-1)
    for e in range(256):
        lst = gr[e * count:e * count + gc[e]]
        assert np.array_equal(lst, orr[e * count:e * count + oc[e]])
        assert np.all(np.diff(lst.astype(np.int64)) > 0)
        assert np.all(flat[lst] == e)
        assert not seen[lst].any()
        seen[lst] = True
    assert seen.all()


# --------------------------------------------------------------------------- lm_head

def _lm_slices(device, rng, rows_per_slice, columns, n=4):
    hosts = [orc.random_matrix(rng, 1, rows_per_slice, columns, 8) for _ in range(n)]
    return hosts, [upload(device, h) for h in hosts]


def test_lm_head_split_logits_and_argmax(device):
    rng = np.random.default_rng(4)
    hosts, slices = _lm_slices(device, rng, 6208, 2048)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=2048).astype(np.float32))
        logits = torch.zeros(4 * 6208, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        dh.lm_head(device, slices, dev_bf16(xb), logits, nxt)
        torch.cuda.synchronize()
        xf = orc.bf16_bits_to_f32(xb)
        want = np.concatenate([orc.qmv_f64(h, xf) for h in hosts])
        got = logits.cpu().numpy()
        assert orc.rel_err(got, want) < 1e-5
        assert int(u32(nxt)[0]) == orc.argmax(got)
    finally:
        for s in slices:
            s.dispose()


@pytest.mark.parametrize("columns", [2048, 1024])   # the one-shot GEMV, and the general one
def test_lm_head_argmax_ties_and_nonfinite(device, columns):
    """The lm_head's token (graph_argmax_blocks/final, gpu_graph.mm:160-175): exact ties
    between logits in different slices and blocks go to the lowest vocabulary index, and a
    non-finite logit makes the token invalid (0xffffffff, ModelTests.cs:23-28)."""
    rng = np.random.default_rng(8)
    rows = 5000
    hosts = [orc.random_matrix(rng, 1, rows, columns, 8) for _ in range(4)]
    # one row with large codes and scales, copied to slice 3 row 4321, slice 1 row 17 and
    # slice 1 row 4999 (the largest logits, exactly equal): the answer is 1 * rows + 17
    wpr = columns // 4
    gpr = columns // 64
    hot_p = np.full(wpr, 0xFFFFFFFF, dtype=np.uint32)
    hot_s = np.full(gpr, orc.f32_to_bf16_bits(np.float32(0.5)), dtype=np.uint16)
    hot_b = np.zeros(gpr, dtype=np.uint16)
    for k, r in ((3, 4321), (1, 17), (1, 4999)):
        hosts[k].packed.reshape(rows, wpr)[r] = hot_p
        hosts[k].scales.reshape(rows, gpr)[r] = hot_s
        hosts[k].biases.reshape(rows, gpr)[r] = hot_b
    slices = [upload(device, h) for h in hosts]
    try:
        xb = orc.f32_to_bf16_bits(np.abs(rng.normal(size=columns)).astype(np.float32) + 0.5)
        logits = torch.zeros(4 * rows, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        dh.lm_head(device, slices, dev_bf16(xb), logits, nxt)
        torch.cuda.synchronize()
        got = logits.cpu().numpy()
        assert got[rows + 17] == got[rows + 4999] == got[3 * rows + 4321] == got.max()
        assert int(u32(nxt)[0]) == rows + 17 == orc.argmax(got)
        # a non-finite activation: every logit NaN, the token invalid
        xn = xb.copy()
        xn[5] = orc.f32_to_bf16_bits(np.array([np.inf], dtype=np.float32))[0]
        dh.lm_head(device, slices, dev_bf16(xn), logits, nxt)
        torch.cuda.synchronize()
        assert int(u32(nxt)[0]) == 0xFFFFFFFF
        # the next call starts clean (the invalid mark does not carry over)
        dh.lm_head(device, slices, dev_bf16(xb), logits, nxt)
        torch.cuda.synchronize()
        assert int(u32(nxt)[0]) == rows + 17
    finally:
        for m in slices:
            m.dispose()


@pytest.mark.parametrize("columns", [2048, 1024])
def test_lm_head_argmax_all_negative_logits(device, columns):
    """Every logit negative (biases of -8 against a positive activation): the token is
    still the largest logit, lowest index first; two calls in a row agree."""
    rng = np.random.default_rng(9)
    rows = 3001
    hosts = [orc.random_matrix(rng, 1, rows, columns, 8) for _ in range(3)]
    for h in hosts:
        h.biases[:] = orc.f32_to_bf16_bits(np.float32(-8.0))
    slices = [upload(device, h) for h in hosts]
    try:
        xb = orc.f32_to_bf16_bits(np.abs(rng.normal(size=columns)).astype(np.float32) + 0.5)
        logits = torch.zeros(3 * rows, dtype=torch.float32, device="cuda")
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        for _ in range(2):
            dh.lm_head(device, slices, dev_bf16(xb), logits, nxt)
            torch.cuda.synchronize()
            got = logits.cpu().numpy()
            assert got.max() < 0
            assert int(u32(nxt)[0]) == orc.argmax(got)
    finally:
        for m in slices:
            m.dispose()


def test_argmax_known_answers(device):
    """graph_checks.mm:89-103 and ModelTests.cs:23-28."""
    n = 248320
    base = (np.arange(n, dtype=np.float32) * np.float32(1e-5)).astype(np.float32)
    cases = []
    cases.append((base.copy(), 248319))
    t = base.copy(); t[100] = t[200] = 10; cases.append((t, 100))
    t = base.copy(); t[0] = np.nan; cases.append((t, 0xFFFFFFFF))
    t = base.copy(); t[5000] = np.inf; cases.append((t, 0xFFFFFFFF))
    cases.append((np.array([1, 3, 3], dtype=np.float32), 1))
    t = np.full(5000, -7, dtype=np.float32); t[1023] = t[1024] = t[4999] = -1; cases.append((t, 1023))
    for v, want in cases:
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        dh.argmax(device, torch.from_numpy(v).cuda(), v.size, nxt)
        torch.cuda.synchronize()
        assert int(u32(nxt)[0]) == want
        assert orc.argmax(v) == want


def test_argmax_block_edges(device):
    """Ties across the 1024-value first-level blocks (and at 4096-value boundaries), a
    maximum in a partial last block, and values that start off 16-byte alignment (the scalar
    load path)."""
    cases = []
    t = np.full(3073, -3, dtype=np.float32); t[1023] = t[1024] = t[2048] = 2; cases.append((t, 1023, 0))
    t = np.full(3073, -3, dtype=np.float32); t[3072] = 5; cases.append((t, 3072, 0))
    t = np.full(3000, -3, dtype=np.float32); t[2047] = 9; t[5] = np.inf; cases.append((t, 0xFFFFFFFF, 0))
    t = np.full(12289, -3, dtype=np.float32); t[4095] = t[4096] = 2; cases.append((t, 4095, 0))
    t = np.full(12289, -3, dtype=np.float32); t[12288] = 5; cases.append((t, 12288, 0))
    t = np.full(12289, -3, dtype=np.float32); t[8191] = t[8192] = t[12000] = 4; cases.append((t, 8191, 0))
    t = np.full(8193, -3, dtype=np.float32); t[7] = 1; t[4100] = 1; cases.append((t, 7, 1))
    t = np.full(8193, -3, dtype=np.float32); t[8000] = np.nan; cases.append((t, 0xFFFFFFFF, 3))
    for v, want, shift in cases:
        buf = torch.full((v.size + shift,), 99.0, device="cuda")
        buf[shift:] = torch.from_numpy(v).cuda()
        nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
        dh.argmax(device, buf[shift:], v.size, nxt)
        torch.cuda.synchronize()
        assert int(u32(nxt)[0]) == want, (v.size, shift)
        assert orc.argmax(v) == want


# ------------------------------------------------------------------------------- MoE

def _moe_layer(rng, E, H, I, bits, router=True):
    mk = lambda e, r, c, b=bits: orc.random_matrix(rng, e, r, c, b)  # noqa: E731
    rt = orc.random_matrix(rng, 1, E, H, 8, scale_lo=1.25e-4, scale_hi=5e-4) if router else None
    return orc.MoeLayer(rt, mk(E, I, H), mk(E, I, H), mk(E, H, I), mk(1, I, H), mk(1, I, H), mk(1, H, I),
                        orc.random_matrix(rng, 1, 1, H, 8))


def _upload_layer(device, L):
    mats = [L.router, L.gate, L.up, L.down, L.shared_gate, L.shared_up, L.shared_down, L.shared_route]
    q = [None if m is None else upload(device, m) for m in mats]
    return q, dh.make_layer(*q)


@pytest.mark.parametrize("bits", [8, 5])
def test_moe_decode_step_matches_oracle(device, bits):
    """Decode MoE step (config 2 shapes with 8-bit; 5-bit experts with 8-bit router)."""
    rng = np.random.default_rng(5)
    E, H, I = 256, 2048, 512
    L = _moe_layer(rng, E, H, I, bits)
    q, layer = _upload_layer(device, L)
    try:
        for step in range(3):
            xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
            rb = orc.f32_to_bf16_bits((rng.normal(size=H) * (0 if step == 0 else 1)).astype(np.float32))
            res = dev_bf16(rb)
            lg = torch.zeros(E, dtype=torch.float32, device="cuda")
            ids = torch.zeros(8, dtype=torch.int32, device="cuda")
            probs = torch.zeros(8, dtype=torch.float32, device="cuda")
            status = torch.zeros(1, dtype=torch.int32, device="cuda")
            rout = torch.zeros((9, H), dtype=torch.float32, device="cuda")
            dh.moe_decode(device, layer, dev_bf16(xb), res,
                          trace=dh.make_trace(logits=lg, ids=ids, probs=probs, status=status, expert_out=rout))
            torch.cuda.synchronize()
            xf = orc.bf16_bits_to_f32(xb)
            # router logits: fp32 GEMV vs fp64
            want_lg = orc.qmv_f64(L.router, xf)
            got_lg = lg.cpu().numpy()
            assert orc.rel_err(got_lg, want_lg) < 1e-5
            # routing decided on the GPU's logits must be bit-exact with the oracle's rule
            oid, opr = orc.top8(got_lg)
            assert np.array_equal(ids.cpu().numpy(), oid)
            assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
            y, ro = orc.moe_f64(L, xf[None, :], oid[None, :], opr[None, :], bf16_operands=False, route_out=True)
            # matmul outputs (8 slot down projections + shared down): fp32 GEMVs vs fp64
            err = orc.rel_err(rout.cpu().numpy(), ro)
            assert err < TOL and err < 1e-4, err
            # residual = bf16(residual + y)
            assert_rounded(host_bf16(res), orc.bf16_bits_to_f32(rb) + y[0], rms(y))
            assert int(status.item()) == 0
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("profile", ["span", "tiny", "huge"])
def test_moe_decode_f16_staging_dynamic_range(device, profile):
    """The decode step's router and expert gate/up stage x as f16 per 32-column chunk (with
    a power-of-two scale per chunk): logits, routing and outputs keep their accuracy for
    activations spread over 2^-20..2^15 in every chunk, or entirely near 2^-20 or 2^30."""
    rng = np.random.default_rng(12)
    E, H, I = 256, 2048, 512
    L = _moe_layer(rng, E, H, I, 8)
    q, layer = _upload_layer(device, L)
    try:
        xb = _dynamic_range_x(rng, H, profile)
        res = dev_bf16(np.zeros(H, dtype=np.uint16))
        lg = torch.zeros(E, dtype=torch.float32, device="cuda")
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        probs = torch.zeros(8, dtype=torch.float32, device="cuda")
        rout = torch.zeros((9, H), dtype=torch.float32, device="cuda")
        dh.moe_decode(device, layer, dev_bf16(xb), res,
                      trace=dh.make_trace(logits=lg, ids=ids, probs=probs, expert_out=rout))
        torch.cuda.synchronize()
        xf = orc.bf16_bits_to_f32(xb)
        got_lg = lg.cpu().numpy()
        assert orc.rel_err(got_lg, orc.qmv_f64(L.router, xf)) < 1e-5
        oid, opr = orc.top8(got_lg)
        assert np.array_equal(ids.cpu().numpy(), oid)
        _, ro = orc.moe_f64(L, xf[None, :], oid[None, :], opr[None, :], bf16_operands=False, route_out=True)
        got = rout.cpu().numpy()
        assert np.all(np.isfinite(got))
        err = orc.rel_err(got, ro)
        assert err < 1e-4, err
    finally:
        for m in q:
            if m is not None:
                m.dispose()


def test_moe_decode_with_supplied_logits(device):
    rng = np.random.default_rng(6)
    E, H, I = 64, 512, 256
    L = _moe_layer(rng, E, H, I, 8, router=False)
    q, layer = _upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        lg = rng.normal(size=E).astype(np.float32)
        res = torch.zeros(H, dtype=torch.int16, device="cuda")
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        dh.moe_decode(device, layer, dev_bf16(xb), res, logits=torch.from_numpy(lg).cuda(),
                      trace=dh.make_trace(ids=ids))
        torch.cuda.synchronize()
        oid, opr = orc.top8(lg)
        assert np.array_equal(ids.cpu().numpy(), oid)
        y = orc.moe_f64(L, orc.bf16_bits_to_f32(xb)[None, :], oid[None, :], opr[None, :], bf16_operands=False)[0]
        assert_rounded(host_bf16(res), y, rms(y))
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("E", [8, 37, 200, 256])
def test_moe_decode_routing_ties_and_expert_counts(device, E):
    """Decode routing for expert counts that fill the router blocks partly, with heavy exact
    ties (and -0 against +0) in supplied logits, against the reference rule (largest, ties
    to the lowest index); a router computed on the GPU for the same counts; and a NaN
    logit, which fails the step with status 1 (Qwen36Model.cs:252)."""
    rng = np.random.default_rng(40 + E)
    H, I = 512, 256
    L = _moe_layer(rng, E, H, I, 8)
    q, layer = _upload_layer(device, L)
    layer_s = dh.make_layer(None, *q[1:])  # the same weights, logits supplied
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        for trial in range(3):
            lg = rng.choice(np.array([-1.5, -0.0, 0.0, 0.25, 2.0], dtype=np.float32), size=E)
            if trial == 2:
                lg[:] = 0.0
                lg[1::2] = -0.0
            ids = torch.zeros(8, dtype=torch.int32, device="cuda")
            probs = torch.zeros(8, dtype=torch.float32, device="cuda")
            status = torch.zeros(1, dtype=torch.int32, device="cuda")
            res = torch.zeros(H, dtype=torch.int16, device="cuda")
            dh.moe_decode(device, layer_s, dev_bf16(xb), res, logits=torch.from_numpy(lg).cuda(),
                          trace=dh.make_trace(ids=ids, probs=probs, status=status))
            torch.cuda.synchronize()
            oid, opr = orc.top8(lg)
            assert np.array_equal(ids.cpu().numpy(), oid), (trial, ids.cpu().numpy(), oid)
            assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
            assert int(status.item()) == 0
        # the router on the GPU
        lgt = torch.zeros(E, dtype=torch.float32, device="cuda")
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        dh.moe_decode(device, layer, dev_bf16(xb), torch.zeros(H, dtype=torch.int16, device="cuda"),
                      trace=dh.make_trace(logits=lgt, ids=ids))
        torch.cuda.synchronize()
        got_lg = lgt.cpu().numpy()
        assert orc.rel_err(got_lg, orc.qmv_f64(L.router, orc.bf16_bits_to_f32(xb))) < 1e-5
        assert np.array_equal(ids.cpu().numpy(), orc.top8(got_lg)[0])
        # a NaN logit: status 1, ids 0, and the residual unchanged
        lg = rng.normal(size=E).astype(np.float32)
        lg[E // 2] = np.nan
        ids = torch.full((8,), 7, dtype=torch.int32, device="cuda")
        status = torch.zeros(1, dtype=torch.int32, device="cuda")
        r0 = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        res = dev_bf16(r0)
        dh.moe_decode(device, layer_s, dev_bf16(xb), res,
                      logits=torch.from_numpy(lg).cuda(), trace=dh.make_trace(ids=ids, status=status))
        torch.cuda.synchronize()
        assert int(status.item()) == 1
        assert not ids.cpu().numpy().any()
        assert np.array_equal(res.cpu().numpy().view(np.uint16), r0)
    finally:
        for m in q:
            if m is not None:
                m.dispose()


def _zipf_logits(rng, T, E, s=1.1):
    """Router logits log p_e + Gumbel with p ~ rank^-s: top-8 = Zipf sampling without
    replacement (config 3)."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = rng.permutation(E)
    g = rng.gumbel(size=(T, E))
    return (np.log(p)[perm][None, :] + g).astype(np.float32)


@pytest.mark.parametrize("T,E,H,I,bits,routing", [
    (64, 32, 256, 128, 8, "zipf"), (65, 32, 256, 128, 5, "uniform"), (200, 256, 512, 128, 8, "zipf"),
    (129, 16, 128, 192, 5, "uniform"), (1, 16, 128, 64, 8, "uniform"),
    (96, 64, 1024, 512, 5, "zipf"),    # 5-bit with K multiples of 512: the streaming kernels
    (96, 64, 1024, 512, 8, "zipf"),    # 8-bit streaming gate/up at K=1024 and down at K=512
    (320, 64, 512, 512, 5, "uniform"), (300, 64, 512, 512, 8, "zipf"),
    (100, 16, 512, 192, 5, "uniform"),  # 5-bit gate/up of 192 rows: expert codes padded to 256
    (120, 16, 512, 256, 5, "zipf"),      # 5-bit split gated, 96-route chunks, popular experts split
    (100, 16, 512, 512, 5, "zipf"),      # 5-bit down in 96-route tiles (experts average 50 routes)
    (200, 16, 512, 256, 5, "uniform")])  # 5-bit split gated in 128-route chunks (experts average 100)
def test_moe_prefill_matches_oracle(device, T, E, H, I, bits, routing):
    rng = np.random.default_rng(T * 7 + E)
    L = _moe_layer(rng, E, H, I, bits, router=False)
    q, layer = _upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        lg = _zipf_logits(rng, T, E) if routing == "zipf" else rng.normal(size=(T, E)).astype(np.float32)
        lb = orc.f32_to_bf16_bits(lg)
        rb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        res = dev_bf16(rb)
        ids = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
        probs = torch.zeros((T, 8), dtype=torch.float32, device="cuda")
        rout = torch.zeros((T * 9, H), dtype=torch.float32, device="cuda")
        dh.moe_prefill(device, layer, T, dev_bf16(xb), dev_bf16(lb), res,
                       trace=dh.make_trace(ids=ids, probs=probs, expert_out=rout))
        torch.cuda.synchronize()
        oid, opr = orc.top8_bf16(lb)
        assert np.array_equal(ids.cpu().numpy(), oid)
        assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
        xf = orc.bf16_bits_to_f32(xb)
        got_ro = rout.cpu().numpy()
        # Per-route down outputs against the fp64 oracle of the reference's BF16 prefill
        # path: dequantized weights, x and the SwiGLU activation rounded to bf16 (RNE) as
        # packed_expert_load / expanded_pack do and as prefill_expert_checks.mm:56 models.
        # (The GPU rounds its fp32 SwiGLU value to bf16, the oracle its fp64 value, so an
        # activation can land one bf16 step apart; that moves outputs by ~1e-3 of RMS.)
        y_bf, ro_bf = orc.moe_f64(L, xf, oid, opr, bf16_operands=True, route_out=True)
        e_bf = orc.rel_err(got_ro, ro_bf)
        assert e_bf < TOL, e_bf
        # Against unrounded fp64 the difference is the bf16 operand rounding itself (a few
        # 2^-9 relative steps at the extremes), the same for the reference's BF16 path.
        _, ro = orc.moe_f64(L, xf, oid, opr, bf16_operands=False, route_out=True)
        assert orc.rel_err(got_ro, ro) < 5e-2
        # residual = bf16(residual + sigmoid-gated shared + probability-weighted experts)
        assert_rounded(host_bf16(res), orc.bf16_bits_to_f32(rb).astype(np.float64) + y_bf, rms(y_bf))
    finally:
        for m in q:
            if m is not None:
                m.dispose()


def test_moe_prefill_side_stream_graph_replays(device):
    """Wide 5-bit routing runs the shared expert's launches on the library's side stream
    (fork and join through events). Captured in a HIP graph with that fork, every replay,
    with eager work between them, must give the eager call's residual bit for bit."""
    T, E, H, I = 200, 16, 512, 256
    rng = np.random.default_rng(31)
    L = _moe_layer(rng, E, H, I, 5, router=False)
    q, layer = _upload_layer(device, L)
    try:
        x = dev_bf16(orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32)))
        lg = dev_bf16(orc.f32_to_bf16_bits(rng.normal(size=(T, E)).astype(np.float32)))
        r0 = dev_bf16(orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32)))
        want = r0.clone()
        dh.moe_prefill(device, layer, T, x, lg, want)
        torch.cuda.synchronize()
        res = r0.clone()
        other = r0.clone()
        g = torch.cuda.CUDAGraph()
        stream = torch.cuda.Stream()
        stream.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(stream):
            with torch.cuda.graph(g, stream=stream):
                dh.moe_prefill(device, layer, T, x, lg, res)
        torch.cuda.synchronize()
        for _ in range(3):
            res.copy_(r0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            assert torch.equal(res, want)
            dh.moe_prefill(device, layer, T, x, lg, other)   # eager work between replays
            torch.cuda.synchronize()
        del g
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("bits,rows,columns,T", [(8, 512, 2048, 256), (5, 300, 512, 130), (8, 129, 256, 65),
                                                 (8, 2048, 4096, 64), (8, 1000, 2048, 1), (5, 300, 512, 3),
                                                 (8, 129, 4096, 4), (8, 1003, 2048, 3)])
def test_dense_matches_oracle(device, bits, rows, columns, T):
    """Up to four tokens the projection runs as a batched fp32 GEMV (the reference's short-
    chunk kernels, gpu_prefill.mm:615-619, do not round operands); longer chunks use bf16
    MFMA operands as the reference's BF16 GEMM does."""
    rng = np.random.default_rng(rows + T)
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, columns)).astype(np.float32))
        y = torch.zeros((T, rows), dtype=torch.float32, device="cuda")
        dh.dense(device, m, T, dev_bf16(xb), y)
        torch.cuda.synchronize()
        xf = orc.bf16_bits_to_f32(xb)
        want = orc.dense_f64(host, xf, round_operands=False)
        if T <= 4:
            assert orc.rel_err(y.cpu().numpy(), want) < 1e-5
        else:
            want_bf = orc.dense_f64(host, xf, round_operands=True)
            assert orc.rel_err(y.cpu().numpy(), want_bf) < 1e-4
            assert orc.rel_err(y.cpu().numpy(), want) < TOL
    finally:
        m.dispose()


@pytest.mark.parametrize("bits,rows,columns,T,y_bf16", [(8, 300, 512, 1024, False), (8, 2048, 4096, 512, True),
                                                        (5, 1000, 2048, 1100, False), (5, 64, 256, 2048, True),
                                                        (8, 4100, 1024, 512, False)])
def test_dense_long_chunks_bf16_gemm(device, bits, rows, columns, T, y_bf16):
    """Long chunks (1024 tokens and more, or 512 and more for matrices of up to 4096 rows)
    run as one dequantization pass into bf16 and a bf16 GEMM with f32 accumulation (the
    reference's BF16 dense path, prefill_bf16.mm:7-53): the result is the fp64 product of
    the same bf16-rounded operands within fp32 accumulation error. (8, 4100, 1024, 512)
    stays on the fused tile (more than 4096 rows at 512 tokens)."""
    rng = np.random.default_rng(rows * 7 + T)
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, columns)).astype(np.float32))
        y = torch.zeros((T, rows), dtype=torch.int16 if y_bf16 else torch.float32, device="cuda")
        dh.dense(device, m, T, dev_bf16(xb), y, y_dtype=dh.BF16 if y_bf16 else dh.F32)
        # a second call (the scratch copy already sized) gives the same bits
        y2 = torch.zeros_like(y)
        dh.dense(device, m, T, dev_bf16(xb), y2, y_dtype=dh.BF16 if y_bf16 else dh.F32)
        torch.cuda.synchronize()
        assert torch.equal(y, y2)
        xf = orc.bf16_bits_to_f32(xb)
        want_bf = orc.dense_f64(host, xf, round_operands=True)
        if y_bf16:
            assert_rounded(host_bf16(y), want_bf, rms(want_bf) * 1e-2)
        else:
            assert orc.rel_err(y.cpu().numpy(), want_bf) < 1e-4
    finally:
        m.dispose()


@pytest.mark.parametrize("bits,rows,columns,T,y_bf16", [
    (8, 8200, 2048, 4100, True),    # 256 x 256 tiles; ragged last row and token tiles
    (8, 2050, 4096, 4100, False),   # 256 x 128 tiles; f32 rows not 16-byte aligned (element stores)
    (5, 1000, 1024, 4096, True)])   # 128 x 128 tiles, 5-bit dequantization
def test_dense_gemm_tile_shapes(device, bits, rows, columns, T, y_bf16):
    """Every block shape of the library's bf16 GEMM (gemm_bf16_kernel, chosen by the tile
    count) against the fp64 product of the same bf16-rounded operands, with partial tiles at
    both edges."""
    rng = np.random.default_rng(rows + T)
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, columns)).astype(np.float32))
        y = torch.zeros((T, rows), dtype=torch.int16 if y_bf16 else torch.float32, device="cuda")
        dh.dense(device, m, T, dev_bf16(xb), y, y_dtype=dh.BF16 if y_bf16 else dh.F32)
        torch.cuda.synchronize()
        want = orc.dense_f64_blas(host, orc.bf16_bits_to_f32(xb), round_operands=True)
        if y_bf16:
            assert_rounded(host_bf16(y), want, rms(want) * 1e-2)
        else:
            assert orc.rel_err(y.cpu().numpy(), want) < 1e-4
    finally:
        m.dispose()


@pytest.mark.parametrize("bits,rows,columns,T", [(8, 16384, 512, 512), (5, 16400, 512, 520)])
def test_dense_two_slab_tiles(device, bits, rows, columns, T):
    """Dense launches with at least 256 (256-row tile, 128-token chunk) items run 256-row
    tiles, two 32-row slabs a wave; ragged rows and tokens included."""
    rng = np.random.default_rng(rows + T)
    host = orc.random_matrix(rng, 1, rows, columns, bits)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, columns)).astype(np.float32))
        y = torch.zeros((T, rows), dtype=torch.float32, device="cuda")
        dh.dense(device, m, T, dev_bf16(xb), y)
        torch.cuda.synchronize()
        want_bf = orc.dense_f64(host, orc.bf16_bits_to_f32(xb), round_operands=True)
        assert orc.rel_err(y.cpu().numpy(), want_bf) < 1e-4
    finally:
        m.dispose()


def _device_copy(dst: int, src: int, n: int) -> None:
    """hipMemcpy through the HIP runtime torch has already loaded (same soname)."""
    hip = ctypes.CDLL("libamdhip64.so.7")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    assert hip.hipMemcpy(dst, src, n, 4) == 0  # hipMemcpyDefault


@pytest.mark.parametrize("path", ["chunks", "staging", "device_ptr", "device_ptr_uncommitted"])
def test_5bit_tile_major_copy_follows_every_write_path(device, path):
    """5-bit matrices with K a multiple of 512 feed the streaming GEMM from a tile-major copy
    of their codes, which every write path must keep equal to the row-major codes: direct
    writes in ragged chunks that start and end inside rows, the host staging buffer, and the
    device pointer followed by dih_quant_matrix_commit, and the device pointer asked for once
    and written twice without a commit. 200 rows (the copy pads to 256).
    Rows rewritten after a multiply must reach the next multiply."""
    L = dh.load()
    rng = np.random.default_rng(5)
    rows, columns, T = 200, 512, 130
    first = orc.random_matrix(rng, 1, rows, columns, 5)
    second = orc.random_matrix(rng, 1, rows, columns, 5)
    # the rewrite: rows 37..149 of `second`, the others kept from `first`
    words = columns * 5 // 32
    mixed = first.packed.copy().reshape(rows, words)
    mixed[37:150] = second.packed.reshape(rows, words)[37:150]
    want_host = orc.QMatrix(mixed, first.scales, first.biases, 1, rows, columns, 5)
    m = device.allocate(1, rows, columns, 5)
    held = []

    def put(packed: np.ndarray, lo: int, hi: int) -> None:
        raw = np.ascontiguousarray(packed).view(np.uint8).reshape(-1)
        if path == "chunks":
            cuts = sorted({lo, hi, lo + (hi - lo) // 3 + 7, lo + 2 * (hi - lo) // 3 - 5})
            for a, b in zip(cuts[:-1], cuts[1:]):
                m.upload(0, raw[a:b], offset=a)
        elif path == "staging":
            m.write(0, raw)
        else:
            t = torch.from_numpy(raw[lo:hi].copy()).cuda()
            torch.cuda.synchronize()
            if path == "device_ptr":
                _device_copy(m.device_ptr(0) + lo, t.data_ptr(), hi - lo)
                err = ctypes.create_string_buffer(256)
                assert L.dih_quant_matrix_commit(m.handle, err, 256) == 0, err.value
            else:
                # the pointer asked for once and kept, no commit: every call rewrites the copy
                if not held:
                    held.append(m.device_ptr(0))
                _device_copy(held[0] + lo, t.data_ptr(), hi - lo)

    try:
        row_bytes = words * 4
        put(first.packed, 0, rows * row_bytes)
        m.upload(1, first.scales)
        m.upload(2, first.biases)
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, columns)).astype(np.float32))
        xf = orc.bf16_bits_to_f32(xb)
        for host in (first, want_host):
            if host is want_host:
                put(mixed, 37 * row_bytes, 150 * row_bytes)
            y = torch.zeros((T, rows), dtype=torch.float32, device="cuda")
            dh.dense(device, m, T, dev_bf16(xb), y)
            torch.cuda.synchronize()
            want_bf = orc.dense_f64(host, xf, round_operands=True)
            assert orc.rel_err(y.cpu().numpy(), want_bf) < 1e-4
    finally:
        m.dispose()


def test_bf16_dense_check_cases(device):
    """bf16_checks.mm:12-35: closed-form weights, amplitudes .2 and 1e10, relative L2 < 2e-5
    against bf16-rounded double products."""
    cols = 256
    for rows in (32, 129):
        for bits in (5, 8):
            r = np.arange(rows)[:, None]
            g = np.arange(4)[None, :]
            scale = orc.round_bf16((np.float32(.00017) * (1 + (r + g) % 13)).astype(np.float32))
            bias = orc.round_bf16((np.float32(-.0271) * (1 + (r + g) % 3)).astype(np.float32))
            c = np.arange(cols)[None, :]
            q = ((r * 37 + c * 19 + 7) & ((1 << bits) - 1)).astype(np.uint32)
            host = orc.QMatrix(orc.pack_codes(q[None], bits), orc.f32_to_bf16_bits(scale),
                               orc.f32_to_bf16_bits(bias), 1, rows, cols, bits)
            m = upload(device, host)
            try:
                for n in (64, 65, 128, 2048):
                    for amp in (.2, 1e10):
                        i = np.arange(n * cols)
                        x = (np.sin(i * np.float32(.019)).astype(np.float32) * np.float32(amp)).reshape(n, cols)
                        xb = orc.f32_to_bf16_bits(x)
                        y = torch.zeros((n, rows), dtype=torch.float32, device="cuda")
                        dh.dense(device, m, n, dev_bf16(xb), y)
                        torch.cuda.synchronize()
                        want = orc.dense_f64(host, orc.bf16_bits_to_f32(xb), round_operands=True)
                        got = y.cpu().numpy().astype(np.float64)
                        rel = np.sqrt(((got - want) ** 2).sum() / max((want ** 2).sum(), 1e-30))
                        assert rel < 2e-5, (rows, bits, n, amp, rel)
            finally:
                m.dispose()
