"""GPU parity at the full size of every benchmark configuration, against the fp64 oracle.

Integer work (top-8 ids, route grouping, argmax) is bit-exact. Matmul outputs satisfy
max|gpu - oracle| / RMS(oracle) <= TOL (1e-2) against the fp64 oracle of the reference's
dequantize-then-matmul on the same packed inputs (tighter bounds where the arithmetic
allows, noted per test). Inputs follow the configurations: x ~ N(0,1) in bf16, codes
U{0..2^bits-1}, scale ~ U(5e-4, 2e-3) in bf16, bias = -2^(bits-1) scale + N(0, 1e-4).

  1  qmv 8-bit [4096 x 2048], M = 1, bf16 out
  2  decode MoE step, 8-bit, 256 experts top-8, hidden 2048, intermediate 512, shared
     expert + sigmoid gate (router GEMV, and N(0,1) router logits supplied)
  3  prefill MoE, 512 tokens, 8-bit, Zipf(1.1) expert popularity
  4  prefill MoE, 2048 tokens, 5-bit, uniform routing
  5  dense 8-bit at 4096 tokens: q/gate 8192x2048, k and v 512x2048, o 2048x4096,
     DeltaNet in_proj 12288x2048
  5b lm_head [248320 x 2048] 8-bit in 4 vocab slices of 62,080 rows, fp32 logits, argmax

Plus the reference's own grouped-expert check (prefill_expert_checks.mm:22-59): 256
experts of closed-form 129 x 256 weights, route counts 64..2048 under three route
patterns, gate/up and down, |gpu - double| <= 2e-6 with bf16-rounded operands.
"""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc
from tests import refcases

pytestmark = pytest.mark.gpu
TOL = 1e-2
H, E, I = 2048, 256, 512


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


def rms(a) -> float:
    a = np.asarray(a, dtype=np.float64)
    return float(np.sqrt(np.mean(a * a)))


def beyond_bf16_rounding(got, exact, scale) -> float:
    """max(|got - exact| - 2^-8 |exact|) / scale: a bf16 result within `x` of TOL*scale of
    the fp64 answer, after one round-to-nearest-even step, gives x <= TOL."""
    got = np.asarray(got, dtype=np.float64)
    exact = np.asarray(exact, dtype=np.float64)
    return float(np.max(np.abs(got - exact) - np.abs(exact) * 2.0 ** -8)) / scale


def moe_layer(rng, bits, router):
    mk = lambda e, r, c: orc.random_matrix(rng, e, r, c, bits)  # noqa: E731
    rt = orc.random_matrix(rng, 1, E, H, 8, scale_lo=1.25e-4, scale_hi=5e-4) if router else None
    return orc.MoeLayer(rt, mk(E, I, H), mk(E, I, H), mk(E, H, I), mk(1, I, H), mk(1, I, H), mk(1, H, I),
                        orc.random_matrix(rng, 1, 1, H, 8))


def upload_layer(device, L):
    mats = [L.router, L.gate, L.up, L.down, L.shared_gate, L.shared_up, L.shared_down, L.shared_route]
    q = [None if m is None else upload(device, m) for m in mats]
    return q, dh.make_layer(*q)


def dispose(mats):
    for m in mats:
        if m is not None:
            m.dispose()


# ------------------------------------------------------------------------- config 1

@pytest.mark.parametrize("y_dtype", [dh.F32, dh.BF16])
def test_config1_qmv(device, y_dtype):
    """The config-1 GEMV (seed 0): the f32 result is the fp32-accumulated dot product
    (1e-5), the bf16 output within one RNE step of it."""
    rng = np.random.default_rng(0)
    host = orc.random_matrix(rng, 1, 4096, 2048, 8)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=2048).astype(np.float32))
        y = torch.zeros(4096, dtype=torch.float32 if y_dtype == dh.F32 else torch.int16, device="cuda")
        dh.qmv(device, m, dev_bf16(xb), y, y_dtype=y_dtype)
        torch.cuda.synchronize()
        want = orc.qmv_f64(host, orc.bf16_bits_to_f32(xb))
        if y_dtype == dh.F32:
            err = orc.rel_err(y.cpu().numpy(), want)
            assert err < 1e-5, err
        else:
            assert beyond_bf16_rounding(host_bf16(y), want, rms(want)) <= 1e-5
    finally:
        m.dispose()


# ------------------------------------------------------------------------- config 2

@pytest.mark.parametrize("supplied_logits", [False, True])
def test_config2_decode_moe_step(device, supplied_logits):
    """One decode token through the full config-2 layer. With the router, its fp32 logits
    match fp64 to 1e-5 and routing is bit-exact on the logits the GPU used; with supplied
    N(0,1) bf16 logits, routing is bit-exact on those. The nine down projections (eight
    slots + shared) are fp32 GEMVs (1e-4), the residual one bf16 rounding of the answer."""
    rng = np.random.default_rng(2)
    L = moe_layer(rng, 8, router=not supplied_logits)
    q, layer = upload_layer(device, L)
    try:
        for step in range(2):
            xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
            rb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
            res = dev_bf16(rb)
            lg = torch.zeros(E, dtype=torch.float32, device="cuda")
            ids = torch.zeros(8, dtype=torch.int32, device="cuda")
            probs = torch.zeros(8, dtype=torch.float32, device="cuda")
            rout = torch.zeros((9, H), dtype=torch.float32, device="cuda")
            trace = dh.make_trace(logits=lg, ids=ids, probs=probs, expert_out=rout)
            xf = orc.bf16_bits_to_f32(xb)
            if supplied_logits:
                lf = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(rng.normal(size=E).astype(np.float32)))
                dh.moe_decode(device, layer, dev_bf16(xb), res, logits=torch.from_numpy(lf).cuda(), trace=trace)
            else:
                dh.moe_decode(device, layer, dev_bf16(xb), res, trace=trace)
            torch.cuda.synchronize()
            if supplied_logits:
                used = lf
            else:
                used = lg.cpu().numpy()
                assert orc.rel_err(used, orc.qmv_f64(L.router, xf)) < 1e-5
            oid, opr = orc.top8(used)
            assert np.array_equal(ids.cpu().numpy(), oid)
            assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
            y, ro = orc.moe_f64(L, xf[None, :], oid[None, :], opr[None, :], bf16_operands=False, route_out=True)
            err = orc.rel_err(rout.cpu().numpy(), ro)
            assert err < 1e-4, err
            exact = orc.bf16_bits_to_f32(rb).astype(np.float64) + y[0]
            assert beyond_bf16_rounding(host_bf16(res), exact, rms(y)) <= TOL
    finally:
        dispose(q)


# --------------------------------------------------------------------- configs 3, 4

def zipf_logits(rng, T, s=1.1):
    """log p_e + Gumbel with p ~ rank^-s over a random expert order: top-8 of these is
    Zipf(s) sampling without replacement (config 3)."""
    p = np.arange(1, E + 1, dtype=np.float64) ** -s
    p /= p.sum()
    perm = rng.permutation(E)
    return (np.log(p)[perm][None, :] + rng.gumbel(size=(T, E))).astype(np.float32)


def run_prefill(device, T, bits, routing, seed, unrounded_tokens):
    rng = np.random.default_rng(seed)
    L = moe_layer(rng, bits, router=False)
    q, layer = upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        lg = zipf_logits(rng, T) if routing == "zipf" else rng.normal(size=(T, E)).astype(np.float32)
        lb = orc.f32_to_bf16_bits(lg)
        rb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        res = dev_bf16(rb)
        ids = torch.zeros((T, 8), dtype=torch.int32, device="cuda")
        probs = torch.zeros((T, 8), dtype=torch.float32, device="cuda")
        rout = torch.zeros((T * 9, H), dtype=torch.float32, device="cuda")
        dh.moe_prefill(device, layer, T, dev_bf16(xb), dev_bf16(lb), res,
                       trace=dh.make_trace(ids=ids, probs=probs, expert_out=rout))
        # the route grouping of the same ids, through the stand-alone entry point
        counts = torch.zeros(E, dtype=torch.int32, device="cuda")
        routes = torch.zeros(E * T, dtype=torch.int32, device="cuda")
        dh.build_groups(device, ids, T, E, counts, routes)
        torch.cuda.synchronize()
        # routing and grouping: bit-exact
        oid, opr = orc.top8_bf16(lb)
        got_ids = ids.cpu().numpy()
        assert np.array_equal(got_ids, oid)
        assert np.max(np.abs(probs.cpu().numpy() - opr)) <= 1e-6
        oc, orr = orc.build_groups(oid, T, E)
        gc = counts.cpu().numpy().view(np.uint32)
        gr = routes.cpu().numpy().view(np.uint32)
        assert np.array_equal(gc, oc)
        for e in np.nonzero(oc)[0]:
            assert np.array_equal(gr[e * T:e * T + oc[e]], orr[e * T:e * T + oc[e]])
        assert int(oc.sum()) == T * 8
        # every route output (T*8 routed + T shared) against the reference's BF16 path:
        # weights, x and the SwiGLU activation rounded to bf16, fp64 sums
        xf = orc.bf16_bits_to_f32(xb)
        got_ro = rout.cpu().numpy()
        y_bf, ro_bf = orc.moe_f64(L, xf, oid, opr, bf16_operands=True, route_out=True)
        err = orc.rel_err(got_ro, ro_bf)
        assert err < TOL, err
        # the residual: bf16(residual + sigma-gated shared + probability-weighted experts)
        exact = orc.bf16_bits_to_f32(rb).astype(np.float64) + y_bf
        assert beyond_bf16_rounding(host_bf16(res), exact, rms(y_bf)) <= TOL
        # against unrounded fp64 (a leading block of tokens): the bf16 operand rounding
        # itself, which the reference's BF16 path shares
        n = unrounded_tokens
        _, ro = orc.moe_f64(L, xf[:n], oid[:n], opr[:n], bf16_operands=False, route_out=True)
        sel = np.concatenate([got_ro[:n * 8], got_ro[T * 8:T * 8 + n]])
        assert orc.rel_err(sel, ro) < 5e-2
        return oc
    finally:
        dispose(q)


def test_config3_prefill_512_tokens_8bit_zipf(device):
    counts = run_prefill(device, 512, 8, "zipf", seed=3, unrounded_tokens=128)
    # Zipf(1.1) popularity: a few hot experts, most with a handful of routes
    assert counts.max() >= 100 and np.median(counts) <= 16


def test_config4_prefill_2048_tokens_5bit_uniform(device):
    counts = run_prefill(device, 2048, 5, "uniform", seed=4, unrounded_tokens=96)
    assert (counts > 0).all() and counts.max() < 128


# ------------------------------------------------------------------------- config 5

@pytest.mark.parametrize("name,rows,cols,T", [("q_gate", 8192, 2048, 4096), ("k", 512, 2048, 4096),
                                              ("v", 512, 2048, 4096), ("o", 2048, 4096, 4096),
                                              ("in_proj", 12288, 2048, 4096), ("q_gate", 8192, 2048, 2048),
                                              ("o", 2048, 4096, 2048)])
def test_config5_dense_4096_tokens(device, name, rows, cols, T):
    """Each config-5 projection at a 4096-token chunk (and the reference's default 2048-token
    prefill chunk): within 1e-4 of the fp64 product of bf16-rounded operands (the reference's
    BF16 GEMM), within TOL of the unrounded one; the bf16 output is one RNE step from the
    f32 output's answer."""
    rng = np.random.default_rng(rows + cols)
    host = orc.random_matrix(rng, 1, rows, cols, 8)
    m = upload(device, host)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, cols)).astype(np.float32))
        x = dev_bf16(xb)
        y = torch.zeros((T, rows), dtype=torch.float32, device="cuda")
        yb = torch.zeros((T, rows), dtype=torch.int16, device="cuda")
        dh.dense(device, m, T, x, y)
        dh.dense(device, m, T, x, yb, y_dtype=dh.BF16)
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        xf = orc.bf16_bits_to_f32(xb)
        want_bf = orc.dense_f64_blas(host, xf, round_operands=True)
        e_bf = orc.rel_err(got, want_bf)
        assert e_bf < 1e-4, e_bf
        want = orc.dense_f64_blas(host, xf, round_operands=False)
        assert orc.rel_err(got, want) < TOL
        assert np.array_equal(yb.cpu().numpy().view(np.uint16), orc.f32_to_bf16_bits(got))
    finally:
        m.dispose()


# ------------------------------------------------------------------------ config 5b

def test_config5b_lm_head_four_slices_of_62080(device):
    """The full vocabulary: fp32 logits within 1e-5 of fp64; the library's argmax is the
    reference rule (largest, ties to the lowest index) applied to those logits, bit-exact,
    and it is the fp64 argmax whenever the fp64 margin exceeds the logits' error."""
    rng = np.random.default_rng(5)
    hosts = [orc.random_matrix(rng, 1, 62080, 2048, 8) for _ in range(4)]
    slices = [upload(device, h) for h in hosts]
    try:
        for _ in range(2):
            xb = orc.f32_to_bf16_bits(rng.normal(size=2048).astype(np.float32))
            logits = torch.full((248320,), float("nan"), dtype=torch.float32, device="cuda")
            nxt = torch.zeros(1, dtype=torch.int32, device="cuda")
            dh.lm_head(device, slices, dev_bf16(xb), logits, nxt)
            torch.cuda.synchronize()
            xf = orc.bf16_bits_to_f32(xb)
            want = np.concatenate([orc.qmv_f64(h, xf) for h in hosts])
            got = logits.cpu().numpy()
            assert orc.rel_err(got, want) < 1e-5
            token = int(nxt.cpu().numpy().view(np.uint32)[0])
            assert token == orc.argmax(got)
            err = float(np.max(np.abs(got - want)))
            top2 = np.sort(want)[-2:]
            if top2[1] - top2[0] > 2 * err:
                assert token == int(np.argmax(want))
    finally:
        dispose(slices)


# ------------------------------------------------- the reference's grouped closed form

def closed_form_weights(kind, rows, cols, bits):
    """value(kind, e, r, col) of prefill_expert_checks.mm:22 for every expert, rounded to
    bf16 as the BF16 path rounds weights: float64 [256, rows, cols]."""
    e = np.arange(256)[:, None, None]
    r = np.arange(rows)[None, :, None]
    c = np.arange(cols)[None, None, :]
    q = (e * 3 + r * 7 + c * 5 + kind * 11) & ((1 << bits) - 1)
    v = q * (c // 64 + 1) / 4096.0 + ((e + r + kind) % 7 - 3) / 1024.0
    return orc.round_bf16(v.astype(np.float32)).astype(np.float64)


def grouped_setup(device, bits, cols):
    rows = 129
    mats = [upload(device, refcases.prefill_matrix(kind, 256, rows, cols, bits)) for kind in range(3)]
    wts = [closed_form_weights(kind, rows, cols, bits) for kind in range(3)]
    n = 2048 * 8 * cols
    x = (np.sin(np.arange(n, dtype=np.float32) * np.float32(.021)) * np.float32(.02)).astype(np.float32)
    xb = orc.f32_to_bf16_bits(x).reshape(2048 * 8, cols)
    return mats, wts, xb, dev_bf16(xb)


@pytest.mark.parametrize("cols", [256, 512])
@pytest.mark.parametrize("bits", [5, 8])
def test_reference_grouped_expert_check(device, bits, cols):
    """prefill_expert_checks.mm:22-59 restated: router logits that select the pattern's ids
    in slot order (100 - slot, others -1000), top-8, grouping, then the grouped gate/up
    (SwiGLU) and the grouped down on their own; every route and row within 2e-6 of the
    double closed form with bf16-rounded weights and inputs. Columns 256 are the check's
    own (the register-ring kernel); 512 runs the same check through the streaming kernels."""
    rows = 129
    mats, wts, xb, xd = grouped_setup(device, bits, cols)
    try:
        _grouped_check(device, bits, cols, rows, mats, wts, xb, xd)
    finally:
        dispose(mats)


def _grouped_check(device, bits, cols, rows, mats, wts, xb, xd):
    xr = orc.bf16_bits_to_f32(xb).astype(np.float64)
    worst = 0.0
    for count in (64, 65, 127, 128, 129, 512, 513, 2048):
        for pattern in (0, 1, 2):
            want_ids = refcases.route_pattern(pattern, count)
            logits = np.full((count, 256), -1000.0, dtype=np.float32)
            for slot in range(8):
                logits[np.arange(count), want_ids[:, slot]] = 100.0 - slot
            ids = torch.zeros((count, 8), dtype=torch.int32, device="cuda")
            probs = torch.zeros((count, 8), dtype=torch.float32, device="cuda")
            dh.top8(device, torch.from_numpy(logits).cuda(), count, 256, ids, probs, logits_dtype=dh.F32)
            counts = torch.zeros(256, dtype=torch.int32, device="cuda")
            routes = torch.zeros(256 * count, dtype=torch.int32, device="cuda")
            dh.build_groups(device, ids, count, 256, counts, routes)
            for down in (False, True):
                y = torch.full((count * 8, rows), float("nan"), device="cuda")
                if down:
                    dh.grouped_qmm(device, mats[2], count, xd, counts, routes, y, input_mode=0)
                else:
                    dh.grouped_qmm(device, mats[0], count, xd, counts, routes, y, up=mats[1], input_mode=1)
                torch.cuda.synchronize()
                assert np.array_equal(ids.cpu().numpy().view(np.uint32), want_ids)
                gc = counts.cpu().numpy().view(np.uint32)
                gr = routes.cpu().numpy().view(np.uint32)
                seen = np.zeros(count * 8, dtype=bool)
                flat = want_ids.reshape(-1)
                for e in range(256):
                    lst = gr[e * count:e * count + gc[e]]
                    assert np.all(flat[lst] == e) and not seen[lst].any()
                    seen[lst] = True
                assert seen.all()
                got = y.cpu().numpy().astype(np.float64)
                want = np.empty_like(got)
                for e in np.unique(flat):
                    r = np.nonzero(flat == e)[0]
                    xin = xr[r] if down else xr[r // 8]
                    if down:
                        want[r] = xin @ wts[2][e].T
                    else:
                        a = xin @ wts[0][e].T
                        b = xin @ wts[1][e].T
                        want[r] = a / (1 + np.exp(-a)) * b
                diff = np.abs(got - want)
                assert np.all(np.isfinite(got)), (count, pattern, down)
                worst = max(worst, float(diff.max()))
                assert diff.max() <= 2e-6, (count, pattern, down, float(diff.max()))
    print(f"grouped check {bits}-bit, {cols} columns: max abs {worst:.3g}")
