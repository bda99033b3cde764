"""GPU tests of the MoE residual update and fused next-layer norm (graph_merge_norm,
gpu_graph.mm:48-61; prefill_merge, gpu_prefill.mm:140-150) against oracle.merge_norm_f64:
f32 residual storage like the reference, or bf16; normed output f32 or bf16."""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc
from tests.test_gpu_hotpath import (TOL, _moe_layer, _upload_layer, _zipf_logits, assert_rounded, dev_bf16,
                                    host_bf16, rms)

pytestmark = pytest.mark.gpu


def _residual(vals, f32):
    v = np.asarray(vals, dtype=np.float32)
    return torch.from_numpy(v).cuda() if f32 else dev_bf16(orc.f32_to_bf16_bits(v))


def _host(t, f32):
    return t.cpu().numpy().astype(np.float64) if f32 else host_bf16(t).astype(np.float64)


def _check(res, normed, r0, y, w, eps, res_f32, normed_f32):
    got_r = _host(res, res_f32)
    want_r, _ = orc.merge_norm_f64(r0, y, residual_bf16=not res_f32)
    if res_f32:
        # f32 sum of the fp32 step output: the step's own error (a few 1e-4 of the update)
        # plus one f32 rounding of the sum
        assert np.max(np.abs(got_r - want_r)) <= 1e-3 * rms(y) + 2.0 ** -23 * np.max(np.abs(want_r)), \
            np.max(np.abs(got_r - want_r))
    else:
        assert_rounded(got_r, np.asarray(r0, np.float64) + y, rms(y))
    # the norm of the residual the GPU stored (isolates the norm from the step's rounding)
    _, want_n = orc.merge_norm_f64(got_r, np.zeros_like(got_r), w, eps, residual_bf16=False)
    got_n = _host(normed, normed_f32)
    if normed_f32:
        assert orc.rel_err(got_n, want_n) < 1e-5
    else:
        assert_rounded(got_n, want_n, 0.0)


@pytest.mark.parametrize("res_f32,normed_f32", [(True, True), (False, False), (True, False)])
@pytest.mark.parametrize("bits,E,H,I", [(8, 256, 2048, 512), (5, 256, 2048, 512),
                                        (8, 16, 1024, 1536)])   # I > 1024: the GEMV-stage path
def test_decode_merge_norm(device, bits, E, H, I, res_f32, normed_f32):
    rng = np.random.default_rng(40 + bits + I)
    L = _moe_layer(rng, E, H, I, bits)
    q, layer = _upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        r0 = rng.normal(size=H).astype(np.float32)
        if not res_f32:
            r0 = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(r0))
        w = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
        eps = 1e-6
        res = _residual(r0, res_f32)
        normed = torch.zeros(H, dtype=torch.float32 if normed_f32 else torch.int16, device="cuda")
        wt = torch.from_numpy(w).cuda()
        ids = torch.zeros(8, dtype=torch.int32, device="cuda")
        probs = torch.zeros(8, dtype=torch.float32, device="cuda")
        dh.moe_decode(device, layer, dev_bf16(xb), res, trace=dh.make_trace(ids=ids, probs=probs),
                      merge=dh.make_merge(res_f32, wt, eps, normed, normed_f32))
        torch.cuda.synchronize()
        xf = orc.bf16_bits_to_f32(xb)
        y = orc.moe_f64(L, xf[None, :], ids.cpu().numpy()[None, :], probs.cpu().numpy()[None, :],
                        bf16_operands=False)
        _check(res, normed, r0[None, :], y, w, eps, res_f32, normed_f32)
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("res_f32,normed_f32", [(True, True), (False, False)])
def test_prefill_merge_norm(device, res_f32, normed_f32):
    rng = np.random.default_rng(77)
    T, E, H, I, bits = 96, 256, 2048, 512, 8
    L = _moe_layer(rng, E, H, I, bits, router=False)
    q, layer = _upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        lb = orc.f32_to_bf16_bits(_zipf_logits(rng, T, E))
        r0 = rng.normal(size=(T, H)).astype(np.float32)
        if not res_f32:
            r0 = orc.bf16_bits_to_f32(orc.f32_to_bf16_bits(r0))
        w = rng.uniform(0.5, 1.5, size=H).astype(np.float32)
        eps = 1e-5
        res = _residual(r0, res_f32)
        normed = torch.zeros((T, H), dtype=torch.float32 if normed_f32 else torch.int16, device="cuda")
        rout = torch.zeros((T * 9, H), dtype=torch.float32, device="cuda")
        dh.moe_prefill(device, layer, T, dev_bf16(xb), dev_bf16(lb), res, trace=dh.make_trace(expert_out=rout),
                       merge=dh.make_merge(res_f32, torch.from_numpy(w).cuda(), eps, normed, normed_f32))
        torch.cuda.synchronize()
        oid, opr = orc.top8_bf16(lb)
        xf = orc.bf16_bits_to_f32(xb)
        y_bf = orc.moe_f64(L, xf, oid, opr, bf16_operands=True)
        got_r = _host(res, res_f32)
        if res_f32:
            assert np.max(np.abs(got_r - (r0 + y_bf))) <= TOL * rms(y_bf)
        else:
            assert_rounded(got_r, r0.astype(np.float64) + y_bf, rms(y_bf))
        _, want_n = orc.merge_norm_f64(got_r, np.zeros_like(got_r), w, eps)
        got_n = _host(normed, normed_f32)
        if normed_f32:
            assert orc.rel_err(got_n, want_n) < 1e-5
        else:
            assert_rounded(got_n, want_n, 0.0)
    finally:
        for m in q:
            if m is not None:
                m.dispose()


def test_merge_options_are_validated(device):
    rng = np.random.default_rng(5)
    L = _moe_layer(rng, 16, 256, 64, 8)
    q, layer = _upload_layer(device, L)
    try:
        x = dev_bf16(orc.f32_to_bf16_bits(rng.normal(size=256).astype(np.float32)))
        r0 = orc.f32_to_bf16_bits(rng.normal(size=256).astype(np.float32))
        res = dev_bf16(r0)
        w = torch.ones(256, device="cuda")
        out = torch.zeros(256, device="cuda")
        bad = [dh.make_merge(False, w, 0.0, out), dh.make_merge(False, w, float("nan"), out),
               dh.make_merge(False, w, 1e-6, None), dh.make_merge(False, w, 1e-6, res)]
        m = dh.make_merge()
        m.residual_f32 = 2
        bad.append(m)
        for mg in bad:
            with pytest.raises(dh.ArgumentError, match="merge options"):
                dh.moe_decode(device, layer, x, res, merge=mg)
        torch.cuda.synchronize()
        assert np.array_equal(res.cpu().numpy().view(np.uint16), r0)   # nothing ran
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("bits,E,H,I", [(8, 256, 2048, 512), (8, 16, 1024, 1536)])   # fast and GEMV-stage paths
@pytest.mark.parametrize("noalloc", [False, True])
def test_decode_nonfinite_logit_leaves_outputs_unchanged(device, bits, E, H, I, noalloc):
    """A non-finite router logit fails the step (status 1, ids 0, probabilities NaN) and leaves
    the residual and the normed row exactly as they were: the reference's host path throws
    before writing any output (SelectExperts, Qwen36Model.cs:252)."""
    if noalloc and I > 1024:
        pytest.skip("the no-allocation entry takes the fast-path shapes only")
    rng = np.random.default_rng(90 + I)
    L = _moe_layer(rng, E, H, I, bits)
    q, layer = _upload_layer(device, L)
    layer_s = dh.make_layer(None, *q[1:])
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
        for bad in (np.nan, np.inf, -np.inf):
            lg = rng.normal(size=E).astype(np.float32)
            lg[E // 3] = bad
            r0 = orc.f32_to_bf16_bits(rng.normal(size=H).astype(np.float32))
            res = dev_bf16(r0)
            normed = torch.full((H,), 7.0, dtype=torch.float32, device="cuda")
            ids = torch.full((8,), 5, dtype=torch.int32, device="cuda")
            probs = torch.zeros(8, dtype=torch.float32, device="cuda")
            status = torch.zeros(1, dtype=torch.int32, device="cuda")
            call = dh.moe_decode_noalloc if noalloc else dh.moe_decode
            call(device, layer_s, dev_bf16(xb), res, logits=torch.from_numpy(lg).cuda(),
                 trace=dh.make_trace(ids=ids, probs=probs, status=status),
                 merge=dh.make_merge(False, torch.ones(H, device="cuda"), 1e-6, normed, True))
            torch.cuda.synchronize()
            assert int(status.item()) == 1, bad
            assert not ids.cpu().numpy().any()
            assert np.isnan(probs.cpu().numpy()).all()
            assert np.array_equal(res.cpu().numpy().view(np.uint16), r0), bad
            assert (normed.cpu().numpy() == 7.0).all(), bad
    finally:
        for m in q:
            if m is not None:
                m.dispose()


@pytest.mark.parametrize("bits,T", [(8, 40), (5, 40), (5, 120)])
def test_prefill_nonfinite_logit_leaves_its_token_unchanged(device, bits, T):
    """Prefill with non-finite router logits in two tokens: status 1; those tokens' ids 0,
    probabilities NaN, residual and normed rows bit-for-bit unchanged; every other token's
    residual and normed rows bit-for-bit what the same call gives without the bad tokens'
    logits (their routes then change only their own rows). At 120 tokens the 5-bit experts
    average 60 routes, and the shared expert runs on the side stream."""
    rng = np.random.default_rng(95 + bits)
    E, H, I = 16, 512, 256
    L = _moe_layer(rng, E, H, I, bits, router=False)
    q, layer = _upload_layer(device, L)
    try:
        xb = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        lg = rng.normal(size=(T, E)).astype(np.float32)
        r0 = orc.f32_to_bf16_bits(rng.normal(size=(T, H)).astype(np.float32))
        w = torch.from_numpy(rng.uniform(0.5, 1.5, size=H).astype(np.float32)).cuda()

        def run(logits):
            res = dev_bf16(r0)
            normed = torch.full((T, H), 3.0, dtype=torch.float32, device="cuda")
            ids = torch.full((T, 8), 9, dtype=torch.int32, device="cuda")
            probs = torch.zeros((T, 8), dtype=torch.float32, device="cuda")
            status = torch.zeros(1, dtype=torch.int32, device="cuda")
            dh.moe_prefill(device, layer, T, dev_bf16(xb), torch.from_numpy(logits).cuda(), res, logits_dtype=dh.F32,
                           trace=dh.make_trace(ids=ids, probs=probs, status=status),
                           merge=dh.make_merge(False, w, 1e-6, normed, True))
            torch.cuda.synchronize()
            return (res.cpu().numpy().view(np.uint16), normed.cpu().numpy(), ids.cpu().numpy(), probs.cpu().numpy(),
                    int(status.item()))

        clean = run(lg)
        assert clean[4] == 0
        bad_lg = lg.copy()
        bad_lg[7, 3] = np.nan
        bad_lg[30, 0] = np.inf
        res, normed, ids, probs, status = run(bad_lg)
        assert status == 1
        good = np.ones(T, dtype=bool)
        good[[7, 30]] = False
        assert not ids[~good].any() and np.isnan(probs[~good]).all()
        assert np.array_equal(res[~good], r0[~good]) and (normed[~good] == 3.0).all()
        assert np.array_equal(ids[good], clean[2][good])
        assert np.array_equal(res[good], clean[0][good]) and np.array_equal(normed[good], clean[1][good])
    finally:
        for m in q:
            if m is not None:
                m.dispose()
