"""GPU parity of dih_delta_rule (gated delta rule over a chunk) against the float64
token-by-token recurrence oracle.delta_rule_f64, following prefill_delta_checks.mm:

* inputs: unit keys sin((t*19+h*7+d)*.071), queries .02*cos((t*7+h*13+d)*.031), values
  .7*sin((t*11+h*17+d)*.013), state .01*sin(i*.003), history i*1e-4 (:10-15, :27-28);
* four decay/beta modes: smooth, exact zeros and ones, 1e-15 decays, and .9999 with one
  key repeated over all tokens (:18-25);
* token counts 1..2048 (:17), each on the library's path (sequential below 64 tokens,
  chunkwise from there) and the counts of the other path forced;
* |out - oracle| <= 1e-5, relative L2 <= 3e-5, |state - oracle| <= 2e-5, history exact
  (:39-44).
"""
import numpy as np
import pytest
import torch

import deepinfer_hip as dh
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

TOKENS = (1, 3, 31, 32, 63, 64, 65, 127, 128, 129, 256, 512, 513, 1024, 2048)
MAX_T = 2048


def _inputs(mode):
    t = np.arange(MAX_T)[:, None, None]
    d = np.arange(128)[None, None, :]
    h16 = np.arange(16)[None, :, None]
    conv = np.zeros((MAX_T, 8192), dtype=np.float32)
    kt = t if mode != 3 else 0
    k = np.sin(((kt * 19 + h16 * 7 + d) * np.float32(0.071)).astype(np.float32)).astype(np.float32)
    k = np.broadcast_to(k, (MAX_T, 16, 128))
    k = (k / np.sqrt(np.sum(k.astype(np.float64) ** 2, axis=2, keepdims=True))).astype(np.float32)
    conv[:, 2048:4096] = k.reshape(MAX_T, 2048)
    q = np.cos(((t * 7 + h16 * 13 + d) * np.float32(0.031)).astype(np.float32)) * np.float32(0.02)
    conv[:, :2048] = q.reshape(MAX_T, 2048)
    h32 = np.arange(32)[None, :, None]
    v = np.sin(((t * 11 + h32 * 17 + d) * np.float32(0.013)).astype(np.float32)) * np.float32(0.7)
    conv[:, 4096:] = v.reshape(MAX_T, 4096)
    th = np.arange(MAX_T)[:, None] + np.arange(32)[None, :]
    if mode == 0:
        a = 0.9 + (th % 10) * 0.009
        b = 0.3 + (th % 7) * 0.09
    elif mode == 1:
        a = np.where(th % 17 == 0, 0.0, np.where(th % 13 == 0, 1.0, 0.7))
        b = np.where(th % 11 == 0, 0.0, 1.0)
    elif mode == 2:
        a = np.where(th % 7 == 0, 1e-15, 0.999)
        b = 0.3 + (th % 7) * 0.09
    else:
        a = np.full(th.shape, 0.9999)
        b = np.full(th.shape, 0.9999)
    state = (np.sin(np.arange(32 * 128 * 128) * np.float32(0.003)) * np.float32(0.01)).astype(np.float32)
    return conv, a.astype(np.float32), b.astype(np.float32), state.reshape(32, 128, 128)


_CACHE = {}


def _oracle(mode):
    """Outputs for MAX_T tokens and the state after each count in TOKENS (one run)."""
    if mode not in _CACHE:
        conv, a, b, state = _inputs(mode)
        outs, states, S, done = [], {}, state, 0
        for T in TOKENS:
            o, S = orc.delta_rule_f64(S, conv[done:T], a[done:T], b[done:T], T - done)
            outs.append(o)
            states[T] = S
            done = T
        _CACHE[mode] = (conv, a, b, state, np.concatenate(outs), states)
    return _CACHE[mode]


def _run(device, mode, T, path, state_in=None):
    conv, a, b, state, _, _ = _oracle(mode)
    raw = np.sin(np.arange(MAX_T * 8192, dtype=np.float32)[: T * 8192] * np.float32(0.007)).reshape(T, 8192)
    hist = (np.arange(3 * 8192) * np.float32(1e-4)).astype(np.float32).reshape(3, 8192)
    d_state = torch.from_numpy(np.ascontiguousarray(state if state_in is None else state_in)).cuda()
    d_hist = torch.from_numpy(hist).cuda()
    out = torch.full((T, 4096), float("nan"), device="cuda")
    dh.delta_rule(device, d_state, d_hist, torch.from_numpy(conv[:T]).cuda(), torch.from_numpy(a[:T]).cuda(),
                  torch.from_numpy(b[:T]).cuda(), torch.from_numpy(raw).cuda(), out, T, path=path)
    torch.cuda.synchronize()
    return out.cpu().numpy(), d_state.cpu().numpy(), d_hist.cpu().numpy(), hist, raw


def _check(got_out, got_state, want_out, want_state):
    diff = np.abs(got_out - want_out)
    assert np.all(np.isfinite(got_out)) and np.max(diff) <= 1e-5, np.max(diff)
    rel = np.sqrt(np.sum(diff ** 2) / max(np.sum(want_out ** 2), 1e-30))
    assert rel <= 3e-5, rel
    sd = np.abs(got_state - want_state)
    assert np.all(np.isfinite(got_state)) and np.max(sd) <= 2e-5, np.max(sd)


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
@pytest.mark.parametrize("T", TOKENS)
def test_delta_rule_against_recurrence(device, mode, T):
    """The library's own path choice (sequential below 64 tokens, chunkwise from there)."""
    _, _, _, _, outs, states = _oracle(mode)
    got_out, got_state, got_hist, hist, raw = _run(device, mode, T, 0)
    _check(got_out, got_state, outs[:T], states[T])
    assert np.array_equal(got_hist, orc.delta_history(hist, raw, T))


@pytest.mark.parametrize("mode,T,path", [(0, 1, 2), (1, 3, 2), (2, 31, 2), (1, 32, 2), (3, 63, 2), (0, 64, 1),
                                         (3, 65, 1), (2, 127, 1), (2, 128, 1), (3, 129, 1), (1, 256, 1),
                                         (0, 513, 1)])
def test_delta_rule_other_path(device, mode, T, path):
    """The path the library would not pick for this count: chunkwise for short chunks
    (partial first block), sequential for long ones."""
    _, _, _, _, outs, states = _oracle(mode)
    got_out, got_state, _, _, _ = _run(device, mode, T, path)
    _check(got_out, got_state, outs[:T], states[T])


def test_delta_rule_carries_state(device):
    """Two chunkwise calls of 100 and 65 tokens equal the recurrence over 165."""
    conv, a, b, state, _, _ = _oracle(0)
    want_out, want_state = orc.delta_rule_f64(state, conv, a, b, 165)
    d_state = torch.from_numpy(np.ascontiguousarray(state)).cuda()
    d_hist = torch.zeros((3, 8192), device="cuda")
    out = torch.zeros((165, 4096), device="cuda")
    raw = torch.zeros((165, 8192), device="cuda")
    dc, da, db = (torch.from_numpy(x[:165]).cuda() for x in (conv, a, b))
    dh.delta_rule(device, d_state, d_hist, dc, da, db, raw, out, 100)
    dh.delta_rule(device, d_state, d_hist, dc[100:], da[100:], db[100:], raw[100:], out[100:], 65)
    torch.cuda.synchronize()
    _check(out.cpu().numpy(), d_state.cpu().numpy(), want_out, want_state)


def test_delta_rule_arguments_are_validated(device):
    s = torch.ones((32, 128, 128), device="cuda")
    h = torch.ones((3, 8192), device="cuda")
    c = torch.zeros((4, 8192), device="cuda")
    ab = torch.zeros((4, 32), device="cuda")
    out = torch.full((4, 4096), 7.0, device="cuda")
    for kw in (dict(tokens=0), dict(tokens=4, path=3), dict(tokens=4, path=-1)):
        with pytest.raises(dh.ArgumentError, match="Invalid delta rule arguments"):
            dh.delta_rule(device, s, h, c, ab, ab, c, out, **kw)
    with pytest.raises(dh.ArgumentError):
        dh.delta_rule(device, s, None, c, ab, ab, c, out, 4)
    torch.cuda.synchronize()
    assert bool((out == 7.0).all()) and bool((s == 1.0).all()) and bool((h == 1.0).all())


@pytest.mark.parametrize("mode", [0, 1, 2, 3])
def test_delta_memory_steps_match_recurrence(device, mode):
    """DeltaMemory (di_delta_create / di_delta_step, quantized.mm:398-423): a zeroed state
    stepped one token at a time from host arrays equals the recurrence from a zero state,
    at the same bar as the chunk path."""
    conv, a, b, _, _, _ = _oracle(mode)
    T = 40
    want_out, want_state = orc.delta_rule_f64(np.zeros((32, 128, 128)), conv, a, b, T)
    mem = device.new_delta_memory()
    try:
        got = np.zeros((T, 4096), dtype=np.float32)
        for t in range(T):
            out = np.full(4096, np.nan, dtype=np.float32)
            mem.step(conv[t, :2048], conv[t, 2048:4096], conv[t, 4096:], a[t], b[t], out)
            got[t] = out
        diff = np.abs(got - want_out)
        assert np.all(np.isfinite(got)) and np.max(diff) <= 1e-5, np.max(diff)
        rel = np.sqrt(np.sum(diff ** 2) / max(np.sum(want_out ** 2), 1e-30))
        assert rel <= 3e-5, rel
    finally:
        mem.dispose()


def test_delta_memory_validation(device):
    """DeltaMemory.Step's dimension check (QuantizedMetal.cs:216-217) and the native null
    check (quantized.mm:410) reject before any GPU work; a second memory is independent."""
    mem = device.new_delta_memory()
    other = device.new_delta_memory()
    try:
        z = np.zeros
        with pytest.raises(dh.ArgumentError, match="Unsupported gated-delta dimensions"):
            mem.step(z(2048), z(2048), z(4095), z(32), z(32), z(4096))
        err = dh._errbuf()
        ms = __import__("ctypes").c_double()
        arr = np.zeros(4096, dtype=np.float32)
        rc = device._lib.dih_delta_step(device.context, mem.handle, None, arr.ctypes.data, arr.ctypes.data,
                                        arr.ctypes.data, arr.ctypes.data, arr.ctypes.data, None, err, dh._ERR)
        assert rc == -1 and dh._msg(err) == "Null delta argument"
        # one step on `mem` with decay 1, beta 1, a unit key and value 1 leaves S = v k^T there
        k = np.zeros(2048, dtype=np.float32)
        k[0] = 1.0
        q = k.copy()
        v = np.ones(4096, dtype=np.float32)
        out = np.zeros(4096, dtype=np.float32)
        mem.step(q, k, v, np.ones(32), np.ones(32), out)
        assert np.allclose(out[:128], 1.0) and np.allclose(out[2 * 128:3 * 128], 0.0)   # head 2 -> key head 1
        out2 = np.zeros(4096, dtype=np.float32)
        other.step(q, k, np.zeros(4096), np.ones(32), np.ones(32), out2)
        assert np.all(out2 == 0.0)
    finally:
        mem.dispose()
        other.dispose()
