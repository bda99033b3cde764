"""Python side of the CPU oracle (test infrastructure only).

Loads ``liboracle.so`` (built from oracle.c by ``make -C oracle``) and adds numpy helpers
that the tests use to build MLX-affine matrices. Only tests/, ``__graft_entry__.smoke()``
and bench.py's ``cpu_baseline`` leg import this module; the product never does.

Layout restated from the reference's loader and packers:
  packed uint32 [E, R, C*bits/32], code c at bit c*bits LSB-first, straddling words
  (Qwen36Weights.cs:73-76; QuantizedTests.cs:155-161), scales/biases bf16 [E, R, C/64].
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        _declare(_lib)
    return _lib


class OrcMatrix(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("biases", ctypes.c_void_p), ("experts", ctypes.c_int),
                ("rows", ctypes.c_int), ("columns", ctypes.c_int), ("bits", ctypes.c_int)]


class OrcMoeLayer(ctypes.Structure):
    _fields_ = [(n, ctypes.POINTER(OrcMatrix)) for n in
                ("router", "gate", "up", "down", "shared_gate", "shared_up",
                 "shared_down", "shared_route")]


def _declare(L):
    P = ctypes.c_void_p
    I = ctypes.c_int
    M = ctypes.POINTER(OrcMatrix)
    L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
    L.orc_bf16_to_f32.restype = ctypes.c_float
    L.orc_f32_to_bf16.argtypes = [ctypes.c_float]
    L.orc_f32_to_bf16.restype = ctypes.c_uint16
    L.orc_code.argtypes = [P, I, I]
    L.orc_code.restype = ctypes.c_uint32
    L.orc_dequant_row.argtypes = [M, I, I, P]
    L.orc_qmv_f64.argtypes = [M, P, P, I, I, P]
    L.orc_dense_f64.argtypes = [M, I, P, I, I, P]
    L.orc_top8.argtypes = [P, I, P, P]
    L.orc_top8.restype = I
    L.orc_top8_bf16.argtypes = [P, I, I, P, P]
    L.orc_top8_bf16.restype = I
    L.orc_build_groups.argtypes = [P, I, I, P, P]
    L.orc_argmax.argtypes = [P, I]
    L.orc_argmax.restype = ctypes.c_uint32
    L.orc_expert_mlp_f64.argtypes = [M, M, M, M, P, P, P, I, P, P]
    L.orc_moe_f64.argtypes = [ctypes.POINTER(OrcMoeLayer), I, P, P, P, I, P, P]
    L.orc_cpu_qmv.argtypes = [M, P, P, I, I, P, I]
    L.orc_cpu_moe_token.argtypes = [ctypes.POINTER(OrcMoeLayer), P, P, I]
    L.orc_cpu_moe_token.restype = I
    L.orc_openmp_threads.restype = I
    L.orc_xorshift_fill.argtypes = [ctypes.c_uint32, P, I, ctypes.c_size_t]
    L.orc_xorshift_fill.restype = ctypes.c_uint32


def _ptr(a: np.ndarray):
    assert a.flags.c_contiguous
    return a.ctypes.data_as(ctypes.c_void_p)


# ---------------------------------------------------------------- bf16 helpers (numpy)

def bf16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16_bits(f: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even (the rule of prefill_expert_checks.mm:24)."""
    u = np.ascontiguousarray(f, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFFFFFF
    return (u >> 16).astype(np.uint16)


def round_bf16(f: np.ndarray) -> np.ndarray:
    return bf16_bits_to_f32(f32_to_bf16_bits(f))


# ---------------------------------------------------------------- packing (numpy)

def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer codes [..., C] LSB-first at bit c*bits into uint32 words
    (the packer of QuantizedTests.cs:155-161 / prefill_expert_checks.mm:16-17)."""
    codes = np.asarray(codes, dtype=np.uint64)
    *lead, C = codes.shape
    assert (C * bits) % 32 == 0
    words = np.zeros(lead + [C * bits // 32], dtype=np.uint64)
    for c in range(C):
        bit = c * bits
        at, shift = bit // 32, bit % 32
        words[..., at] |= (codes[..., c] << shift) & 0xFFFFFFFF
        if shift + bits > 32:
            words[..., at + 1] |= codes[..., c] >> (32 - shift)
    return words.astype(np.uint32)


def unpack_codes(words: np.ndarray, bits: int, columns: int) -> np.ndarray:
    """Independent numpy unpack: treat each row as one little-endian bit string."""
    w = np.ascontiguousarray(words, dtype=np.uint32)
    *lead, nw = w.shape
    bitsarr = np.unpackbits(w.view(np.uint8).reshape(*lead, nw * 4), axis=-1, bitorder="little")
    bitsarr = bitsarr[..., : columns * bits].reshape(*lead, columns, bits).astype(np.uint32)
    return (bitsarr << np.arange(bits, dtype=np.uint32)).sum(axis=-1).astype(np.uint32)


class QMatrix:
    """A host MLX-affine matrix plus its ctypes view for the C oracle."""

    def __init__(self, packed, scales, biases, experts, rows, columns, bits):
        self.packed = np.ascontiguousarray(packed, dtype=np.uint32)
        self.scales = np.ascontiguousarray(scales, dtype=np.uint16)
        self.biases = np.ascontiguousarray(biases, dtype=np.uint16)
        self.experts, self.rows, self.columns, self.bits = experts, rows, columns, bits
        assert self.packed.size == experts * rows * columns * bits // 32
        assert self.scales.size == experts * rows * columns // 64 == self.biases.size
        self.c = OrcMatrix(self.packed.ctypes.data, self.scales.ctypes.data,
                           self.biases.ctypes.data, experts, rows, columns, bits)

    @classmethod
    def from_codes(cls, codes, scales, biases, bits):
        E, R, C = codes.shape
        return cls(pack_codes(codes, bits), scales, biases, E, R, C, bits)

    def dequant(self, round_bf=False) -> np.ndarray:
        """Dense float32 weights [E, R, C] (numpy, independent of oracle.c)."""
        codes = unpack_codes(self.packed.reshape(self.experts, self.rows, -1), self.bits, self.columns)
        s = bf16_bits_to_f32(self.scales).reshape(self.experts, self.rows, -1)
        b = bf16_bits_to_f32(self.biases).reshape(self.experts, self.rows, -1)
        s = np.repeat(s, 64, axis=-1)
        b = np.repeat(b, 64, axis=-1)
        w = (codes.astype(np.float32) * s + b).astype(np.float32)
        return round_bf16(w) if round_bf else w


def random_matrix(rng: np.random.Generator, experts, rows, columns, bits, scale_lo=5e-4,
                  scale_hi=2e-3, bias_sd=1e-4) -> QMatrix:
    """Synthetic MLX-affine weights of the benchmark configs: codes U{0..2^bits-1} (uniform
    random packed words, so every bit field is uniform), scale ~U(lo, hi) in bf16,
    bias = -2^(bits-1)*scale + N(0, bias_sd) in bf16."""
    words = rng.integers(0, 1 << 32, size=(experts, rows, columns * bits // 32), dtype=np.uint64)
    s = rng.uniform(scale_lo, scale_hi, size=(experts, rows, columns // 64)).astype(np.float32)
    sb = f32_to_bf16_bits(s)
    b = -(1 << (bits - 1)) * bf16_bits_to_f32(sb) + rng.normal(0, bias_sd, size=s.shape).astype(np.float32)
    return QMatrix(words.astype(np.uint32), sb, f32_to_bf16_bits(b.astype(np.float32)), experts, rows,
                   columns, bits)


# ---------------------------------------------------------------- oracle wrappers

def qmv_f64(m: QMatrix, x: np.ndarray, experts=None, batched=False) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    count = 1 if experts is None else len(experts)
    ids = None if experts is None else np.ascontiguousarray(experts, dtype=np.uint32)
    y = np.zeros(count * m.rows, dtype=np.float64)
    lib().orc_qmv_f64(ctypes.byref(m.c), _ptr(x), None if ids is None else _ptr(ids), count,
                      1 if batched else 0, _ptr(y))
    return y


def dense_f64(m: QMatrix, x: np.ndarray, expert=0, round_operands=True) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    T = x.shape[0]
    y = np.zeros((T, m.rows), dtype=np.float64)
    lib().orc_dense_f64(ctypes.byref(m.c), expert, _ptr(x), T, 1 if round_operands else 0, _ptr(y))
    return y


def dense_f64_blas(m: QMatrix, x: np.ndarray, expert=0, round_operands=True) -> np.ndarray:
    """The product of dense_f64 (Y[t][r] = sum_c w(e,r,c) X[t][c], prefill_bf16_product
    prefill_bf16.mm:26-37) for chunk sizes where a scalar loop is too slow: weights from the
    numpy dequantization, operands widened to float64 and multiplied by BLAS. With
    round_operands the bf16 products are exact in float64, so the result differs from
    dense_f64 only in the order of the float64 sums."""
    x = np.asarray(x, dtype=np.float32)
    one = QMatrix(m.packed.reshape(m.experts, -1)[expert], m.scales.reshape(m.experts, -1)[expert],
                  m.biases.reshape(m.experts, -1)[expert], 1, m.rows, m.columns, m.bits)
    w = one.dequant(round_bf=round_operands)[0].astype(np.float64)
    xd = (round_bf16(x) if round_operands else x).astype(np.float64)
    return xd @ w.T


def top8(logits: np.ndarray):
    logits = np.ascontiguousarray(logits, dtype=np.float32)
    ids = np.zeros(8, dtype=np.int32)
    probs = np.zeros(8, dtype=np.float32)
    rc = lib().orc_top8(_ptr(logits), logits.size, _ptr(ids), _ptr(probs))
    if rc != 0:
        raise ValueError("Non-finite router logits.")
    return ids, probs


def top8_bf16(logits_bits: np.ndarray):
    logits_bits = np.ascontiguousarray(logits_bits, dtype=np.uint16)
    T, E = logits_bits.shape
    ids = np.zeros((T, 8), dtype=np.int32)
    probs = np.zeros((T, 8), dtype=np.float32)
    bad = lib().orc_top8_bf16(_ptr(logits_bits), T, E, _ptr(ids), _ptr(probs))
    if bad >= 0:
        raise ValueError(f"Non-finite router logits at token {bad}.")
    return ids, probs


def build_groups(ids: np.ndarray, tokens: int, experts: int):
    ids = np.ascontiguousarray(ids, dtype=np.uint32).reshape(-1)
    counts = np.zeros(experts, dtype=np.uint32)
    routes = np.zeros(experts * tokens, dtype=np.uint32)
    lib().orc_build_groups(_ptr(ids), tokens, experts, _ptr(counts), _ptr(routes))
    return counts, routes


def argmax(values: np.ndarray) -> int:
    values = np.ascontiguousarray(values, dtype=np.float32)
    return int(lib().orc_argmax(_ptr(values), values.size))


def expert_mlp_f64(gate, up, down, shared, x, sx, experts):
    x = np.ascontiguousarray(x, dtype=np.float32)
    sx = np.ascontiguousarray(sx, dtype=np.float32)
    ids = np.ascontiguousarray(experts, dtype=np.uint32)
    out = np.zeros(len(ids) * down.rows, dtype=np.float64)
    sout = np.zeros(shared.rows, dtype=np.float64)
    lib().orc_expert_mlp_f64(ctypes.byref(gate.c), ctypes.byref(up.c), ctypes.byref(down.c),
                             ctypes.byref(shared.c), _ptr(x), _ptr(sx), _ptr(ids), len(ids),
                             _ptr(out), _ptr(sout))
    return out, sout


class MoeLayer:
    """Host weights of one MoE layer (Qwen36Weights.cs:93-100)."""

    def __init__(self, router, gate, up, down, shared_gate, shared_up, shared_down, shared_route):
        self.router, self.gate, self.up, self.down = router, gate, up, down
        self.shared_gate, self.shared_up = shared_gate, shared_up
        self.shared_down, self.shared_route = shared_down, shared_route
        P = ctypes.pointer
        self.c = OrcMoeLayer(*(P(m.c) if m is not None else ctypes.POINTER(OrcMatrix)()
                               for m in (router, gate, up, down, shared_gate, shared_up,
                                         shared_down, shared_route)))


def moe_f64(layer: MoeLayer, x: np.ndarray, ids: np.ndarray, probs: np.ndarray,
            bf16_operands=True, route_out=False):
    x = np.ascontiguousarray(x, dtype=np.float32)
    T, H = x.shape
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    probs = np.ascontiguousarray(probs, dtype=np.float32)
    y = np.zeros((T, H), dtype=np.float64)
    ro = np.zeros((T * 9, H), dtype=np.float64) if route_out else None
    lib().orc_moe_f64(ctypes.byref(layer.c), T, _ptr(x), _ptr(ids), _ptr(probs),
                      1 if bf16_operands else 0, _ptr(y), None if ro is None else _ptr(ro))
    return (y, ro) if route_out else y


def merge_norm_f64(residual, y, weight=None, epsilon=1e-6, residual_bf16=False):
    """MoE merge into the residual and the next layer's RMSNorm (graph_merge_norm,
    gpu_graph.mm:48-61; prefill_merge, gpu_prefill.mm:140-150), rows = tokens:
    r = residual + y, stored in f32 (the reference) or as bf16 (RNE); normed =
    r * (mean(r^2) + eps)^-1/2 * weight over the stored r. Returns (stored r, normed) in
    float64 (normed None without weight)."""
    r = np.asarray(residual, dtype=np.float64) + np.asarray(y, dtype=np.float64)
    r = np.atleast_2d(r)
    if residual_bf16:
        stored = bf16_bits_to_f32(f32_to_bf16_bits(r.astype(np.float32))).astype(np.float64)
    else:
        stored = r.astype(np.float32).astype(np.float64)
    if weight is None:
        return stored, None
    inv = 1.0 / np.sqrt(np.mean(stored * stored, axis=1, keepdims=True) + float(epsilon))
    return stored, stored * inv * np.asarray(weight, dtype=np.float64)[None, :]


# ---------------------------------------------------------------- attention (numpy)
# Full-attention layer geometry (Qwen3.6-35B-A3B as the reference hard-codes it):
# 16 query heads share 2 KV heads (8 per group), head dim 256; the KV cache holds
# [position][kv head][256] bf16 (stride 512), the q projection output [token][16][512]
# interleaves each head's 256 query values with its 256 output-gate values
# (gpu_graph.mm:199-213; prefill_attention_bf16.mm:13-14, 34, 48).
ATT_HEADS, ATT_KV_HEADS, ATT_DIM = 16, 2, 256


def xorshift_values(seed: int, n: int, interleave: int = 1):
    """Inputs as the reference's attention checks draw them (orc_xorshift_fill):
    returns ([f32[n]] * interleave, next seed)."""
    outs = [np.zeros(n, dtype=np.float32) for _ in range(interleave)]
    ptrs = (ctypes.c_void_p * interleave)(*[o.ctypes.data for o in outs])
    seed = lib().orc_xorshift_fill(ctypes.c_uint32(seed), ptrs, interleave, n)
    return outs, int(seed)


def _attention_rows(S, V, partition, key_tile, round_probs):
    """Online softmax over one KV head for rows of scores S [R, n] (masked keys -inf)
    against values V [n, 256], exactly as the reference's double oracle forms it
    (prefill_attention_checks.mm:59-67, the arithmetic of prefill_attention_bf16.mm:32-54
    and graph_attention_combine gpu_graph.mm:199-213): partitions of `partition` keys,
    each scanned in `key_tile`-key blocks with a running maximum; the block's
    probabilities exp(s - max) enter the partition sum unrounded and the value product
    rounded to bf16 (through f32) when `round_probs`; partitions are combined against
    the global maximum. Returns the normalized [R, 256]."""
    R, n = S.shape
    with np.errstate(invalid="ignore", over="ignore"):
        M = np.max(S, axis=1)
        total = np.zeros(R)
        weighted = np.zeros((R, V.shape[1]))
        for start in range(0, n, partition):
            pm = np.full(R, -np.inf)
            psum = np.zeros(R)
            num = np.zeros((R, V.shape[1]))
            for block in range(start, min(start + partition, n), key_tile):
                end = min(block + key_tile, start + partition, n)
                Sb = S[:, block:end]
                nxt = np.maximum(pm, np.max(Sb, axis=1))
                alpha = np.where(np.isfinite(pm), np.exp(pm - nxt), 0.0)
                psum *= alpha
                num *= alpha[:, None]
                P = np.where(np.isfinite(Sb), np.exp(Sb - nxt[:, None]), 0.0)
                psum += P.sum(axis=1)
                if round_probs:
                    P = round_bf16(P.astype(np.float32)).astype(np.float64)
                num += P @ V[block:end]
                pm = nxt
            scale = np.where(np.isfinite(pm), np.exp(pm - M), 0.0)
            total += scale * psum
            weighted += scale[:, None] * num
    return weighted / total[:, None]


def attention_f64(q, keys, values, gate_raw, position, bf16_operands=True, partition=1024,
                  key_tile=32, round_probs=None):
    """Causal GQA attention of a chunk of `T` query tokens at cache positions
    position..position+T-1 with the output gate, in float64.

    q f32 [T, 16*256] (normed and rotated queries); keys/values [>= position+T, 512]
    (the bf16 cache's values as f32); gate_raw [T, 8192] (q projection output, head h's
    gate at h*512+256+d). Token t attends keys 0..position+t with scores q.k/16
    (prefill_attention_bf16.mm:39); out[t, h*256+d] = softmax-weighted values times
    sigmoid(gate) (gpu_graph.mm:212).

    bf16_operands=True is the reference's BF16 path as its own double oracle states it
    (prefill_attention_checks.mm:53, 57-67): q rounded to bf16 (RNE), probabilities
    rounded per key block (see _attention_rows; partition/key_tile select the blocks).
    bf16_operands=False is the plain softmax of the fp32 path (:68-69)."""
    q = np.asarray(q, dtype=np.float32)
    T = q.shape[0]
    n = position + T
    D = ATT_DIM
    K = np.asarray(keys[:n], dtype=np.float64).reshape(n, ATT_KV_HEADS, D)
    V = np.asarray(values[:n], dtype=np.float64).reshape(n, ATT_KV_HEADS, D)
    qq = (round_bf16(q) if bf16_operands else q).astype(np.float64).reshape(T, ATT_HEADS, D)
    if round_probs is None:
        round_probs = bf16_operands
    group = ATT_HEADS // ATT_KV_HEADS
    out = np.zeros((T, ATT_HEADS, D))
    last = position + np.arange(T)
    for kh in range(ATT_KV_HEADS):
        Q = qq[:, kh * group:(kh + 1) * group, :].reshape(T * group, D)
        rows_last = np.repeat(last, group)
        for r0 in range(0, T * group, 1024):
            r1 = min(r0 + 1024, T * group)
            S = (Q[r0:r1] @ K[:, kh, :].T) / 16.0
            S[np.arange(n)[None, :] > rows_last[r0:r1, None]] = -np.inf
            if bf16_operands or round_probs:
                res = _attention_rows(S, V[:, kh, :], partition, key_tile, round_probs)
            else:
                m = np.max(S, axis=1, keepdims=True)
                P = np.exp(S - m)
                res = (P @ V[:, kh, :]) / P.sum(axis=1, keepdims=True)
            out.reshape(T * ATT_HEADS, D)[np.arange(r0, r1) // group * ATT_HEADS
                                          + kh * group + np.arange(r0, r1) % group] = res
    gate = np.asarray(gate_raw, dtype=np.float64).reshape(T, ATT_HEADS, 2 * D)[:, :, D:]
    return (out / (1.0 + np.exp(-gate))).reshape(T, ATT_HEADS * D)


# ---------------------------------------------------------------- gated delta rule (numpy)
# Linear-attention (Gated DeltaNet) layer geometry as the reference hard-codes it: the
# convolved projection row [8192] holds q (16 key heads x 128) at 0, k (16 x 128) at 2048
# and v (32 value heads x 128) at 4096; value head h reads key head h/2; the state is
# [32 heads][128 value rows][128 key dims] f32 (gpu_prefill.mm:177-191).
DELTA_HEADS, DELTA_KEY_HEADS, DELTA_DIM, DELTA_ROW = 32, 16, 128, 8192


def delta_rule_f64(state, conv, decay, beta, tokens):
    """The gated delta rule, token by token in float64 (prefill_delta_checks.mm:33-37, the
    recurrence of prefill_delta gpu_prefill.mm:181-187). For every token t and value row
    (head h, row r; key head h/2):
        S[h,r,:] *= a[t,h]
        c = (v[t,h,r] - S[h,r,:].k[t]) * b[t,h]
        S[h,r,:] += k[t] * c
        out[t, h*128+r] = S[h,r,:].q[t]
    state [32,128,128] (not modified), conv [>=tokens, 8192], decay/beta [>=tokens, 32].
    Returns (out [tokens, 4096], state after the chunk), float64."""
    S = np.array(state, dtype=np.float64).reshape(DELTA_HEADS, DELTA_DIM, DELTA_DIM)
    conv = np.asarray(conv, dtype=np.float64)
    a = np.asarray(decay, dtype=np.float64)
    b = np.asarray(beta, dtype=np.float64)
    kh = np.arange(DELTA_HEADS) // 2
    out = np.zeros((tokens, DELTA_HEADS * DELTA_DIM))
    for t in range(tokens):
        q = conv[t, :2048].reshape(DELTA_KEY_HEADS, DELTA_DIM)[kh]          # [32,128]
        k = conv[t, 2048:4096].reshape(DELTA_KEY_HEADS, DELTA_DIM)[kh]
        v = conv[t, 4096:8192].reshape(DELTA_HEADS, DELTA_DIM)
        S *= a[t, :, None, None]
        pred = np.einsum("hrd,hd->hr", S, k)
        corr = (v - pred) * b[t, :, None]
        S += corr[:, :, None] * k[:, None, :]
        out[t] = np.einsum("hrd,hd->hr", S, q).reshape(-1)
    return out, S


def delta_history(history, raw, tokens):
    """The convolution history after a chunk (gpu_prefill.mm:189-190): row j of the new
    [3, 8192] history is old row j+tokens when j+tokens < 3, else raw row j+tokens-3."""
    h = np.asarray(history)
    r = np.asarray(raw)
    return np.stack([h[j + tokens] if j + tokens < 3 else r[j + tokens - 3] for j in range(3)])


def cpu_qmv(m: QMatrix, x, experts=None, batched=False, threads=1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    count = 1 if experts is None else len(experts)
    ids = None if experts is None else np.ascontiguousarray(experts, dtype=np.uint32)
    y = np.zeros(count * m.rows, dtype=np.float32)
    lib().orc_cpu_qmv(ctypes.byref(m.c), _ptr(x), None if ids is None else _ptr(ids), count,
                      1 if batched else 0, _ptr(y), threads)
    return y


def cpu_moe_token(layer: MoeLayer, x, threads=1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(layer.down.rows, dtype=np.float32)
    if lib().orc_cpu_moe_token(ctypes.byref(layer.c), _ptr(x), _ptr(y), threads) != 0:
        raise ValueError("Non-finite router logits.")
    return y


def rel_err(actual, expected) -> float:
    """max |actual - expected| / RMS(expected): the north-star tolerance measure."""
    a = np.asarray(actual, dtype=np.float64)
    e = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(e * e)))
    return float(np.max(np.abs(a - e))) / max(rms, 1e-30)
