"""CPU checks that pin the oracle (oracle/oracle.c via oracle/oracle.py).

Each oracle function is checked against something it does not itself compute: the
reference's own closed forms and known answers (QuantizedTests.cs, graph_checks.mm,
prefill_expert_checks.mm, split_prefix.cu's self-test, ModelTests.cs), an independent
numpy implementation (bit-string unpack, dense matmul), torch's bf16 conversion, or brute
force. A planted-mistake test shows the unpack check rejects a wrong bit layout.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as orc
from tests import refcases


# ------------------------------------------------------------ bf16 round-to-nearest-even

def test_bf16_rne_matches_torch_and_known_values():
    rng = np.random.default_rng(0)
    v = np.concatenate([rng.normal(size=20000).astype(np.float32) * 10 ** rng.uniform(-6, 6, 20000).astype(np.float32),
                        np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -1 - 2 ** -8, 0.0, -0.0, 65504.0], dtype=np.float32)])
    ours = orc.f32_to_bf16_bits(v)
    ref = torch.from_numpy(v).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    assert [int(orc.lib().orc_f32_to_bf16(float(x))) for x in (1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8)] == [0x3F80, 0x3F80, 0x3F82]
    assert orc.lib().orc_bf16_to_f32(0x3B80) == 2 ** -8 and orc.lib().orc_bf16_to_f32(0xBE80) == -0.25


# ---------------------------------------------------------------------- unpack + dequant

@pytest.mark.parametrize("bits", [5, 8])
def test_code_extraction_matches_independent_bitstring_unpack(bits):
    rng = np.random.default_rng(bits)
    words = rng.integers(0, 2 ** 32, size=(3, 7, 256 * bits // 32), dtype=np.uint64).astype(np.uint32)
    want = orc.unpack_codes(words, bits, 256)
    L = orc.lib()
    for e in range(3):
        for r in range(7):
            row = np.ascontiguousarray(words[e, r])
            got = [L.orc_code(row.ctypes.data, bits, c) for c in range(256)]
            assert got == list(want[e, r])


def test_planted_unpack_mistake_is_caught():
    """A bit layout off by one position (MSB-first within each code) must not reproduce the
    reference's closed form; the check below has teeth."""
    m = refcases.populate(2, 5, 128, 5, 3)
    words = m.packed.reshape(2, 5, -1)
    codes = orc.unpack_codes(words, 5, 128)
    wrong = np.zeros_like(codes)
    for b in range(5):
        wrong |= ((codes >> b) & 1) << (4 - b)
    c = np.arange(128)[None, None, :]
    e = np.arange(2)[:, None, None]
    r = np.arange(5)[None, :, None]
    closed = (c * 7 + e * 3 + r * 5 + 3 * 11) & 31
    assert np.array_equal(codes, closed)
    assert not np.array_equal(wrong, closed)


@pytest.mark.parametrize("bits", [5, 8])
@pytest.mark.parametrize("columns", [64, 192, 256, 512, 2048, 4096])
def test_dequant_row_reproduces_reference_scalar_weight(bits, columns):
    """Populate + ScalarWeight (QuantizedTests.cs:136-165): the packed matrix the reference's
    test writes dequantizes, row by row, to exactly the closed-form float32 weights."""
    m = refcases.populate(9, 5, columns, bits, 3)
    want = refcases.scalar_weights(9, 5, columns, bits, 3)
    out = np.zeros(columns, dtype=np.float32)
    for e in (0, 4, 8):
        for r in range(5):
            orc.lib().orc_dequant_row(orc.ctypes.byref(m.c), e, r, out.ctypes.data)
            assert np.array_equal(out, want[e, r])
    assert np.array_equal(m.dequant(), want)


# -------------------------------------------------------------------------------- GEMV

@pytest.mark.parametrize("bits", [5, 8])
def test_qmv_selected_expert_closed_form(bits):
    """SelectedExpertGemv (QuantizedTests.cs:228-256): scale 1.0, bias 0.5 =>
    y = sum (q + .5) x exactly."""
    e = np.arange(3)[:, None, None]
    r = np.arange(7)[None, :, None]
    c = np.arange(128)[None, None, :]
    q = ((c * 7 + e * 3 + r) & ((1 << bits) - 1)).astype(np.uint32)
    m = orc.QMatrix(orc.pack_codes(q, bits), np.full(42, 0x3F80, np.uint16), np.full(42, 0x3F00, np.uint16), 3, 7, 128, bits)
    x = np.sin(np.arange(256, dtype=np.float32) * np.float32(.17)).astype(np.float32)
    y = orc.qmv_f64(m, x, [2, 0], batched=True)
    for slot, ex in enumerate([2, 0]):
        want = (q[ex].astype(np.float64) + .5) @ x[slot * 128:(slot + 1) * 128].astype(np.float64)
        assert np.max(np.abs(y[slot * 7:(slot + 1) * 7] - want)) < 1e-9


def test_qmv_cuda_selftest_known_answer():
    """di_cuda_prefix_selftest (split_prefix.cu:621-649): w=(i*17+3)%256, scale 0x3b80 (1/256),
    bias 0xbe80 (-0.25) => y = sum (w/256 - .25) x; two experts selected [1, 0]."""
    w = ((np.arange(2 * 13 * 256) * 17 + 3) % 256).astype(np.uint32).reshape(2, 13, 256)
    m = orc.QMatrix(orc.pack_codes(w, 8), np.full(2 * 13 * 4, 0x3B80, np.uint16), np.full(2 * 13 * 4, 0xBE80, np.uint16),
                    2, 13, 256, 8)
    x = (((np.arange(256) * 11) % 23 - 11) / np.float32(23)).astype(np.float32)
    y = orc.qmv_f64(m, x, [1, 0])
    for s, e in enumerate([1, 0]):
        want = (w[e].astype(np.float64) / 256 - .25) @ x.astype(np.float64)
        assert np.max(np.abs(y[s * 13:(s + 1) * 13] - want)) < 1e-12


def test_qmv_zero_codes_bias_only_closed_form():
    """IndependentMixedGemvs (QuantizedTests.cs:166-209): zero codes, scale 1, bias b => b*sum(x)."""
    m = orc.QMatrix(np.zeros(3 * 7 * 128 * 8 // 32, np.uint32), np.full(3 * 7 * 2, 0x3F80, np.uint16),
                    orc.f32_to_bf16_bits((2 + (np.arange(42) // 2) * .25).astype(np.float32)), 3, 7, 128, 8)
    x = ((np.arange(256) - 100) * np.float32(.005)).astype(np.float32)
    y = orc.qmv_f64(m, x, [2, 0], batched=True)
    for slot, e in enumerate([2, 0]):
        for r in range(7):
            want = (2 + (e * 7 + r) * .25) * x[slot * 128:(slot + 1) * 128].astype(np.float64).sum()
            assert abs(y[slot * 7 + r] - want) < 1e-9


@pytest.mark.parametrize("bits", [5, 8])
def test_qmv_and_dense_match_numpy_matmul(bits):
    rng = np.random.default_rng(11)
    m = orc.random_matrix(rng, 4, 33, 320, bits)
    W = m.dequant().astype(np.float64)
    x = rng.normal(size=(6, 320)).astype(np.float32)
    y = orc.qmv_f64(m, x[0], [3])
    assert np.max(np.abs(y - W[3] @ x[0])) < 1e-9
    d = orc.dense_f64(m, x, expert=2, round_operands=False)
    assert np.max(np.abs(d - x.astype(np.float64) @ W[2].T)) < 1e-9
    d_bf = orc.dense_f64(m, x, expert=2, round_operands=True)
    want_bf = orc.round_bf16(x).astype(np.float64) @ orc.round_bf16(W[2].astype(np.float32)).astype(np.float64).T
    assert np.max(np.abs(d_bf - want_bf)) < 1e-9


def test_cpu_baseline_path_matches_fp64():
    """The reference-faithful fp32 CPU path (MatVec.cs:40-55 after row dequant) agrees with the
    fp64 oracle to fp32 accuracy, single- and multi-threaded (identical results)."""
    rng = np.random.default_rng(12)
    m = orc.random_matrix(rng, 3, 100, 2048, 8)
    x = rng.normal(size=2048).astype(np.float32)
    a = orc.cpu_qmv(m, x, [2, 1], threads=1)
    b = orc.cpu_qmv(m, x, [2, 1], threads=4)
    assert np.array_equal(a, b)
    assert orc.rel_err(a, orc.qmv_f64(m, x, [2, 1])) < 1e-5


# ------------------------------------------------------------------------------ routing

def test_top8_reference_known_answers():
    """graph_checks.mm:63-77 (stable-sort oracle, probability closed form) and the routing
    KAT of QuantizedTests.cs:280-288."""
    for v in refcases.top8_cases():
        ids, probs = orc.top8(v)
        exp = refcases.stable_top8(v)
        assert np.array_equal(ids, exp)
        ch = v[exp].astype(np.float64)
        p = np.exp(ch - ch[0])
        p /= p.sum()
        assert np.max(np.abs(probs - p)) <= 1e-6
    ids, probs = orc.top8((np.arange(256) * np.float32(.01)).astype(np.float32))
    assert list(ids) == list(range(255, 247, -1))
    assert abs(probs.sum() - 1) <= 1e-6 and probs[0] > probs[7]
    with pytest.raises(ValueError):
        orc.top8(np.where(np.arange(256) == 9, np.nan, 0).astype(np.float32))


def test_top8_bf16_matches_brute_force_with_ties():
    rng = np.random.default_rng(3)
    lg = orc.round_bf16(rng.normal(size=(500, 256)).astype(np.float32))
    lg[::5, 20:60] = 2.5
    ids, _ = orc.top8_bf16(orc.f32_to_bf16_bits(lg))
    for t in range(500):
        assert np.array_equal(ids[t], refcases.stable_top8(lg[t]))


@pytest.mark.parametrize("count", [64, 65, 127, 128, 129, 512, 513, 2048])
@pytest.mark.parametrize("pattern", [0, 1, 2])
def test_build_groups_invariants(count, pattern):
    """prefill_expert_checks.mm:44-52: every route once, under its expert, counts; plus the
    ascending order of prefill_build_groups' prefix sum (prefill_moe.mm:12-14)."""
    ids = refcases.route_pattern(pattern, count)
    counts, routes = orc.build_groups(ids, count, 256)
    flat = ids.reshape(-1)
    assert np.array_equal(counts, np.bincount(flat, minlength=256))
    seen = np.zeros(count * 8, bool)
    for e in range(256):
        lst = routes[e * count:e * count + counts[e]]
        assert np.array_equal(lst, np.flatnonzero(flat == e))
        seen[lst] = True
    assert seen.all()
    tiles = sum((int(c) + 63) // 64 for c in counts)
    assert tiles == sum(1 for e in range(256) for s in range(0, counts[e], 64))


def test_argmax_known_answers():
    """graph_checks.mm:89-103 and ModelTests.cs:23-28."""
    base = (np.arange(248320, dtype=np.float32) * np.float32(1e-5)).astype(np.float32)
    assert orc.argmax(base) == 248319
    t = base.copy(); t[100] = t[200] = 10
    assert orc.argmax(t) == 100
    t = base.copy(); t[0] = np.nan
    assert orc.argmax(t) == 0xFFFFFFFF
    assert orc.argmax(np.array([1, 3, 3], np.float32)) == 1
    assert orc.argmax(np.array([np.inf], np.float32)) == 0xFFFFFFFF


# --------------------------------------------------------------------------- MoE blocks

def _layer(rng, E, H, I, bits):
    mk = lambda e, r, c, b=bits: orc.random_matrix(rng, e, r, c, b)  # noqa: E731
    return orc.MoeLayer(orc.random_matrix(rng, 1, E, H, 8, 1.25e-4, 5e-4), mk(E, I, H), mk(E, I, H), mk(E, H, I),
                        mk(1, I, H), mk(1, I, H), mk(1, H, I), orc.random_matrix(rng, 1, 1, H, 8))


def _numpy_moe(L, x, ids, probs, rounded):
    r = orc.round_bf16 if rounded else (lambda a: a)
    W = {k: getattr(L, k).dequant().astype(np.float32) for k in ("gate", "up", "down", "shared_gate", "shared_up",
                                                                "shared_down", "shared_route")}
    if rounded:
        for k in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
            W[k] = orc.round_bf16(W[k])
    W = {k: v.astype(np.float64) for k, v in W.items()}
    silu = lambda v: v / (1 + np.exp(-v))  # noqa: E731
    y = np.zeros((x.shape[0], L.down.rows))
    for t in range(x.shape[0]):
        xt = r(x[t]).astype(np.float64)
        sa = silu(W["shared_gate"][0] @ xt) * (W["shared_up"][0] @ xt)
        sa = r(sa.astype(np.float32)).astype(np.float64) if rounded else sa
        gate = 1 / (1 + np.exp(-(W["shared_route"][0, 0] @ x[t].astype(np.float64))))
        y[t] = (W["shared_down"][0] @ sa) * gate
        for s in range(8):
            e = ids[t, s]
            a = silu(W["gate"][e] @ xt) * (W["up"][e] @ xt)
            a = r(a.astype(np.float32)).astype(np.float64) if rounded else a
            y[t] += probs[t, s] * (W["down"][e] @ a)
    return y


@pytest.mark.parametrize("rounded", [False, True])
def test_moe_f64_matches_numpy_composition(rounded):
    """Moe (Qwen36Model.cs:218-245) / prefill merge order, against a numpy composition of
    dense matmuls (independent of oracle.c's loops)."""
    rng = np.random.default_rng(21)
    L = _layer(rng, 16, 128, 64, 5)
    x = orc.round_bf16(rng.normal(size=(5, 128)).astype(np.float32))
    ids, probs = orc.top8_bf16(orc.f32_to_bf16_bits(rng.normal(size=(5, 16)).astype(np.float32)))
    y = orc.moe_f64(L, x, ids, probs, bf16_operands=rounded)
    want = _numpy_moe(L, x, ids, probs, rounded)
    assert np.max(np.abs(y - want)) < 1e-6 * max(1.0, np.abs(want).max())


def test_expert_mlp_matches_reference_closed_form():
    """FusedExperts (QuantizedTests.cs:71-117) on the reference's closed-form weights."""
    g, u = refcases.populate(9, 192, 128, 8, 1), refcases.populate(9, 192, 128, 8, 2)
    d, s = refcases.populate(9, 128, 192, 5, 3), refcases.populate(1, 128, 64, 5, 4)
    x = (np.sin(np.arange(128, dtype=np.float32) * np.float32(.13)) * np.float32(.1)).astype(np.float32)
    sx = (np.cos(np.arange(64, dtype=np.float32) * np.float32(.07)) * np.float32(.2)).astype(np.float32)
    ids = [8, 0, 6, 2, 5, 1, 7, 3]
    out, sout = orc.expert_mlp_f64(g, u, d, s, x, sx, ids)
    wg, wu = refcases.scalar_weights(9, 192, 128, 8, 1), refcases.scalar_weights(9, 192, 128, 8, 2)
    wd, ws = refcases.scalar_weights(9, 128, 192, 5, 3), refcases.scalar_weights(1, 128, 64, 5, 4)
    for slot, e in enumerate(ids):
        gg = wg[e].astype(np.float64) @ x
        uu = wu[e].astype(np.float64) @ x
        act = gg / (1 + np.exp(-gg)) * uu
        # ScalarWeight differs from the exact q*s+b by at most one fp32 rounding
        assert np.max(np.abs(out[slot * 128:(slot + 1) * 128] - wd[e].astype(np.float64) @ act)) < 3e-6
    assert np.max(np.abs(sout - ws[0].astype(np.float64) @ sx)) < 3e-6


def test_cpu_moe_token_matches_fp64():
    """The CPU baseline's MoE token (fp32, reference host order) against fp64."""
    rng = np.random.default_rng(31)
    L = _layer(rng, 32, 256, 128, 8)
    x = orc.round_bf16(rng.normal(size=256).astype(np.float32))
    y = orc.cpu_moe_token(L, x)
    logits = orc.cpu_qmv(L.router, x)
    ids, probs = orc.top8(logits)
    want = orc.moe_f64(L, x[None, :], ids[None, :], probs[None, :], bf16_operands=False)[0]
    assert orc.rel_err(y, want) < 1e-4


def test_merge_norm_closed_forms():
    """merge_norm_f64 pinned by closed forms of RMSNorm: a constant row c gives
    c / sqrt(c^2 + eps) * w; a row scaled by k gives k r / sqrt(k^2 mean(r^2) + eps) * w; bf16
    storage rounds r before the norm; eps enters once, under the square root."""
    w = np.linspace(0.5, 2.0, 64)
    for c, eps in ((3.0, 1e-6), (-0.25, 1e-2), (1e-3, 1e-6)):
        stored, normed = orc.merge_norm_f64(np.full((1, 64), c - 1.0), np.ones((1, 64)), w, eps)
        assert np.allclose(stored, c, rtol=1e-6) and np.all(stored == stored[0, 0])
        cs = stored[0, 0]                      # c after the f32 storage rounding
        assert np.allclose(normed[0], cs / np.sqrt(cs * cs + eps) * w, rtol=1e-12)
    rng = np.random.default_rng(1)
    r = rng.normal(size=(3, 64)).astype(np.float32).astype(np.float64)
    for k in (2.0, 0.5, 1024.0):
        _, a = orc.merge_norm_f64(k * r, np.zeros_like(r), w, 1e-6)
        ms = np.mean(r * r, axis=1, keepdims=True)
        assert np.allclose(a, k * r / np.sqrt(k * k * ms + 1e-6) * w, rtol=1e-12)
    # bf16 storage: 1 + 2^-9 rounds to 1 (tie to even), 1 + 3*2^-9 to 1 + 2^-7
    s, _ = orc.merge_norm_f64(np.array([[1.0, 1.0]]), np.array([[2.0 ** -9, 3 * 2.0 ** -9]]), residual_bf16=True)
    assert s.tolist() == [[1.0, 1.0 + 2.0 ** -7]]
    # f32 storage: the sum is rounded to f32 before the norm
    s, _ = orc.merge_norm_f64(np.array([[1.0]]), np.array([[2.0 ** -30]]))
    assert s.tolist() == [[1.0]]


# ---------------------------------------------------------------- attention

def _xorshift_py(seed, n):
    out = []
    for _ in range(n):
        seed ^= (seed << 13) & 0xFFFFFFFF
        seed ^= seed >> 17
        seed ^= (seed << 5) & 0xFFFFFFFF
        out.append(np.float32((int(seed % 10001) - 5000)) / np.float32(12500.0))
    return np.array(out, dtype=np.float32), seed


def test_xorshift_generator():
    """orc_xorshift_fill against a pure-Python restatement of prefill_attention_checks.mm:18,
    including the interleaved key/value fill of :20-24."""
    (a,), s = orc.xorshift_values(0x6a51c9e7, 300)
    b, s2 = _xorshift_py(0x6a51c9e7, 300)
    assert np.array_equal(a, b) and s == s2
    (k, v), _ = orc.xorshift_values(s, 50, 2)
    c, _ = _xorshift_py(s, 100)
    assert np.array_equal(k, c[0::2]) and np.array_equal(v, c[1::2])
    assert np.all(np.abs(a) <= 0.4)


def _attention_inputs(T, position, seed=3):
    rng = np.random.default_rng(seed)
    n = position + T
    q = rng.uniform(-0.4, 0.4, size=(T, 4096)).astype(np.float32)
    k = orc.round_bf16(rng.uniform(-0.4, 0.4, size=(n, 512)).astype(np.float32))
    v = orc.round_bf16(rng.uniform(-0.4, 0.4, size=(n, 512)).astype(np.float32))
    g = rng.uniform(-2, 2, size=(T, 8192)).astype(np.float32)
    return q, k, v, g


def test_attention_zero_queries_closed_form():
    """bf16_attention_long_checks.mm:13,20: q = 0 makes every score 0, so each head
    averages its KV head's values; with values 1 / -2 and gates 0 the output is .5 / -1."""
    T, position = 6, 45
    v = np.where(np.arange(512) < 256, 1.0, -2.0)[None, :].repeat(position + T, 0)
    for part, tile in ((1024, 32), (16, 4)):
        out = orc.attention_f64(np.zeros((T, 4096)), np.zeros_like(v), v, np.zeros((T, 8192)), position,
                                partition=part, key_tile=tile)
        assert np.all(out[:, :2048] == 0.5) and np.all(out[:, 2048:] == -1.0)


def test_attention_single_key():
    """The first token of an empty cache sees one key: out = v * sigmoid(gate), whatever q."""
    q, k, v, g = _attention_inputs(1, 0)
    out = orc.attention_f64(q, k, v, g, 0).reshape(16, 256)
    gate = g.reshape(16, 512)[:, 256:].astype(np.float64)
    want = v[0].reshape(2, 256).astype(np.float64)[np.arange(16) // 8] / (1 + np.exp(-gate))
    assert np.allclose(out, want, rtol=1e-15, atol=0)


def _softmax_loops(q, k, v, g, position):
    """Brute force over (token, head) with scipy's softmax (independent of the oracle's
    vectorized masking and head grouping)."""
    from scipy.special import softmax
    T = q.shape[0]
    out = np.zeros((T, 16, 256))
    for t in range(T):
        for h in range(16):
            kh = h // 8
            keys = k[:position + t + 1, kh * 256:(kh + 1) * 256].astype(np.float64)
            s = keys @ q[t, h * 256:(h + 1) * 256].astype(np.float64) / 16
            p = softmax(s)
            out[t, h] = p @ v[:position + t + 1, kh * 256:(kh + 1) * 256]
            out[t, h] *= 1 / (1 + np.exp(-g[t, h * 512 + 256:(h + 1) * 512].astype(np.float64)))
    return out.reshape(T, 4096)


def test_attention_plain_softmax_brute_force():
    q, k, v, g = _attention_inputs(5, 11)
    want = _softmax_loops(q, k, v, g, 11)
    got = orc.attention_f64(q, k, v, g, 11, bf16_operands=False)
    assert np.allclose(got, want, rtol=1e-12, atol=1e-15)
    # q rounded to bf16, probabilities unrounded: the same softmax over rounded queries
    got = orc.attention_f64(q, k, v, g, 11, bf16_operands=True, round_probs=False)
    assert np.allclose(got, _softmax_loops(orc.round_bf16(q), k, v, g, 11), rtol=1e-12, atol=1e-15)


@pytest.mark.parametrize("partition,tile", [(1024, 32), (64, 32), (32, 32), (7, 3), (5, 5)])
def test_attention_online_recurrence(partition, tile):
    """Without probability rounding the partitioned online softmax equals the softmax for
    any partition and key block (a missed rescale or a wrong combine fails this)."""
    q, k, v, g = _attention_inputs(9, 70, seed=8)
    exact = orc.attention_f64(orc.round_bf16(q), k, v, g, 70, bf16_operands=False)
    got = orc.attention_f64(q, k, v, g, 70, partition=partition, key_tile=tile, round_probs=False)
    assert np.allclose(got, exact, rtol=1e-11, atol=1e-14)


def test_attention_probability_rounding():
    """Rounding each probability to bf16 moves it by at most 2^-9 relative; the output
    moves by at most 2^-9 * max|v| * sigmoid(gate), and does move (the rounding is real)."""
    q, k, v, g = _attention_inputs(12, 200, seed=9)
    unrounded = orc.attention_f64(q, k, v, g, 200, round_probs=False)
    rounded = orc.attention_f64(q, k, v, g, 200)
    d = np.abs(rounded - unrounded)
    assert np.max(d) <= 2.0 ** -9 * np.max(np.abs(v)) and np.max(d) > 1e-7
    # the rounding points depend on the key blocks: another block size changes the result
    other = orc.attention_f64(q, k, v, g, 200, key_tile=64)
    assert np.max(np.abs(other - rounded)) > 1e-8


def test_attention_causal_mask():
    """Row t reads keys 0..position+t only: changing key/value rows past that leaves the
    row unchanged and changes the later rows."""
    q, k, v, g = _attention_inputs(4, 20, seed=10)
    base = orc.attention_f64(q, k, v, g, 20)
    k2, v2 = k.copy(), v.copy()
    k2[22:] += 0.25
    v2[22:] -= 0.5
    moved = orc.attention_f64(q, k2, v2, g, 20)
    assert np.array_equal(base[:2], moved[:2])
    assert np.all(np.max(np.abs(base[2:] - moved[2:]), axis=1) > 1e-3)


# ---------------------------------------------------------------- gated delta rule

def _delta_inputs(T, seed=4, unit_k=True):
    rng = np.random.default_rng(seed)
    conv = rng.normal(size=(T, 8192)).astype(np.float32) * 0.3
    if unit_k:
        k = conv[:, 2048:4096].reshape(T, 16, 128).astype(np.float64)
        k /= np.linalg.norm(k, axis=2, keepdims=True)
        conv[:, 2048:4096] = k.reshape(T, 2048)
    state = (rng.normal(size=(32, 128, 128)) * 0.01).astype(np.float32)
    a = rng.uniform(0.5, 1.0, size=(T, 32)).astype(np.float32)
    b = rng.uniform(0.0, 1.0, size=(T, 32)).astype(np.float32)
    return state, conv, a, b


def test_delta_rule_closed_forms():
    """a = 1, b = 0 leaves the state alone and reads it out: out = S0 q. a = 0, b = 1 with
    unit keys forgets everything: S_t = v_t k_t^T, so out_t = v_t (k_t . q_t)."""
    state, conv, a, b = _delta_inputs(5)
    out, S = orc.delta_rule_f64(state, conv, np.ones_like(a), np.zeros_like(b), 5)
    assert np.array_equal(S, state.astype(np.float64))
    q = conv[:, :2048].reshape(5, 16, 128).astype(np.float64)[:, np.arange(32) // 2]
    want = np.einsum("hrd,thd->thr", state.astype(np.float64), q).reshape(5, 4096)
    assert np.allclose(out, want, rtol=1e-12, atol=1e-15)
    out, S = orc.delta_rule_f64(state, conv, np.zeros_like(a), np.ones_like(b), 5)
    k = conv[:, 2048:4096].reshape(5, 16, 128).astype(np.float64)[:, np.arange(32) // 2]
    v = conv[:, 4096:].reshape(5, 32, 128).astype(np.float64)
    assert np.allclose(out, (v * np.einsum("thd,thd->th", k, q)[:, :, None]).reshape(5, 4096), rtol=1e-12,
                       atol=1e-14)
    assert np.allclose(S, v[-1][:, :, None] * k[-1][:, None, :], rtol=1e-12, atol=1e-15)


def test_delta_rule_writes_the_value():
    """The delta rule's defining property: with b = 1 the updated state maps k_t to
    a*S_prev*k_t*(1 - |k_t|^2) + v_t*|k_t|^2, i.e. to v_t exactly for a unit key, whatever
    it held before and whatever the decay."""
    state, conv, a, b = _delta_inputs(3, seed=6)
    for t in range(1, 4):
        bb = b.copy()
        bb[t - 1] = 1.0
        _, S0 = orc.delta_rule_f64(state, conv, a, bb, t - 1)
        _, S = orc.delta_rule_f64(state, conv, a, bb, t)
        k = conv[t - 1, 2048:4096].reshape(16, 128).astype(np.float64)[np.arange(32) // 2]
        v = conv[t - 1, 4096:].reshape(32, 128).astype(np.float64)
        kk = np.sum(k * k, axis=1)[:, None]
        prev = a[t - 1][:, None].astype(np.float64) * np.einsum("hrd,hd->hr", S0, k)
        assert np.allclose(np.einsum("hrd,hd->hr", S, k), prev * (1 - kk) + v * kk, rtol=1e-11, atol=1e-13)
        assert np.max(np.abs(kk - 1)) < 1e-6 and np.allclose(np.einsum("hrd,hd->hr", S, k), v, atol=1e-5)


def test_delta_rule_brute_force_rows():
    """Pure-Python loops over a few rows (independent of the vectorized head mapping)."""
    T = 4
    state, conv, a, b = _delta_inputs(T, seed=7, unit_k=False)
    out, S = orc.delta_rule_f64(state, conv, a, b, T)
    for head, row in ((0, 0), (5, 77), (31, 127)):
        s = [float(x) for x in state[head, row]]
        kh = head // 2
        for t in range(T):
            s = [x * float(a[t, head]) for x in s]
            k = [float(conv[t, 2048 + kh * 128 + d]) for d in range(128)]
            q = [float(conv[t, kh * 128 + d]) for d in range(128)]
            pred = sum(x * y for x, y in zip(s, k))
            c = (float(conv[t, 4096 + head * 128 + row]) - pred) * float(b[t, head])
            s = [x + y * c for x, y in zip(s, k)]
            assert abs(out[t, head * 128 + row] - sum(x * y for x, y in zip(s, q))) < 1e-12
        assert np.allclose(S[head, row], s, rtol=0, atol=1e-14)


def test_delta_rule_chunk_composition():
    """Two calls that carry the state equal one call over the whole sequence."""
    T = 9
    state, conv, a, b = _delta_inputs(T, seed=8)
    out, S = orc.delta_rule_f64(state, conv, a, b, T)
    o1, S1 = orc.delta_rule_f64(state, conv, a, b, 4)
    o2, S2 = orc.delta_rule_f64(S1, conv[4:], a[4:], b[4:], 5)
    assert np.allclose(np.concatenate([o1, o2]), out, rtol=1e-12, atol=1e-15)
    assert np.allclose(S2, S, rtol=1e-12, atol=1e-15)


def test_delta_history_roll():
    hist = np.arange(3 * 8)[:, None].repeat(2, 1).reshape(3, 16)[:, :8].astype(np.float32)
    raw = 100 + np.arange(5 * 8).reshape(5, 8).astype(np.float32)
    assert np.array_equal(orc.delta_history(hist, raw, 1), np.stack([hist[1], hist[2], raw[0]]))
    assert np.array_equal(orc.delta_history(hist, raw, 2), np.stack([hist[2], raw[0], raw[1]]))
    assert np.array_equal(orc.delta_history(hist, raw, 5), raw[2:5])


@pytest.mark.parametrize("rounded", [False, True])
def test_moe_f64_sigmoid_gated_combine_closed_form(rounded):
    """The sigma-gated combine (Moe, Qwen36Model.cs:230-244) by a closed form. With every
    code 0 and scale 1, each weight equals its row's bias, so a row of any matrix reduces to
    b_row * sum(x): gate_i = bg_i S, up_i = bu_i S with S = sum(x), act_i = silu(gate_i) up_i,
    down_h = bd_h sum_i act_i, and the shared route is sigmoid(br S). Hence
        y[h] = sigmoid(br S) bsd_h A_shared + sum_slot p_slot bd[e_slot]_h A[e_slot]
    with A = sum_i act_i. One-hot probabilities leave the shared term plus one expert."""
    E, H, I = 12, 128, 64

    def const_rows(experts, rows, cols, vals):
        bias = np.repeat(orc.f32_to_bf16_bits(vals.astype(np.float32)).reshape(experts, rows, 1), cols // 64, axis=2)
        return orc.QMatrix(np.zeros(experts * rows * cols * 8 // 32, np.uint32),
                           np.full(experts * rows * (cols // 64), 0x3F80, np.uint16), bias, experts, rows, cols, 8)

    e_, r_ = np.meshgrid(np.arange(E), np.arange(I), indexing="ij")
    bg = ((e_ * 3 + r_) % 7 - 3) / 32.0
    bu = ((e_ + r_ * 5) % 5 + 1) / 64.0
    e2, h2 = np.meshgrid(np.arange(E), np.arange(H), indexing="ij")
    bd = ((e2 * 5 + h2 * 3) % 9 - 4) / 16.0
    bsg = (np.arange(I) % 3 - 1) / 8.0
    bsu = (np.arange(I) % 4 + 1) / 16.0
    bsd = (np.arange(H) % 5 - 2) / 4.0
    br = np.array([0.375])
    L = orc.MoeLayer(None, const_rows(E, I, H, bg), const_rows(E, I, H, bu), const_rows(E, H, I, bd),
                     const_rows(1, I, H, bsg), const_rows(1, I, H, bsu), const_rows(1, H, I, bsd),
                     const_rows(1, 1, H, br))
    T = 3
    x = np.zeros((T, H), dtype=np.float32)
    x[0, :4] = [0.5, 0.25, -0.125, 1.0]           # S = 1.625
    x[1, 10] = -2.0                                # S = -2
    x[2, ::2] = 0.015625                           # S = 1
    ids = np.array([[3, 0, 7, 11, 1, 2, 4, 5], [6, 8, 9, 10, 0, 1, 2, 3], [2, 4, 6, 8, 10, 11, 1, 0]], np.int32)
    probs = np.zeros((T, 8), dtype=np.float32)
    probs[0] = [0.5, 0.25, 0.125, 0.0625, 0.03125, 0.015625, 0.0078125, 0.0078125]
    probs[1, 0] = 1.0                              # one-hot: the shared term plus expert 6
    probs[2] = 0.125
    y = orc.moe_f64(L, x, ids, probs, bf16_operands=rounded)

    def silu(v):
        return v / (1 + np.exp(-v))

    def act_sum(g_rows, u_rows, S):
        a = silu(g_rows * S) * (u_rows * S)
        if rounded:
            a = orc.round_bf16(a.astype(np.float32)).astype(np.float64)
        return a.sum()

    for t in range(T):
        S = float(x[t].astype(np.float64).sum())
        want = 1 / (1 + np.exp(-br[0] * S)) * bsd * act_sum(bsg, bsu, S)
        for s in range(8):
            e = ids[t, s]
            want = want + float(probs[t, s]) * bd[e] * act_sum(bg[e], bu[e], S)
        assert np.max(np.abs(y[t] - want)) <= 1e-12 * max(1.0, np.abs(want).max()), t


def test_dense_blas_matches_dense_f64():
    """dense_f64_blas (the BLAS form used at full chunk sizes) against the scalar dense_f64,
    both rounding modes, an expert other than 0 and both bit widths."""
    rng = np.random.default_rng(41)
    for bits in (5, 8):
        m = orc.random_matrix(rng, 3, 70, 384, bits)
        x = rng.normal(size=(9, 384)).astype(np.float32)
        for rnd in (False, True):
            a = orc.dense_f64(m, x, expert=2, round_operands=rnd)
            b = orc.dense_f64_blas(m, x, expert=2, round_operands=rnd)
            assert np.max(np.abs(a - b)) <= 1e-12 * np.abs(a).max()
