"""Closed-form fixtures restated from the reference's own tests (data generators only).

populate()/scalar_weight(): QuantizedTests.cs:136-165.
prefill_value(): prefill_expert_checks.mm:13-22.
"""
import numpy as np

from oracle.oracle import QMatrix, f32_to_bf16_bits, pack_codes


def scalar_weight(bits, expert, row, column, seed):
    """ScalarWeight (QuantizedTests.cs:136-141), evaluated in float32 like C#."""
    group = column // 64
    q = (column * 7 + expert * 3 + row * 5 + seed * 11) & ((1 << bits) - 1)
    s = np.float32(((group + seed) % 3 + 1) / np.float32(512.0))
    b = np.float32(((row + group + seed) % 5 - 2) / np.float32(32.0))
    return np.float32(np.float32(q) * s + b)


def populate(experts, rows, columns, bits, seed) -> QMatrix:
    """Populate (QuantizedTests.cs:142-165)."""
    e = np.arange(experts)[:, None, None]
    r = np.arange(rows)[None, :, None]
    c = np.arange(columns)[None, None, :]
    codes = ((c * 7 + e * 3 + r * 5 + seed * 11) & ((1 << bits) - 1)).astype(np.uint32)
    g = np.arange(columns // 64)[None, None, :]
    scales = (((g + seed) % 3 + 1) / 512.0 + 0 * e + 0 * r).astype(np.float32)
    biases = (((r + g + seed) % 5 - 2) / 32.0 + 0 * e).astype(np.float32)
    # values are exact in bf16, so the >>16 truncation of the reference equals RNE here
    sb = (scales.view(np.uint32) >> 16).astype(np.uint16)
    bb = (biases.view(np.uint32) >> 16).astype(np.uint16)
    return QMatrix(pack_codes(codes, bits), sb, bb, experts, rows, columns, bits)


def scalar_weights(experts, rows, columns, bits, seed) -> np.ndarray:
    e = np.arange(experts)[:, None, None]
    r = np.arange(rows)[None, :, None]
    c = np.arange(columns)[None, None, :]
    q = ((c * 7 + e * 3 + r * 5 + seed * 11) & ((1 << bits) - 1)).astype(np.float32)
    g = c // 64
    s = (((g + seed) % 3 + 1) / np.float32(512.0)).astype(np.float32)
    b = (((r + g + seed) % 5 - 2) / np.float32(32.0)).astype(np.float32)
    return (q * s + b).astype(np.float32)


def prefill_matrix(kind, experts, rows, columns, bits) -> QMatrix:
    """The matrices of prefill_expert_checks.mm:10-19 (kind 0 gate, 1 up, 2 down)."""
    e = np.arange(experts)[:, None, None]
    r = np.arange(rows)[None, :, None]
    c = np.arange(columns)[None, None, :]
    codes = ((e * 3 + r * 7 + c * 5 + kind * 11) & ((1 << bits) - 1)).astype(np.uint32)
    a = np.arange(columns // 64)[None, None, :]
    scale = ((a + 1) / 4096.0 + 0 * e + 0 * r).astype(np.float32)
    bias = (((e + r + kind) % 7 - 3) / 1024.0 + 0 * a).astype(np.float32)
    return QMatrix(pack_codes(codes, bits), f32_to_bf16_bits(scale), f32_to_bf16_bits(bias),
                   experts, rows, columns, bits)


def prefill_value(kind, e, r, col, bits):
    """value(kind,e,r,col) of prefill_expert_checks.mm:22 (double)."""
    q = (e * 3 + r * 7 + col * 5 + kind * 11) & ((1 << bits) - 1)
    return float(q) * (col // 64 + 1) / 4096.0 + ((e + r + kind) % 7 - 3) / 1024.0


def route_pattern(pattern, count):
    """Route patterns of prefill_expert_checks.mm:27."""
    t = np.arange(count)[:, None]
    slot = np.arange(8)[None, :]
    if pattern == 0:
        ids = slot + 0 * t
    elif pattern == 1:
        ids = (t * 7 + slot * 13) % 256
    else:
        ids = (t // 5 * 11 + slot * 19) % 256
    return ids.astype(np.uint32)


def top8_cases():
    """The five top-8 logit vectors of graph_checks.mm:63-66."""
    i = np.arange(256)
    return [
        np.zeros(256, dtype=np.float32),
        (i.astype(np.float32) * np.float32(0.01)).astype(np.float32),
        np.where((i % 32 == 0) | (i == 255), 3.0, -1.0).astype(np.float32),
        ((i - 128).astype(np.float32) * np.float32(100.0)).astype(np.float32),
        (((i * 7919) % 97 - 48).astype(np.float32) * np.float32(0.07)).astype(np.float32),
    ]


def stable_top8(values):
    """graph_checks.mm:67-68: sort by value descending, ties by index ascending."""
    order = np.lexsort((np.arange(values.size), -values.astype(np.float64)))
    return order[:8]
