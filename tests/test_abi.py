"""CPU checks of the C ABI library: it loads, exports exactly what include/deepinfer_hip.h
declares, and fails loudly (no CPU fallback) where no gfx950 device is present."""
import ctypes
import os
import re

import pytest

import deepinfer_hip as dh

HEADER = dh.HEADER_PATH


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dih_[a-z0-9_]+)\s*\(", text)))


def test_library_is_built_and_loads():
    assert os.path.exists(dh.LIB_PATH), "build with __graft_entry__.build()"
    dh.load()


def test_every_declared_entry_point_is_exported():
    lib = ctypes.CDLL(dh.LIB_PATH)
    names = declared()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), n
    assert sorted(dh.EXPORTS) == names


def test_only_declared_symbols_are_exported():
    """The library hides its internals (-fvisibility=hidden): the dynamic symbol table holds
    the dih_ entry points and nothing else of ours."""
    import subprocess
    out = subprocess.run(["nm", "-D", "--defined-only", dh.LIB_PATH], capture_output=True, text=True).stdout
    ours = sorted({l.split()[-1] for l in out.splitlines() if " T " in l and "dih" in l})
    assert ours == declared()


def test_attention_default_rounding_partition_is_the_reference_one():
    """gpu_prefill.mm:393 (attentionPartitionTokens = 1024) for every call shape; an explicit
    partition is kept; invalid arguments give -1 (no device needed)."""
    for position, tokens in [(0, 1), (5000, 1), (40000, 1), (0, 2048), (30720, 2048), (100, 7)]:
        assert dh.attention_partition(position, tokens) == 1024
    assert dh.attention_partition(100, 7, 32) == 32
    assert dh.load().dih_attention_partition(0, 1, 48) == -1


def test_version_string():
    assert "gfx950" in dh.version()


@pytest.mark.skipif(os.path.exists("/dev/kfd") and os.access("/dev/kfd", os.R_OK | os.W_OK),
                    reason="a GPU node is present")
def test_context_creation_fails_loudly_without_gpu():
    with pytest.raises(dh.InvalidOperationError):
        dh.QuantizedHip()


def test_host_side_argument_validation_without_gpu():
    """Validation that happens before any device call (QuantizedMetal.cs:14, 34-36)."""
    with pytest.raises(dh.ArgumentOutOfRangeError):
        dh.QuantizedHip(residency_refresh_milliseconds=60001)


# Every entry point the reference's P/Invoke table binds (QuantNative,
# QuantizedMetal.cs:242-274); each needs a dih_ counterpart for the drop-in swap.
REFERENCE_QUANT_NATIVE = [
    "di_quant_create", "di_quant_create_configured", "di_quant_destroy", "di_quant_residency_bytes",
    "di_quant_residency_prepare", "di_quant_matrix_create", "di_quant_matrix_buffer", "di_quant_matrix_destroy",
    "di_quant_batch", "di_quant_matvec", "di_quant_experts", "di_quant_embedding",
    "di_delta_create", "di_delta_destroy", "di_delta_step",
]


def test_every_reference_native_entry_has_a_counterpart():
    names = set(declared())
    missing = [n for n in REFERENCE_QUANT_NATIVE if "dih_" + n[3:] not in names]
    assert not missing, missing
